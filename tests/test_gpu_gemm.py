"""GPU parity of the MXFP4 GEMM against the CPU oracle, through the C ABI.

Known answers restate the scaled-MFMA probe of the reference
(kernel/mfma_probe.hip:95-126) at GEMM level: they pin the operand layout,
the per-lane scale byte selection (op_sel), the nibble order and the output
(lane, acc) -> (m, n) map of the kernels.  Then every kernel configuration
runs the golden config-0 problem and ragged shapes, with and without MBS
factors and split-K, against the oracle at the north-star tolerance."""
import os

import numpy as np
import pytest

import oracle
from gpu_util import Case, assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cfg0.npz")


def n_configs():
    import mbs_amd

    return mbs_amd.ext().num_configs()


def config_name(c):
    import mbs_amd

    return mbs_amd.ext().config_name(c)


def whole_k_only(c):
    """The 32x32x64-MFMA tiles run whole-K (K % 512 == 0), single-split plans."""
    return config_name(c).endswith("_m32")


def configs_for(M, K):
    """Configurations that take M rows (decode kernels up to their M) and K."""
    return [c for c in range(n_configs())
            if not (config_name(c).startswith("skinny") and M > (16 if "m16" in config_name(c) else 32))
            and not (whole_k_only(c) and K % 512)]


def split_counts(c, counts):
    return (1,) if whole_k_only(c) else counts


def ones(R, K):
    return np.full((R, K // 2), 0x22, np.uint8)


@pytest.mark.parametrize("M,N,K", [(16, 16, 128), (32, 64, 512), (128, 256, 512)])
def test_known_answers_default_plan(dev, M, N, K):
    s = lambda R, v: np.full((R, K // 32), v, np.uint8)
    say(f"known answers M={M} N={N} K={K}")
    for sa, sb, want in [(127, 127, K), (128, 127, 2 * K), (126, 127, K / 2), (128, 128, 4 * K)]:
        c = Case(ones(M, K), s(M, sa), ones(N, K), s(N, sb))
        out = bf16_to_f32(c.run())[:M]
        assert np.all(out == want), (sa, sb, np.unique(out))
    # per-block scales 127 + block%4 -> 32 * (1+2+4+8) per 128-K step
    sb = (127 + np.arange(K // 32) % 4).astype(np.uint8)[None, :].repeat(M, 0)
    out = bf16_to_f32(Case(ones(M, K), sb, ones(N, K), s(N, 127)).run())[:M]
    assert np.all(out == 480 * (K // 128))
    # row scales 2^(m%8) and column scales 2^(n%8): decodes the output map
    sr = (127 + np.arange(M) % 8).astype(np.uint8)[:, None].repeat(K // 32, 1)
    sc = (127 + np.arange(N) % 8).astype(np.uint8)[:, None].repeat(K // 32, 1)
    out = bf16_to_f32(Case(ones(M, K), sr, ones(N, K), sc).run())[:M]
    exp = K * 2.0 ** ((np.arange(M) % 8)[:, None] + (np.arange(N) % 8)[None, :])
    np.testing.assert_array_equal(out, exp)


def test_one_hot_products(dev):
    M, N, K = 64, 64, 512
    rng = np.random.default_rng(1)
    s = np.full((64, K // 32), 127, np.uint8)
    for _ in range(12):
        m, n, k = (int(v) for v in (rng.integers(0, M), rng.integers(0, N), rng.integers(0, K)))
        say(f"one-hot m={m} n={n} k={k}")
        a = np.zeros((M, K // 2), np.uint8)
        b = np.zeros((N, K // 2), np.uint8)
        a[m, k // 2] = 0x4 << (4 * (k % 2))
        b[n, k // 2] = 0x5 << (4 * (k % 2))
        for cfg in configs_for(M, K):
            out = bf16_to_f32(Case(a, s, b, s).run(config=cfg))[:M]
            exp = np.zeros((M, N), np.float32)
            exp[m, n] = 6.0
            np.testing.assert_array_equal(out, exp, err_msg=config_name(cfg))


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("factors", [False, True])
def test_golden_cfg0_every_config(dev, gold, factors):
    af, bf = (gold["a_factor"], gold["b_factor"]) if factors else (None, None)
    c = Case(gold["x_packed"], gold["x_scales"], gold["w_packed"], gold["w_scales"], af, bf)
    ref = oracle.bf16_bits_to_f32(gold["c_mbs_bf16"] if factors else gold["c_bf16"])
    M = c.M
    say(f"golden cfg0 factors={factors} default plan")
    assert_close(bf16_to_f32(c.run())[:M], ref, "default plan")
    for cfg in configs_for(M, c.K):
        for splits in split_counts(cfg, (1, 2)):
            say(f"golden cfg0 factors={factors} config={config_name(cfg)} splits={splits}")
            got = bf16_to_f32(c.run(config=cfg, splits=splits))[:M]
            assert_close(got, ref, f"{config_name(cfg)} splits={splits}")


def rand_case(rng, M, N, K, factors=False, lo=118, hi=132):
    xp = rng.integers(0, 256, (M, K // 2), dtype=np.uint8)
    wp = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    xs = rng.integers(lo, hi, (M, K // 32), dtype=np.uint8)
    ws = rng.integers(lo, hi, (N, K // 32), dtype=np.uint8)
    af = rng.integers(0, 256, M).astype(np.uint8) if factors else None
    bf = rng.integers(0, 256, N).astype(np.uint8) if factors else None
    return Case(xp, xs, wp, ws, af, bf)


RAGGED = [
    (1, 16, 64), (5, 48, 192), (17, 80, 320), (33, 144, 448), (100, 272, 640),
    (129, 304, 1024), (250, 528, 1536), (31, 1040, 2048),
]


@pytest.mark.parametrize("M,N,K", RAGGED)
def test_ragged_every_config(dev, M, N, K):
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    for factors in (False, True):
        c = rand_case(rng, M, N, K, factors)
        ref = oracle.bf16_bits_to_f32(c.reference())
        say(f"ragged M={M} N={N} K={K} factors={factors} default")
        assert_close(bf16_to_f32(c.run())[:M], ref, "default plan")
        for cfg in configs_for(M, K):
            for splits in split_counts(cfg, (1, 3)):
                say(f"ragged M={M} N={N} K={K} factors={factors} {config_name(cfg)} s={splits}")
                got = bf16_to_f32(c.run(config=cfg, splits=splits))[:M]
                assert_close(got, ref, f"{config_name(cfg)} splits={splits}")


def test_padding_rows_untouched_and_deterministic(dev):
    import torch

    rng = np.random.default_rng(2)
    M, N, K = 45, 96, 512
    c = rand_case(rng, M, N, K, factors=True)
    for cfg in [None] + configs_for(M, K):
        for splits in (1,) if cfg is None else split_counts(cfg, (1, 2)):
            say(f"padding rows config={cfg} splits={splits}")
            out = torch.full((c.Mpad, N), 7.0, dtype=torch.bfloat16, device=c.A.device)
            out = c.run(config=cfg, splits=splits, out=out)
            o = bf16_to_f32(out)
            assert np.all(o[M:] == 7.0), cfg
            again = bf16_to_f32(c.run(config=cfg, splits=splits))
            np.testing.assert_array_equal(o[:M], again[:M])
            if cfg is None:
                break


def test_edge_scales(dev):
    """All-zero blocks (E8M0 0x00), saturated blocks, tiny and huge scales,
    and a NaN scale (0xFF) confined to its own rows."""
    rng = np.random.default_rng(3)
    M, N, K = 64, 128, 1024
    xp = rng.integers(0, 256, (M, K // 2), dtype=np.uint8)
    wp = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    xs = rng.integers(118, 132, (M, K // 32), dtype=np.uint8)
    ws = rng.integers(118, 132, (N, K // 32), dtype=np.uint8)
    xp[3, :] = 0
    xs[3, :] = 0                      # all-zero row, scale 2^-127
    xs[5, :4] = 0                     # tiny scales with live data
    xp[7, :] = 0x77                   # +6 everywhere (saturated code)
    xs[7, :] = 200                    # large but finite products
    ws[9, :] = 60
    xs[11, 2] = 255                   # NaN scale: row 11 becomes NaN
    c = Case(xp, xs, wp, ws)
    ref = oracle.bf16_bits_to_f32(c.reference())
    assert np.all(np.isnan(ref[11]))
    for cfg in [None] + configs_for(M, K):
        say(f"edge scales config={cfg}")
        got = bf16_to_f32(c.run(config=cfg) if cfg is not None else c.run())[:M]
        assert_close(got, ref, f"config {cfg}")


def test_pybind_module_matches_c_abi(dev, gold):
    import torch

    import mbs_amd

    m = mbs_amd.ext()
    c = Case(gold["x_packed"], gold["x_scales"], gold["w_packed"], gold["w_scales"],
             gold["a_factor"], gold["b_factor"])
    say("pybind gemm_a4w4 vs C ABI")
    via_c = bf16_to_f32(c.run())[: c.M]
    # the reference's 6-argument call with [M,1] / [N,1] factors
    out6 = m.gemm_a4w4(c.A, c.B, c.As, c.Bs, c.Af.view(-1, 1), c.Bf.view(-1, 1))
    assert out6.shape == (c.M, c.N) and out6.dtype == torch.bfloat16
    np.testing.assert_array_equal(bf16_to_f32(out6), via_c)
    # bench_one.py's 4-argument call (factors omitted)
    out4 = m.gemm_a4w4(c.A, c.B, c.As, c.Bs)
    plain = Case(gold["x_packed"], gold["x_scales"], gold["w_packed"], gold["w_scales"])
    np.testing.assert_array_equal(bf16_to_f32(out4), bf16_to_f32(plain.run())[: c.M])
    assert_close(bf16_to_f32(out4), oracle.bf16_bits_to_f32(gold["c_bf16"]), "4-arg call")
    # 1-byte dtype views are accepted like the reference (A.view(kByte))
    out_i8 = m.gemm_a4w4(c.A.view(torch.int8), c.B.view(torch.int8), c.As, c.Bs)
    np.testing.assert_array_equal(bf16_to_f32(out_i8), bf16_to_f32(out4))
    with pytest.raises(RuntimeError, match="together"):
        m.gemm_a4w4(c.A, c.B, c.As, c.Bs, c.Af, None)
    with pytest.raises(RuntimeError, match="A_scale must hold"):
        m.gemm_a4w4(c.A, c.B, c.As[:10], c.Bs)


def test_empty_batch(dev, gold):
    """M == 0 (an expert without tokens): the module returns an empty [0, N]
    bf16 tensor and launches nothing, with and without factors, for the default
    plan and a forced configuration; the next call still computes normally."""
    import torch

    import mbs_amd

    m = mbs_amd.ext()
    c = Case(gold["x_packed"], gold["x_scales"], gold["w_packed"], gold["w_scales"])
    say("empty batch M=0")
    A0 = c.A[:0]
    As0 = torch.empty(0, dtype=torch.uint8, device=c.A.device)
    Af0 = torch.empty(0, dtype=torch.uint8, device=c.A.device)
    Bf = torch.zeros(c.N, dtype=torch.uint8, device=c.A.device)
    for out in (m.gemm_a4w4(A0, c.B, As0, c.Bs), m.gemm_a4w4(A0, c.B, As0, c.Bs, Af0, Bf),
                m.gemm_a4w4_config(0, 1, A0, c.B, As0, c.Bs),
                m.gemm_a4w4(A0, c.B, As0, c.Bs, alpha=2.0)):
        assert out.shape == (0, c.N) and out.dtype == torch.bfloat16 and out.is_cuda
    torch.cuda.synchronize()
    assert_close(bf16_to_f32(m.gemm_a4w4(c.A, c.B, c.As, c.Bs)),
                 oracle.bf16_bits_to_f32(gold["c_bf16"]), "call after the empty batch")


def test_output_past_2gib(dev):
    """An output larger than 2^31 bytes of fp32 partials (M*N*4 > 2^31; ragged M):
    the default plan and a forced split-K plan, whose workspace is 4.3 GB, both
    address tiles beyond 2 GiB through 64-bit tile bases.  Rows at the 2^31-byte
    boundaries and the last rows are checked against the oracle."""
    import torch

    import mbs_amd

    M, N, K = 33000, 16384, 512
    rng = np.random.default_rng(33)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
    w = torch.from_numpy((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    c = Case.from_bf16(x.to(torch.bfloat16), w.to(torch.bfloat16))
    rows = np.unique(np.concatenate([[0, 1, 16383, 16384, 32767, 32768, M - 2, M - 1],
                                     rng.integers(0, M, 12)]))
    ref = oracle.bf16_bits_to_f32(c.reference(rows))
    names = [mbs_amd.ext().config_name(i) for i in range(mbs_amd.ext().num_configs())]
    for cfg, splits in [(None, 0), (names.index("bdirect_256x256_w2x2"), 2)]:
        say(f"output past 2 GiB M={M} N={N} K={K} config={cfg} splits={splits}")
        out = c.run(config=cfg, splits=splits)
        got = bf16_to_f32(out[torch.from_numpy(rows).to(out.device)])
        assert_close(got, ref, f"config {cfg} splits {splits}")
        del out
        torch.cuda.empty_cache()


def test_misaligned_views(dev, gold):
    """Operands that are views starting off a 16-byte boundary (factors off a
    4-byte one): the module copies them into aligned storage and gives the
    aligned call's bytes; the C ABI refuses them (MBS_ERR_ARGUMENT)."""
    import torch

    import mbs_amd
    from gpu_util import clib, ptr, stream_ptr

    c = Case(gold["x_packed"], gold["x_scales"], gold["w_packed"], gold["w_scales"],
             gold["a_factor"], gold["b_factor"])
    say("misaligned operand views")
    want = mbs_amd.gemm_a4w4(c.A, c.B, c.As, c.Bs, c.Af, c.Bf)

    def shifted(t, off):
        buf = torch.empty(t.numel() + off, dtype=torch.uint8, device=t.device)
        v = buf[off:].view(t.shape)
        v.copy_(t)
        return v

    for off in (1, 4, 8):
        views = [shifted(t, off) for t in (c.A, c.B, c.As, c.Bs, c.Af, c.Bf)]
        assert views[0].data_ptr() % 16 != 0
        got = mbs_amd.gemm_a4w4(*views)
        torch.cuda.synchronize()
        assert torch.equal(got, want), off
    L = clib()
    out = torch.empty(c.Mpad, c.N, dtype=torch.bfloat16, device=c.A.device)
    A8 = shifted(c.A, 8)
    st = L.mbs_gemm_a4w4_launch(ptr(A8), ptr(c.B), ptr(c.As), ptr(c.Bs), None, None, ptr(out), c.M,
                                c.N, c.K, c.Mpad, c.snp, None, 0, stream_ptr())
    assert st == 1 and b"aligned" in L.mbs_last_error()
