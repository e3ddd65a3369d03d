"""GPU parity of the grouped (mixture-of-experts) GEMM: one launch over E
experts against E separate dense launches on the same bytes (bit for bit:
the per-element accumulation order does not depend on the tile), and against
the oracle's run_torch per expert.  Covers every
grouped configuration, empty experts, many small experts, MBS factors, a
64-wide K tail, offsets given on the device, alpha with a bias per expert,
and the host-side checks."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu


def make_problem(rng, rows, N, K, factors=False):
    """Expert row counts `rows` (multiples of 32) -> host bytes of A (all
    experts' rows stacked), the E weight matrices and their scales."""
    M = int(sum(rows))
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((len(rows), N, K)) * 0.05).astype(np.float32)
    xp, xs = oracle.quantize_mxfp4(x)
    wq = [oracle.quantize_mxfp4(w[e]) for e in range(len(rows))]
    af = rng.integers(0, 256, M, dtype=np.uint8) if factors else None
    bf = rng.integers(0, 256, (len(rows), N), dtype=np.uint8) if factors else None
    offs = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    return M, xp, xs, wq, af, bf, offs


def device_operands(dev, M, N, K, xp, xs, wq, af, bf):
    import torch

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    A = t(xp)
    As = t(oracle.shuffle_scales(xs, K, pad=127))
    B = t(np.stack([oracle.shuffle_b(wp) for wp, _ in wq]))
    Bs = t(np.stack([oracle.shuffle_scales(ws, K, pad=127).reshape(-1) for _, ws in wq]))
    Af = None if af is None else t(af)
    Bf = None if bf is None else t(bf.reshape(-1))
    return A, As, B, Bs, Af, Bf


def dense_expert(dev, e, offs, N, K, xp, xs, wq, af, bf):
    """The dense launch of expert e alone (its rows of A, its weights)."""
    import torch

    import mbs_amd

    r0, r1 = offs[e], offs[e + 1]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    A = t(xp[r0:r1])
    As = t(oracle.shuffle_scales(xs[r0:r1], K, pad=127))
    B = t(oracle.shuffle_b(wq[e][0]))
    Bs = t(oracle.shuffle_scales(wq[e][1], K, pad=127))
    Af = None if af is None else t(af[r0:r1])
    Bf = None if bf is None else t(bf[e])
    return mbs_amd.gemm_a4w4(A, B, As, Bs, Af, Bf)


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("rows,N,K", [([64, 0, 96, 32], 512, 1024), ([256, 128], 256, 2048)])
def test_grouped_matches_dense_per_expert(dev, config, rows, N, K):
    import torch

    import mbs_amd

    name = mbs_amd.ext().grouped_config_name(config)
    say(f"grouped config={name} rows={rows} N={N} K={K}")
    rng = np.random.default_rng(len(rows) * 100 + N + K + config)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, rows, N, K)
    A, As, B, Bs, Af, Bf = device_operands(dev, M, N, K, xp, xs, wq, af, bf)
    got = mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.from_numpy(offs), config=config)
    torch.cuda.synchronize()
    for e in range(len(rows)):
        if rows[e] == 0:
            continue
        want = dense_expert(dev, e, offs, N, K, xp, xs, wq, af, bf)
        assert torch.equal(got[offs[e]:offs[e + 1]], want), (name, e)
        ref = oracle.bf16_bits_to_f32(oracle.run_torch(xp[offs[e]:offs[e + 1]], wq[e][0],
                                                       xs[offs[e]:offs[e + 1]], wq[e][1]))
        assert_close(bf16_to_f32(got[offs[e]:offs[e + 1]]), ref, f"{name} expert {e}")


@pytest.mark.parametrize("rows,N,K,factors", [
    ([32] * 24, 256, 512, False),              # many small experts (one partial tile each)
    ([96, 160, 0, 32, 224], 768, 1088, True),  # factors, K % 128 == 64 (K tail)
    ([0, 0, 288], 1024, 4096, True),           # leading empty experts
    ([256] * 8, 7168, 2048, False),            # configs[3] expert shapes: the tuned-table
    ([256] * 8, 2112, 7168, False),            # plans (256x256 and 128x256)
])
def test_grouped_default_plan(dev, rows, N, K, factors):
    import torch

    import mbs_amd

    say(f"grouped default rows={rows[:6]}.. E={len(rows)} N={N} K={K} factors={factors}")
    rng = np.random.default_rng(sum(rows) + N + K)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, rows, N, K, factors)
    A, As, B, Bs, Af, Bf = device_operands(dev, M, N, K, xp, xs, wq, af, bf)
    goff = torch.from_numpy(offs).to(dev)       # offsets already on the device
    got = mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, goff, Af, Bf)
    torch.cuda.synchronize()
    for e in range(len(rows)):
        if rows[e] == 0:
            continue
        r0, r1 = offs[e], offs[e + 1]
        want = dense_expert(dev, e, offs, N, K, xp, xs, wq, af, bf)
        assert torch.equal(got[r0:r1], want), e
        ref = oracle.bf16_bits_to_f32(oracle.run_torch(
            xp[r0:r1], wq[e][0], xs[r0:r1], wq[e][1],
            None if af is None else af[r0:r1], None if bf is None else bf[e]))
        assert_close(bf16_to_f32(got[r0:r1]), ref, f"expert {e}")


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4, 5])
def test_grouped_alpha_bias(dev, config):
    """Affine epilogue per expert: bf16(C * alpha * f(a) * f(b) + bias[e]) --
    the dense launch of each expert with its own bias row, bit for bit, and
    the oracle's epilogue within tolerance."""
    import torch

    import mbs_amd

    rows, N, K = [64, 0, 96, 32], 512, 1024
    name = mbs_amd.ext().grouped_config_name(config)
    say(f"grouped alpha/bias config={name} rows={rows} N={N} K={K}")
    rng = np.random.default_rng(77 + config)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, rows, N, K, factors=True)
    A, As, B, Bs, Af, Bf = device_operands(dev, M, N, K, xp, xs, wq, af, bf)
    bias = oracle.f32_to_bf16_bits((rng.standard_normal((len(rows), N)) * 2).astype(np.float32))
    bias_t = torch.from_numpy(bias.view(np.int16)).to(dev).view(torch.bfloat16)
    got = mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.from_numpy(offs), Af, Bf, config=config,
                                    alpha=-0.75, bias=bias_t)
    torch.cuda.synchronize()
    for e in range(len(rows)):
        if rows[e] == 0:
            continue
        r0, r1 = offs[e], offs[e + 1]
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        want = mbs_amd.gemm_a4w4(t(xp[r0:r1]), t(oracle.shuffle_b(wq[e][0])),
                                 t(oracle.shuffle_scales(xs[r0:r1], K, pad=127)),
                                 t(oracle.shuffle_scales(wq[e][1], K, pad=127)), t(af[r0:r1]), t(bf[e]),
                                 alpha=-0.75, bias=bias_t[e])
        assert torch.equal(got[r0:r1], want), (name, e)
        c32 = (oracle.dequant_mxfp4(xp[r0:r1], xs[r0:r1]).astype(np.float64)
               @ oracle.dequant_mxfp4(wq[e][0], wq[e][1]).astype(np.float64).T).astype(np.float32)
        ref = oracle.bf16_bits_to_f32(oracle.epilogue_affine_bf16(c32, af[r0:r1], bf[e], -0.75, bias[e]))
        assert_close(bf16_to_f32(got[r0:r1]), ref, f"{name} expert {e}")
    with pytest.raises(RuntimeError, match="bias"):
        mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.from_numpy(offs), bias=bias_t[0])


def test_grouped_rejects_bad_offsets(dev):
    import torch

    import mbs_amd

    say("grouped offset checks")
    rng = np.random.default_rng(1)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, [64, 64], 256, 512)
    A, As, B, Bs, _, _ = device_operands(dev, M, 256, 512, xp, xs, wq, None, None)
    for bad in ([0, 48, 128], [0, 96, 64], [32, 64, 128], [0, 64, 160]):
        with pytest.raises(RuntimeError, match="group_offsets"):
            mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.tensor(bad, dtype=torch.int32))


def _grouped_c_call(dev, A, B, As, Bs, goff, E, M, N, K, out, config=-1):
    """mbs_gemm_a4w4_grouped_launch through the C ABI into a caller-filled output."""
    import ctypes

    import mbs_amd
    from gpu_util import ptr, stream_ptr

    L = mbs_amd.clib()
    P, I = ctypes.c_void_p, ctypes.c_int
    L.mbs_gemm_a4w4_grouped_launch.argtypes = [P, P, P, P, P, P, P, I, P, I, I, I, I, I, I, P]
    L.mbs_gemm_a4w4_grouped_launch.restype = I
    snp = oracle.scale_pad(K)
    return L.mbs_gemm_a4w4_grouped_launch(ptr(A), ptr(B), ptr(As), ptr(Bs), None, None, ptr(goff),
                                          E, ptr(out), M, N, K, oracle.round_up(M, 32), snp, config,
                                          stream_ptr())


@pytest.mark.parametrize("config", [0, 1, 2, 3, 4, 5])
def test_grouped_all_experts_empty_writes_nothing(dev, config):
    """Every expert empty (offsets all 0) with M > 0: the kernel has no work
    units; every workgroup leaves before its first load and the output keeps
    the caller's bytes."""
    import torch

    say(f"grouped all-empty config={config}")
    rng = np.random.default_rng(5)
    M, N, K = 64, 256, 512
    _, xp, xs, wq, _, _, _ = make_problem(rng, [64, 0], N, K)
    A, As, B, Bs, _, _ = device_operands(dev, M, N, K, xp, xs, wq, None, None)
    out = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=dev)
    goff = torch.zeros(3, dtype=torch.int32, device=dev)
    assert _grouped_c_call(dev, A, B, As, Bs, goff, 2, M, N, K, out, config) == 0
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_grouped_unaligned_expert_is_skipped_and_reported(dev):
    """An expert whose first row is not a multiple of 32 gets no tiles (its
    rows keep the caller's bytes); the aligned experts are still exact, and
    check_groups / validate=True report the offsets."""
    import torch

    import mbs_amd

    say("grouped unaligned expert start")
    rng = np.random.default_rng(9)
    N, K = 256, 512
    M, xp, xs, wq, _, _, _ = make_problem(rng, [64, 32, 64], N, K)
    offs = np.array([0, 64, 80, 160], np.int32)    # expert 2 starts at row 80
    A, As, B, Bs, _, _ = device_operands(dev, M, N, K, xp, xs, wq, None, None)
    goff = torch.from_numpy(offs).to(dev)
    assert mbs_amd.check_groups(goff, M) == (1, 0)
    assert mbs_amd.check_groups(torch.tensor([0, 64, 32, 200], dtype=torch.int32, device=dev), M) == (0, 2)
    with pytest.raises(RuntimeError, match="not a multiple of 32"):
        mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, goff, validate=True)
    out = torch.full((M, N), 3.0, dtype=torch.bfloat16, device=dev)
    assert _grouped_c_call(dev, A, B, As, Bs, goff, 3, M, N, K, out) == 0
    torch.cuda.synchronize()
    assert bool((out[80:160] == 3.0).all())
    for e, (r0, r1) in enumerate([(0, 64), (64, 80)]):
        ref = oracle.bf16_bits_to_f32(oracle.run_torch(xp[r0:r1], wq[e][0], xs[r0:r1], wq[e][1]))
        assert_close(bf16_to_f32(out[r0:r1]), ref, f"expert {e}")
    assert mbs_amd.check_groups(torch.from_numpy(np.array([0, 64, 96, 160], np.int32)).to(dev), M) == (0, 0)


def test_grouped_many_experts(dev):
    """256 experts (most empty, the prefix sums span every thread of the
    workgroup scan): bit-identical to the dense launch per non-empty expert."""
    import torch

    import mbs_amd

    E, N, K = 256, 128, 512
    rows = [0] * E
    for e in (0, 1, 63, 64, 130, 200, 254, 255):
        rows[e] = 32 * (1 + e % 3)
    say(f"grouped E={E} N={N} K={K}")
    rng = np.random.default_rng(11)
    M, xp, xs, wq, af, bf, offs = make_problem(rng, rows, N, K)
    A, As, B, Bs, _, _ = device_operands(dev, M, N, K, xp, xs, wq, None, None)
    for config in range(mbs_amd.ext().grouped_num_configs()):
        got = mbs_amd.gemm_a4w4_grouped(A, B, As, Bs, torch.from_numpy(offs).to(dev), config=config,
                                        validate=True)
        torch.cuda.synchronize()
        for e in range(E):
            if rows[e]:
                want = dense_expert(dev, e, offs, N, K, xp, xs, wq, None, None)
                assert torch.equal(got[offs[e]:offs[e + 1]], want), (config, e)
