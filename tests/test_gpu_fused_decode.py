"""GPU parity of the decode GEMM that takes a bf16 activation
(gemm_a4w4_bf16a / mbs_gemm_a4w4_bf16a_launch): the decode kernel quantizes
each A block in registers, so its output must equal, bit for bit, the
quantizer (quantize_mxfp4) followed by the packed GEMM run with the same
configuration and split count; and it must meet the north-star tolerance
against the CPU oracle on the same bytes."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu


def fused(x, B, Bs, alpha=1.0, bias=None):
    """mbs_gemm_a4w4_bf16a_launch through the C ABI (the kernel path for every M <= 32)."""
    import ctypes

    import torch

    import mbs_amd
    from gpu_util import ptr, stream_ptr

    L = mbs_amd.clib()
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.mbs_gemm_a4w4_bf16a_launch.argtypes = [P, P, P, P, I, I, I, I, I, ctypes.c_float, P, P, S, P]
    L.mbs_gemm_a4w4_bf16a_launch.restype = I
    L.mbs_gemm_a4w4_bf16a_workspace_bytes.argtypes = [I, I, I]
    L.mbs_gemm_a4w4_bf16a_workspace_bytes.restype = S
    M, K = x.shape
    N = B.shape[0]
    Mpad = oracle.round_up(M, 32)
    out = torch.empty(Mpad, N, dtype=torch.bfloat16, device=x.device)
    ws = L.mbs_gemm_a4w4_bf16a_workspace_bytes(M, N, K)
    wst = torch.empty(max(ws, 1), dtype=torch.uint8, device=x.device)
    st = L.mbs_gemm_a4w4_bf16a_launch(ptr(x), ptr(B), ptr(Bs), ptr(out), M, N, K, Mpad,
                                      oracle.scale_pad(K), alpha, ptr(bias), ptr(wst), ws,
                                      stream_ptr())
    assert st == 0, L.mbs_last_error()
    return out[:M]


def plan_of(m, M, N, K):
    """(config index, split count) of the bf16-A plan."""
    name, rest = m.bf16a_plan_name(M, N, K).split(" ", 1)
    splits = int(rest.split("splits=")[1].split()[0])
    names = [m.config_name(i) for i in range(m.num_configs())]
    return names.index(name), splits, name


def operands(M, N, K, seed, special=False):
    import torch

    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32) * np.exp(rng.uniform(-2, 2, (M, 1)))
    if special and M >= 4:
        x[0, :32] = 0.0                     # zero block -> scale 0
        x[1, 40] = np.inf                   # inf -> block scale 254, inf/NaN outputs
        x[2, :32] = -1e-40                  # negative subnormals -> -0 codes
        x[3, 7] = 3e38                      # huge next to normal values
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    wb = torch.from_numpy(w).to(torch.bfloat16)
    return xb, wb


@pytest.mark.parametrize("M,N,K", [(1, 8192, 8192), (4, 8192, 8192), (16, 8192, 8192),
                                   (17, 8192, 8192), (32, 8192, 8192), (1, 1280, 512),
                                   (16, 2112, 7168), (5, 48, 192), (32, 2048, 8192),
                                   (3, 4096, 320)])
def test_bf16a_matches_quantize_then_gemm(dev, M, N, K):
    import mbs_amd

    m = mbs_amd.ext()
    xb, wb = operands(M, N, K, seed=M * 7 + N + K, special=(M >= 4 and K >= 64))
    x = xb.to(dev)
    Wq, Bs = mbs_amd.quantize_mxfp4(wb.to(dev), shuffle=True)
    B = mbs_amd.shuffle_weight(Wq)
    cfg, splits, name = plan_of(m, M, N, K)
    say(f"bf16a M={M} N={N} K={K} plan={name} splits={splits}")
    got = fused(x, B, Bs)
    A, As = mbs_amd.quantize_mxfp4(x, shuffle=True)
    two_step = m.gemm_a4w4_config(cfg, splits, A, B, As, Bs)
    assert got.shape == (M, N)
    f, t = bf16_to_f32(got), bf16_to_f32(two_step)
    assert np.array_equal(np.isnan(f), np.isnan(t))
    np.testing.assert_array_equal(f[~np.isnan(f)].view(np.uint32), t[~np.isnan(t)].view(np.uint32))
    # and the oracle, on the same bytes; rows 1 and 3 of the special case
    # overflow in fp32 accumulation (inf/NaN depend on the summation order)
    xp, xs = oracle.quantize_mxfp4(xb.float().numpy())
    wp, ws = oracle.quantize_mxfp4(wb.float().numpy())
    ref = oracle.bf16_bits_to_f32(oracle.run_torch(xp, wp, xs, ws))
    rows = [r for r in range(M) if not (M >= 4 and K >= 64 and r in (1, 3))]
    assert_close(f[rows], ref[rows], f"bf16a {M}x{N}x{K}")


def test_bf16a_default_plan_for_decode_shapes(dev):
    """For the decode shapes of configs[2] the bf16-A plan is the default plan,
    so the one-launch path equals quantize + gemm_a4w4 bit for bit."""
    import mbs_amd

    m = mbs_amd.ext()
    for M in (1, 4, 16, 32):
        assert m.bf16a_plan_name(M, 8192, 8192) == m.plan_name(M, 8192, 8192)
    xb, wb = operands(16, 8192, 8192, seed=3)
    x = xb.to(dev)
    Wq, Bs = mbs_amd.quantize_mxfp4(wb.to(dev), shuffle=True)
    B = mbs_amd.shuffle_weight(Wq)
    A, As = mbs_amd.quantize_mxfp4(x, shuffle=True)
    want = bf16_to_f32(mbs_amd.gemm_a4w4(A, B, As, Bs))
    say("bf16a kernel vs default two-step M=16")
    np.testing.assert_array_equal(bf16_to_f32(fused(x, B, Bs)), want)
    # the module routes M <= 8 through the kernel and larger M through the two steps
    say("module routing M=16 and M=4")
    np.testing.assert_array_equal(bf16_to_f32(mbs_amd.gemm_a4w4_bf16a(x, B, Bs)), want)
    A4, As4 = mbs_amd.quantize_mxfp4(x[:4], shuffle=True)
    np.testing.assert_array_equal(bf16_to_f32(mbs_amd.gemm_a4w4_bf16a(x[:4], B, Bs)),
                                  bf16_to_f32(mbs_amd.gemm_a4w4(A4, B, As4, Bs)))


def test_bf16a_alpha_bias_empty_and_large_m(dev):
    import torch

    import mbs_amd

    m = mbs_amd.ext()
    N, K = 2048, 1024
    xb, wb = operands(40, N, K, seed=11)
    x = xb.to(dev)
    Wq, Bs = mbs_amd.quantize_mxfp4(wb.to(dev), shuffle=True)
    B = mbs_amd.shuffle_weight(Wq)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(5)) * 0.1).to(torch.bfloat16).to(dev)
    say("bf16a alpha/bias M=8")
    cfg, splits, _ = plan_of(m, 8, N, K)
    A, As = mbs_amd.quantize_mxfp4(x[:8], shuffle=True)
    want = bf16_to_f32(m.gemm_a4w4_config(cfg, splits, A, B, As, Bs, alpha=0.75, bias=bias))
    np.testing.assert_array_equal(bf16_to_f32(fused(x[:8].contiguous(), B, Bs, 0.75, bias)), want)
    np.testing.assert_array_equal(
        bf16_to_f32(mbs_amd.gemm_a4w4_bf16a(x[:8], B, Bs, alpha=0.75, bias=bias)), want)
    say("bf16a M=0 and M=40 (quantize-then-GEMM form)")
    empty = mbs_amd.gemm_a4w4_bf16a(x[:0], B, Bs)
    assert empty.shape == (0, N)
    A40, As40 = mbs_amd.quantize_mxfp4(x, shuffle=True)
    np.testing.assert_array_equal(bf16_to_f32(mbs_amd.gemm_a4w4_bf16a(x, B, Bs)),
                                  bf16_to_f32(mbs_amd.gemm_a4w4(A40, B, As40, Bs)))
    with pytest.raises(RuntimeError, match="K must be a multiple of 64"):
        mbs_amd.gemm_a4w4_bf16a(x[:4, :96].contiguous(), B[:, :48].contiguous(), Bs)
