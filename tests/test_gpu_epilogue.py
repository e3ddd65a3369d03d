"""GPU parity of the affine epilogue (out = bf16(C * alpha * f(a) * f(b) +
bias[n])) on every kernel configuration, with and without split-K and MBS
factors: alpha 1 without bias gives exactly the plain launch's bytes, a
power-of-two alpha scales them exactly, and alpha with a bias matches the
oracle's epilogue_affine_bf16 within the north-star tolerance."""
import numpy as np
import pytest

import oracle
from gpu_util import Case, assert_close, bf16_to_f32, say
from test_gpu_gemm import config_name, configs_for, split_counts

pytestmark = pytest.mark.gpu


def operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    xp, xs = oracle.quantize_mxfp4(x)
    wp, ws = oracle.quantize_mxfp4(w)
    af = rng.integers(0, 256, M, dtype=np.uint8)
    bf = rng.integers(0, 256, N, dtype=np.uint8)
    bias = oracle.f32_to_bf16_bits((rng.standard_normal(N) * 2).astype(np.float32))
    return xp, xs, wp, ws, af, bf, bias


@pytest.mark.parametrize("M,N,K", [(128, 256, 1024), (16, 512, 512)])
@pytest.mark.parametrize("factors", [False, True])
def test_affine_epilogue_every_config(dev, M, N, K, factors):
    import torch

    import mbs_amd

    xp, xs, wp, ws, af, bf, bias = operands(M, N, K, M + N + K + int(factors))
    case = Case(xp, xs, wp, ws, af if factors else None, bf if factors else None, dev=dev)
    bias_t = torch.from_numpy(bias.view(np.int16)).to(dev).view(torch.bfloat16)
    c32 = oracle.dequant_mxfp4(xp, xs).astype(np.float64) @ oracle.dequant_mxfp4(wp, ws).astype(np.float64).T
    ref = oracle.bf16_bits_to_f32(oracle.epilogue_affine_bf16(
        c32.astype(np.float32), af if factors else None, bf if factors else None, 0.75, bias))
    m = mbs_amd.ext()
    for cfg in configs_for(M, K):
        for splits in split_counts(cfg, (1, 2)):
            say(f"affine M={M} N={N} K={K} factors={factors} config={config_name(cfg)} splits={splits}")
            args = (case.A, case.B, case.As, case.Bs, case.Af, case.Bf)
            plain = m.gemm_a4w4_config(cfg, splits, *args)
            same = m.gemm_a4w4_config(cfg, splits, *args, 1.0, None)
            assert torch.equal(plain, same)
            x2 = m.gemm_a4w4_config(cfg, splits, *args, 2.0, None)
            np.testing.assert_array_equal(bf16_to_f32(x2), bf16_to_f32(plain) * 2)
            got = m.gemm_a4w4_config(cfg, splits, *args, 0.75, bias_t)
            assert_close(bf16_to_f32(got), ref, f"{config_name(cfg)} splits={splits}")


def test_affine_default_plan_large(dev):
    import torch

    import mbs_amd

    M, N, K = 1024, 2048, 2048
    say(f"affine default plan M={M} N={N} K={K}")
    xp, xs, wp, ws, af, bf, bias = operands(M, N, K, 7)
    case = Case(xp, xs, wp, ws, af, bf, dev=dev)
    bias_t = torch.from_numpy(bias.view(np.int16)).to(dev).view(torch.bfloat16)
    got = mbs_amd.gemm_a4w4(case.A, case.B, case.As, case.Bs, case.Af, case.Bf, alpha=-1.5, bias=bias_t)
    rows = np.arange(0, M, 37)
    c32 = (oracle.dequant_mxfp4(xp[rows], xs[rows]).astype(np.float64)
           @ oracle.dequant_mxfp4(wp, ws).astype(np.float64).T).astype(np.float32)
    ref = oracle.bf16_bits_to_f32(oracle.epilogue_affine_bf16(c32, af[rows], bf, -1.5, bias))
    assert_close(bf16_to_f32(got)[rows], ref, "default plan, alpha -1.5, bias")
