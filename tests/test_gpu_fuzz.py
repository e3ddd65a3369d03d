"""Seeded random-shape parity sweep of the default plan (whatever kernel,
tile and split count the planner picks) through the Python operator:
M from decode sizes to a few thousand rows, N any multiple of 16, K any
multiple of 64 (64-wide K tails included), with and without MBS factors,
alpha and a column bias; then the same with a random forced configuration
and split count per case.  Each case is checked against the oracle's
dequantize -> fp64 matmul -> affine bf16 epilogue within the north-star
tolerance.  Operand sizes are capped (M*N*K <= 1e9) so the oracle stays
quick."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu


def cases(n=24, seed=2026, max_macs=1e9):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        band = rng.integers(0, 3)
        M = int(rng.integers(1, 33) if band == 0 else rng.integers(33, 700) if band == 1
                else rng.integers(700, 4000))
        K = 64 * int(rng.integers(1, 160))
        n_max = max(1, min(400, int(max_macs // (M * K * 16))))
        N = 16 * int(rng.integers(1, n_max + 1))
        out.append((len(out), M, N, K, bool(rng.random() < 0.5), bool(rng.random() < 0.5)))
    return out


def operands(dev, idx, M, N, K, factors, affine):
    import torch

    rng = np.random.default_rng(1000 + idx)
    x = (rng.standard_normal((M, K)) * np.exp(rng.uniform(-2, 2, (M, 1)))).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x[rng.random(M) < 0.05] = 0.0                      # some all-zero rows
    xp, xs = oracle.quantize_mxfp4(x)
    wp, ws = oracle.quantize_mxfp4(w)
    af = rng.integers(0, 256, M, dtype=np.uint8) if factors else None
    bf = rng.integers(0, 256, N, dtype=np.uint8) if factors else None
    alpha = float(rng.choice([0.5, -1.25, 3.0])) if affine else 1.0
    bias = (oracle.f32_to_bf16_bits((rng.standard_normal(N) * 4).astype(np.float32))
            if affine else None)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    A, B = t(xp), t(oracle.shuffle_b(wp))
    As, Bs = t(oracle.shuffle_scales(xs, K, pad=127)), t(oracle.shuffle_scales(ws, K, pad=127))
    bias_t = None if bias is None else t(bias.view(np.int16)).view(torch.bfloat16)
    c32 = (oracle.dequant_mxfp4(xp, xs).astype(np.float64)
           @ oracle.dequant_mxfp4(wp, ws).astype(np.float64).T).astype(np.float32)
    ref = oracle.bf16_bits_to_f32(oracle.epilogue_affine_bf16(c32, af, bf, alpha, bias))
    return (A, B, As, Bs, t(af), t(bf)), alpha, bias_t, ref


@pytest.mark.parametrize("idx,M,N,K,factors,affine", cases())
def test_random_shape_default_plan(dev, idx, M, N, K, factors, affine):
    import torch

    import mbs_amd

    args, alpha, bias_t, ref = operands(dev, idx, M, N, K, factors, affine)
    say(f"fuzz {idx}: M={M} N={N} K={K} factors={factors} alpha={alpha} bias={bias_t is not None} "
        f"plan={mbs_amd.ext().plan_name(M, N, K)}")
    got = mbs_amd.gemm_a4w4(*args, alpha=alpha, bias=bias_t)
    torch.cuda.synchronize()
    assert tuple(got.shape) == (M, N)
    assert_close(bf16_to_f32(got), ref, f"case {idx}")


@pytest.mark.parametrize("idx,M,N,K,factors,affine", cases(seed=7, max_macs=4e8))
def test_random_shape_forced_config(dev, idx, M, N, K, factors, affine):
    """The same sweep with a random kernel configuration and split count
    per case (decode kernels only where M fits them)."""
    import torch

    import mbs_amd

    m = mbs_amd.ext()
    rng = np.random.default_rng(5000 + idx)
    names = [m.config_name(c) for c in range(m.num_configs())]
    fit = [c for c, nm in enumerate(names)
           if (not nm.startswith("skinny") or M <= (16 if "m16" in nm else 32))
           and (not nm.endswith("_m32") or K % 512 == 0)]
    cfg = int(rng.choice(fit))
    splits = 1 if names[cfg].endswith("_m32") else int(rng.integers(1, 4))
    args, alpha, bias_t, ref = operands(dev, 100 + idx, M, N, K, factors, affine)
    say(f"fuzz forced {idx}: M={M} N={N} K={K} factors={factors} alpha={alpha} "
        f"bias={bias_t is not None} config={names[cfg]} splits={splits}")
    got = m.gemm_a4w4_config(cfg, splits, *args, alpha, bias_t)
    torch.cuda.synchronize()
    assert_close(bf16_to_f32(got)[:M], ref, f"case {idx} {names[cfg]} splits={splits}")
