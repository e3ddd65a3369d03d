"""Seeded synthetic operands for the five benchmark configurations.

The distributions are the ones BASELINE.json's configs name; the reference
itself draws unseeded ``torch.randn`` bf16 operands (test_gemm_a4w4.py:135-136,
bench_one.py:21-22), so these generators add a seed (``1000 + config index``,
A from ``seed``, W from ``seed + 1``) to make every run reproducible.  All
draws use a CPU ``torch.Generator`` so the bytes do not depend on the device.

Each generator returns bf16 CPU tensors ``x`` [M, K] and ``w`` [N, K]; the
MXFP4 quantization is a separate step (``mbs_amd.formats.quantize_mxfp4`` on
the GPU, or the CPU oracle in the tests).
"""
from __future__ import annotations

import math

import torch

# (config index) -> base seed
SEED_BASE = 1000


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def normal(rows: int, cols: int, std: float, seed: int) -> torch.Tensor:
    x = torch.randn(rows, cols, generator=_gen(seed), dtype=torch.float32)
    return (x * std).to(torch.bfloat16)


def normal_with_outlier_channels(rows: int, cols: int, seed: int, frac: float = 0.01,
                                 gain: float = 20.0) -> torch.Tensor:
    """N(0,1) with ``round(frac*cols)`` K-channels (columns) scaled by ``gain``."""
    g = _gen(seed)
    x = torch.randn(rows, cols, generator=g, dtype=torch.float32)
    n_out = max(1, int(round(frac * cols)))
    cols_out = torch.randperm(cols, generator=g)[:n_out]
    x[:, cols_out] *= gain
    return x.to(torch.bfloat16)


def laplace(rows: int, cols: int, seed: int, scale: float = 1.0) -> torch.Tensor:
    """Laplace(0, scale) by the inverse CDF of a seeded uniform draw."""
    u = torch.rand(rows, cols, generator=_gen(seed), dtype=torch.float64) - 0.5
    x = -scale * torch.sign(u) * torch.log1p(-2.0 * u.abs())
    return x.to(torch.bfloat16)


def rowwise_lognormal_sigma(rows: int, cols: int, seed: int, lo: float = 0.005,
                            hi: float = 0.05) -> torch.Tensor:
    """Row r ~ N(0, sigma_r) with log sigma_r ~ U(log lo, log hi)."""
    g = _gen(seed)
    u = torch.rand(rows, 1, generator=g, dtype=torch.float64)
    sigma = torch.exp(math.log(lo) + u * (math.log(hi) - math.log(lo)))
    x = torch.randn(rows, cols, generator=g, dtype=torch.float64) * sigma
    return x.to(torch.bfloat16)


def inject_edge_blocks(x: torch.Tensor, seed: int, frac_zero: float = 0.02,
                       frac_sat: float = 0.02) -> torch.Tensor:
    """Set some 32-element K-blocks to all-zero (-> E8M0 0x00) and some to
    +-7 * 2^k (-> amax 7*2^k, block exponent k, every element saturates to
    +-6 * 2^k)."""
    g = _gen(seed)
    R, K = x.shape
    nb = K // 32
    xb = x.to(torch.float32).reshape(R, nb, 32).clone()
    pick = torch.rand(R, nb, generator=g)
    zero = pick < frac_zero
    sat = (pick >= frac_zero) & (pick < frac_zero + frac_sat)
    xb[zero] = 0.0
    k = torch.randint(-6, 4, (R, nb, 1), generator=g).to(torch.float32)
    sign = torch.where(torch.rand(R, nb, 32, generator=g) < 0.5, -1.0, 1.0)
    satv = sign * 7.0 * torch.exp2(k)
    xb = torch.where(sat.unsqueeze(-1), satv, xb)
    return xb.reshape(R, K).to(torch.bfloat16)


# --------------------------------------------------------------- configs

CFG0 = dict(M=128, N=256, K=512)
CFG1 = dict(M=8192, N=8192, K=8192)
CFG2_M = (1, 4, 16, 32)
CFG2_NK = (8192, 8192)
CFG3_M = (256, 2048)
CFG3_NK = ((7168, 2048), (4096, 7168), (2112, 7168))
CFG4_M = (1000, 3333)
CFG4_N = (1280, 5120)
CFG4_K = (512, 12288)


def config_shapes(cfg: int) -> list[tuple[int, int, int]]:
    """Every (M, N, K) of one configuration."""
    if cfg == 0:
        return [(CFG0["M"], CFG0["N"], CFG0["K"])]
    if cfg == 1:
        return [(CFG1["M"], CFG1["N"], CFG1["K"])]
    if cfg == 2:
        return [(m, CFG2_NK[0], CFG2_NK[1]) for m in CFG2_M]
    if cfg == 3:
        return [(m, n, k) for m in CFG3_M for (n, k) in CFG3_NK]
    if cfg == 4:
        return [(m, n, k) for m in CFG4_M for n in CFG4_N for k in CFG4_K]
    raise ValueError(cfg)


def make_operands(cfg: int, M: int, N: int, K: int) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (x [M,K], w [N,K]) for configuration ``cfg`` at shape (M,N,K).

    The seed also folds in the shape so the several shapes of one
    configuration get independent draws."""
    seed = SEED_BASE + cfg + 7919 * (M + 31 * N + 997 * K)
    if cfg == 0:
        return normal(M, K, 1.0, seed), normal(N, K, 0.02, seed + 1)
    if cfg in (1, 2):
        return normal_with_outlier_channels(M, K, seed), normal(N, K, 0.02, seed + 1)
    if cfg == 3:
        return laplace(M, K, seed), rowwise_lognormal_sigma(N, K, seed + 1)
    if cfg == 4:
        x = inject_edge_blocks(normal(M, K, 1.0, seed), seed + 2)
        w = inject_edge_blocks(normal(N, K, 0.02, seed + 1), seed + 3)
        return x, w
    raise ValueError(cfg)


def make_factors(M: int, N: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    """MBS factor bytes, [M, 1] and [N, 1] uint8 (test_gemm_a4w4.py:146-147)."""
    g = _gen(seed)
    a = torch.randint(0, 256, (M, 1), generator=g, dtype=torch.int32).to(torch.uint8)
    b = torch.randint(0, 256, (N, 1), generator=g, dtype=torch.int32).to(torch.uint8)
    return a, b
