"""Pin the oracle's scalar conversions against independent statements of the
same mathematics (not retypings of the oracle's code):

* e2m1 decode  -- the OCP MX v1.0 bit formula (sign, 2-bit exponent bias 1,
  1-bit mantissa, subnormal at exponent 0); code 0x2 == +1.0 as
  kernel/mfma_probe.hip:20 of the reference uses it.
* E8M0 decode  -- math.ldexp(1, e-127) in double (exact), 255 -> NaN.
* MBS factor   -- the exact rational 256/(256+b) rounded to the nearest fp32
  by exhaustive neighbour comparison with Fractions, for all 256 bytes; plus
  the bit construction of test_gemm_a4w4.py:47-51.
* bf16 cast    -- torch's own .to(torch.bfloat16) on random and special values.
"""
import math
from fractions import Fraction

import numpy as np
import pytest


def ocp_e2m1(code: int) -> float:
    s = -1.0 if code & 8 else 1.0
    e = (code >> 1) & 3
    m = code & 1
    if e == 0:
        return s * m * 0.5
    return s * 2.0 ** (e - 1) * (1.0 + m / 2.0)


def test_e2m1_table_matches_ocp_formula(oracle_mod):
    tab = oracle_mod.e2m1_table()
    for c in range(16):
        assert tab[c] == ocp_e2m1(c), c
        assert math.copysign(1.0, tab[c]) == math.copysign(1.0, ocp_e2m1(c)), c
    assert tab[0x2] == 1.0  # mfma_probe.hip:20


def test_e8m0_table(oracle_mod):
    tab = oracle_mod.e8m0_table()
    for e in range(255):
        assert float(tab[e]) == math.ldexp(1.0, e - 127), e
    assert math.isnan(tab[255])
    assert tab.view(np.uint32)[0] == 0x00400000  # 2^-127 is an fp32 subnormal


def nearest_f32(fr: Fraction) -> np.float32:
    """Nearest float32 to an exact positive rational (ties to even)."""
    f = np.float32(float(fr))
    best = f
    for cand in (np.nextafter(f, np.float32(0)), np.nextafter(f, np.float32(np.inf))):
        dc, db = abs(Fraction(float(cand)) - fr), abs(Fraction(float(best)) - fr)
        if dc < db or (dc == db and (int(cand.view(np.uint32)) & 1) == 0):
            best = cand
    return best


def test_mbs_factor_exhaustive(oracle_mod):
    tab = oracle_mod.mbs_factor_table()
    for b in range(256):
        exact = Fraction(256, 256 + b)
        assert tab[b] == nearest_f32(exact), b
        # the bit construction 0x3F800000 | b << 15 is exactly 1 + b/256
        one = np.array([0x3F800000 | (b << 15)], dtype=np.uint32).view(np.float32)[0]
        assert Fraction(float(one)) == 1 + Fraction(b, 256)


def test_bf16_rne_matches_torch(oracle_mod):
    import torch

    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e3),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.0078125, 1.01171875, 3.4e38, -3.4e38,
                  1e-40, -1e-40, np.inf, -np.inf], dtype=np.float32),
        # exact ties in the bf16 rounding: low 16 bits 0x8000
        (rng.integers(0, 2**15, 500, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    x = x[np.isfinite(x) | np.isinf(x)]  # NaN payloads are checked separately below
    ours = oracle_mod.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    # the C restatement agrees with the numpy one
    L = oracle_mod.lib()
    for v in x[:2000]:
        assert L.oracle_f32_to_bf16(float(v)) == oracle_mod.f32_to_bf16_bits(np.array([v]))[0]
    nan = oracle_mod.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0
