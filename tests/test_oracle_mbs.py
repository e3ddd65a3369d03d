"""Pin the oracle's MBS quantization (reference docs/kernel_advanced.md:120-129:
per-row max -> scale = 6/max -> top 8 mantissa bits of scale as the factor
byte; the GEMM epilogue divides by 1 + factor/256, test_gemm_a4w4.py:47-51).

The factor byte is recomputed in exact rational arithmetic: 6/amax as a
Fraction, rounded to fp32 (nearest, ties to even) by explicit mantissa
search, then truncated to 8 fraction bits.  Hand-derived known answers and a
bound that the scaled row maximum must satisfy catch an off-by-one shift, a
wrong mantissa slice, or a multiplier applied as a divisor."""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle


def fp32_rne(q: Fraction) -> Fraction:
    """Nearest fp32 to a positive rational (ties to even), exactly; +inf as None."""
    e = math.floor(math.log2(q.numerator) - math.log2(q.denominator))
    while Fraction(2) ** e > q:
        e -= 1
    while Fraction(2) ** (e + 1) <= q:
        e += 1
    if e > 127:
        return None
    e = max(e, -126)                  # subnormal range shares the 2^-126 spacing
    ulp = Fraction(2) ** (e - 23)
    k = q / ulp
    lo = math.floor(k)
    rem = k - lo
    m = lo + (1 if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2) else 0)
    r = m * ulp
    if r >= Fraction(2) ** 128:
        return None
    return r


def factor_byte_exact(amax: float) -> int:
    if not (amax > 0) or math.isinf(amax):
        return 0
    q = fp32_rne(Fraction(6) / Fraction(amax))
    if q is None:                      # 6/amax overflows: +inf, mantissa 0
        return 0
    e = 0
    while Fraction(2) ** e > q:
        e -= 1
    while Fraction(2) ** (e + 1) <= q:
        e += 1
    frac = q / Fraction(2) ** e - 1    # in [0, 1), 23 fraction bits
    return math.floor(frac * 256)


@pytest.mark.parametrize("amax,want", [
    (6.0, 0),      # 6/6 = 1.0
    (3.0, 0),      # 2.0
    (4.0, 128),    # 1.5 = 1.1000_0000b
    (1.0, 128),    # 6 = 1.5 * 4
    (5.0, 51),     # 1.2: fraction 0.2 * 256 = 51.2
    (7.5, 153),    # 0.8 = 1.6 / 2: 0.6 * 256 = 153.6
    (0.0, 0),
    (math.inf, 0),
    (1e-45, 0),    # 6/denormal overflows to +inf
])
def test_factor_byte_known_answers(amax, want):
    assert oracle.mbs_factor_byte(amax) == want
    assert factor_byte_exact(amax) == want


def test_factor_byte_matches_exact_division():
    rng = np.random.default_rng(11)
    bits = rng.integers(0x0080, 0x7F80, 3000).astype(np.uint32) << 16  # positive bf16 values
    vals = bits.view(np.float32)
    for v in list(vals) + [np.float32(6 * 2.0 ** k) for k in range(-20, 20)]:
        assert oracle.mbs_factor_byte(float(v)) == factor_byte_exact(float(v)), v


def test_scaled_row_maximum_bound():
    """6/amax = 2^E (1.f), m = 1.b <= 1.f < m + 2^-8, so the scaled maximum
    amax*m lies in (6*2^-E*(1 - 2^-8), 6*2^-E]: right below a 6*2^j grid top."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 256)) * np.exp(rng.uniform(-8, 8, (64, 1)))).astype(np.float32)
    x = x.astype(np.float32)
    for row in x:
        amax = float(np.max(np.abs(row)))
        b = oracle.mbs_factor_byte(amax)
        m = Fraction(256 + b, 256)
        q = Fraction(6) / Fraction(amax)
        E = math.floor(math.log2(float(q)))
        if Fraction(2) ** E > q:
            E -= 1
        top = Fraction(6) * Fraction(2) ** (-E)
        scaled = Fraction(amax) * m
        assert top * (1 - Fraction(1, 256)) < scaled <= top


def test_mbs_quantize_is_plain_quantize_of_scaled_rows():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((9, 96)).astype(np.float32)
    x[2] = 0.0
    x[4, 7] = np.nan
    x = x.astype(np.float32)
    p, s, f = oracle.quantize_mxfp4_mbs(x)
    for r in range(x.shape[0]):
        row = x[r]
        fb = 0 if np.isnan(row).any() else oracle.mbs_factor_byte(float(np.max(np.abs(row))))
        assert f[r] == fb
        m = np.float32(1 + fb / 256)
        pr, sr = oracle.quantize_mxfp4((row * m)[None, :])
        np.testing.assert_array_equal(p[r], pr[0])
        np.testing.assert_array_equal(s[r], sr[0])


def test_row_maximum_survives_quantization():
    """What the row multiplier buys: the block holding the row maximum no
    longer saturates.  With MBS the dequantized maximum (divided by m) is
    within 2^-8 of the true maximum on every row; plain MXFP4 clips a block
    maximum whose scaled value lands in (6, 8) -- by up to 25% -- and does
    so on some of these rows."""
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((200, 128)) * np.exp(rng.uniform(-3, 3, (200, 1)))).astype(np.float32)
    p, s, f = oracle.quantize_mxfp4_mbs(x)
    deq = oracle.dequant_mxfp4(p, s)
    pp, ps = oracle.quantize_mxfp4(x)
    deq_plain = oracle.dequant_mxfp4(pp, ps)
    worst_plain = 0.0
    for r in range(x.shape[0]):
        k = int(np.argmax(np.abs(x[r])))
        true = abs(float(x[r, k]))
        got = abs(float(deq[r, k])) / (1 + f[r] / 256)
        assert abs(got - true) <= true * 2.0 ** -8, (r, got, true)
        worst_plain = max(worst_plain, abs(abs(float(deq_plain[r, k])) - true) / true)
    assert worst_plain > 0.05
