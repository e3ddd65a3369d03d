"""Pin the oracle's affine epilogue (out = bf16(c * ((f(a) * alpha) * f(b)) +
bias), fp32, no fused multiply-add): it reduces to the pinned MBS epilogue at
alpha 1 without bias, scales exactly by powers of two, and matches an
element-by-element restatement in explicitly rounded fp32 arithmetic
(struct-packed single precision), which would catch a fused add, a bias
added before the scaling, or alpha applied after the bf16 rounding."""
import struct

import numpy as np

import oracle


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def bf16_rne_bits(x: float) -> int:
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    if (u & 0x7FFFFFFF) > 0x7F800000:
        return ((u >> 16) | 0x40) & 0xFFFF
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def test_reduces_to_mbs_epilogue():
    rng = np.random.default_rng(2)
    c = (rng.standard_normal((33, 48)) * 10).astype(np.float32)
    af = rng.integers(0, 256, 33, dtype=np.uint8)
    bf = rng.integers(0, 256, 48, dtype=np.uint8)
    np.testing.assert_array_equal(oracle.epilogue_affine_bf16(c, af, bf), oracle.epilogue_bf16(c, af, bf))
    np.testing.assert_array_equal(oracle.epilogue_affine_bf16(c), oracle.epilogue_bf16(c))


def test_power_of_two_alpha_is_exact():
    rng = np.random.default_rng(3)
    c = (rng.standard_normal((16, 64)) * 3).astype(np.float32)
    base = oracle.bf16_bits_to_f32(oracle.epilogue_affine_bf16(c))
    for a in (0.25, 2.0, 8.0):
        got = oracle.bf16_bits_to_f32(oracle.epilogue_affine_bf16(c, alpha=a))
        np.testing.assert_array_equal(got, base * np.float32(a))


def test_elementwise_restatement():
    rng = np.random.default_rng(4)
    M, N = 7, 9
    c = (rng.standard_normal((M, N)) * 5).astype(np.float32)
    af = rng.integers(0, 256, M, dtype=np.uint8)
    bf = rng.integers(0, 256, N, dtype=np.uint8)
    bias = oracle.f32_to_bf16_bits(rng.standard_normal(N).astype(np.float32))
    alpha = 0.7
    got = oracle.epilogue_affine_bf16(c, af, bf, alpha, bias)
    for m in range(M):
        for n in range(N):
            sa = f32(float(oracle.mbs_factor(af[m])) * f32(alpha))
            s = f32(sa * float(oracle.mbs_factor(bf[n])))
            v = f32(float(c[m, n]) * s)
            b = struct.unpack("<f", struct.pack("<I", int(bias[n]) << 16))[0]
            assert got[m, n] == bf16_rne_bits(f32(v + b)), (m, n)
