"""Pin the oracle's dequantizer, contraction and epilogue:

* dequant: every (code, exponent) product against exact rationals, plus the
  whole-matrix dequant against a per-element rational evaluation.
* contraction: the oracle's fp32 matmul against a float64 matmul of the same
  dequantized operands, within the textbook fp32 summation bound
  K * eps32 * sum|a||b|; and its torch path (run_torch) against the C loop.
* known answers restated from kernel/mfma_probe.hip:95-126 at GEMM level
  (A = B = 1.0 with scale 127 gives K; scale 128 doubles; per-row scales
  2^r put 2^r in row r), and one-hot operands that locate a single product at
  (m, n) -- a transposed operand or swapped nibble moves it.
* epilogue: run_torch_mbs's c * (f(a) f(b)) order (test_gemm_a4w4.py:65-69).
"""
from fractions import Fraction

import numpy as np
import pytest


def test_dequant_every_code_and_exponent(oracle_mod):
    codes = np.arange(16, dtype=np.uint8)
    packed = np.repeat((codes | (codes << 4))[None, :], 256, axis=0)   # [256, 16] -> K=32
    scales = np.arange(256, dtype=np.uint8)[:, None]
    out = oracle_mod.dequant_mxfp4(packed, scales)
    e2m1 = [Fraction(0), Fraction(1, 2), Fraction(1), Fraction(3, 2), Fraction(2), Fraction(3),
            Fraction(4), Fraction(6)]
    fmax = Fraction(float(np.finfo(np.float32).max))
    for e in range(255):
        for k in range(32):
            c = k // 2   # byte k//2 holds code k//2 in both nibbles
            v = e2m1[c & 7] * Fraction(2) ** (e - 127)
            if c & 8:
                v = -v
            if abs(v) > fmax:   # e >= 253 with a large code: fp32 overflow
                assert np.isinf(out[e, k]) and (out[e, k] < 0) == bool(c & 8), (e, k)
            else:
                assert Fraction(float(out[e, k])) == v, (e, k)
    assert np.all(np.isnan(out[255]))


def rand_mx(rng, R, K, lo=110, hi=135):
    packed = rng.integers(0, 256, (R, K // 2), dtype=np.uint8)
    scales = rng.integers(lo, hi, (R, K // 32), dtype=np.uint8)
    return packed, scales


def test_nibble_order_low_first(oracle_mod):
    packed = np.array([[0x2 | (0x4 << 4)] * 16], dtype=np.uint8)   # k even: 1.0, k odd: 2.0
    out = oracle_mod.dequant_mxfp4(packed, np.array([[127]], np.uint8))
    assert np.all(out[0, 0::2] == 1.0) and np.all(out[0, 1::2] == 2.0)


def test_gemm_vs_float64(oracle_mod):
    rng = np.random.default_rng(5)
    M, N, K = 24, 40, 256
    ap, asc = rand_mx(rng, M, K)
    bp, bsc = rand_mx(rng, N, K)
    a = oracle_mod.dequant_mxfp4(ap, asc)
    b = oracle_mod.dequant_mxfp4(bp, bsc)
    c32 = oracle_mod.gemm_f32_small(a, b)
    c64 = a.astype(np.float64) @ b.astype(np.float64).T
    bound = K * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64).T)
    assert np.all(np.abs(c32 - c64) <= bound + 1e-30)
    # run_torch (torch.mm fp32) and the C loop agree to the same bound
    ct = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(ap, bp, asc, bsc))
    cl = oracle_mod.bf16_bits_to_f32(oracle_mod.epilogue_bf16(c32))
    ulp = np.abs(cl) * 2.0 ** -7
    assert np.all(np.abs(ct - cl) <= 2 * bound + ulp)


def ones_operand(R, K):
    return np.full((R, K // 2), 0x22, np.uint8)   # every element e2m1 0x2 = +1.0


@pytest.mark.parametrize("K", [128, 512])
def test_known_answers(oracle_mod, K):
    M, N = 16, 16
    a, b = ones_operand(M, K), ones_operand(N, K)
    s127 = np.full((M, K // 32), 127, np.uint8)
    c = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(a, b, s127, s127[:N]))
    assert np.all(c == K)                                      # probe case "unity": 128 at K=128
    c = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(a, b, s127 + 1, s127[:N]))
    assert np.all(c == 2 * K)                                  # scale 128 doubles
    c = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(a, b, s127 + 1, s127[:N] + 1))
    assert np.all(c == 4 * K)
    c = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(a, b, s127 - 1, s127[:N]))
    assert np.all(c == K / 2)
    # per-K-block scales 127 + block%4: sum over blocks of 32 * 2^(block%4)
    sb = (127 + (np.arange(K // 32) % 4)).astype(np.uint8)[None, :].repeat(M, 0)
    c = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(a, b, sb, s127[:N]))
    assert np.all(c == 32 * 15 * (K // 128))                   # probe case 480 at K=128
    # row scales 2^r and column scales 2^n: C[m][n] = K * 2^(m+n)
    sr = (127 + np.arange(M)).astype(np.uint8)[:, None].repeat(K // 32, 1)
    c = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(a, b, sr, sr[:N]))
    exp = K * 2.0 ** (np.arange(M)[:, None] + np.arange(N)[None, :])
    np.testing.assert_array_equal(c, exp)


def test_one_hot_locates_products(oracle_mod):
    M, N, K = 32, 48, 256
    rng = np.random.default_rng(9)
    for _ in range(20):
        m, n, k = rng.integers(0, M), rng.integers(0, N), rng.integers(0, K)
        a = np.zeros((M, K // 2), np.uint8)
        b = np.zeros((N, K // 2), np.uint8)
        a[m, k // 2] = (0x4 if k % 2 == 0 else 0x40)   # 2.0 at (m, k)
        b[n, k // 2] = (0x5 if k % 2 == 0 else 0x50)   # 3.0 at (n, k)
        s = np.full((max(M, N), K // 32), 127, np.uint8)
        c = oracle_mod.bf16_bits_to_f32(oracle_mod.run_torch(a, b, s[:M], s[:N]))
        exp = np.zeros((M, N), np.float32)
        exp[m, n] = 6.0
        np.testing.assert_array_equal(c, exp)


def test_mbs_epilogue_order(oracle_mod):
    rng = np.random.default_rng(4)
    c = rng.standard_normal((8, 12)).astype(np.float32)
    af = rng.integers(0, 256, 8).astype(np.uint8)
    bf = rng.integers(0, 256, 12).astype(np.uint8)
    tab = oracle_mod.mbs_factor_table()
    exp = c * (tab[af][:, None] * tab[bf][None, :])      # fp32 throughout, factor product first
    got = oracle_mod.epilogue_bf16(c, af, bf)
    np.testing.assert_array_equal(got, oracle_mod.f32_to_bf16_bits(exp.astype(np.float32)))
    # b = 0 means f = 1 exactly: the factor path is the identity
    np.testing.assert_array_equal(oracle_mod.epilogue_bf16(c, np.zeros(8, np.uint8), np.zeros(12, np.uint8)),
                                  oracle_mod.epilogue_bf16(c))


def test_reference_from_kernel_inputs_round_trip(oracle_mod):
    rng = np.random.default_rng(8)
    M, N, K = 40, 48, 320
    ap, asc = rand_mx(rng, M, K)
    bp, bsc = rand_mx(rng, N, K)
    direct = oracle_mod.run_torch(ap, bp, asc, bsc)
    via = oracle_mod.reference_from_kernel_inputs(
        ap, oracle_mod.shuffle_b(bp), oracle_mod.shuffle_scales(asc, K),
        oracle_mod.shuffle_scales(bsc, K), M, N, K)
    np.testing.assert_array_equal(direct, via)
