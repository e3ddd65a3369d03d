"""Pin the oracle's byte layouts against the reference's own index algebra,
evaluated independently with numpy reshape/transpose (analyze.txt:1-20 of the
reference) rather than the closed-form offsets the oracle uses
(kernel/gemm_a4w4.hip:19-25,84-105):

* B preshuffle (16,16): [N,Kp] viewed [N/16,16,Kp/32,2,16], permuted
  (0,2,3,1,4)  (analyze.txt:13-20).
* scale shuffle: [R,S] viewed [R/32,2,16,S/8,2,4], permuted (0,3,5,2,4,1)
  (analyze.txt:1-10).

Plus round trips, bijectivity, and the property the MFMA relies on: one
16-row x 128-K B fragment is 1 KiB contiguous with lane L at L*16, and one
scale dword per lane covers (row L%16 and L%16+16) x (K-half 0 and 1).
"""
import numpy as np
import pytest


def permute_b(w):
    N, Kp = w.shape
    return w.reshape(N // 16, 16, Kp // 32, 2, 16).transpose(0, 2, 3, 1, 4).reshape(N, Kp)


def permute_scales(s):
    R, S = s.shape
    return s.reshape(R // 32, 2, 16, S // 8, 2, 4).transpose(0, 3, 5, 2, 4, 1).reshape(R, S)


@pytest.mark.parametrize("N,K", [(16, 64), (32, 512), (48, 192), (256, 1024)])
def test_shuffle_b_matches_view_permute(oracle_mod, N, K):
    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sb = oracle_mod.shuffle_b(w)
    np.testing.assert_array_equal(sb, permute_b(w))
    np.testing.assert_array_equal(oracle_mod.unshuffle_b(sb), w)


def test_flat_b_is_a_bijection_and_fragments_are_contiguous(oracle_mod):
    N, K = 64, 384
    Kp = K // 2
    L = oracle_mod.lib()
    offs = np.array([[L.oracle_flat_b(n, kp, Kp) for kp in range(Kp)] for n in range(N)])
    assert sorted(offs.ravel().tolist()) == list(range(N * Kp))
    # MFMA fragment (16 rows at n0, K-blocks 4t..4t+3): lane L = block*16 + row
    for n0 in (0, 16, 48):
        for t in range(K // 128):
            for lane in range(64):
                row, blk = lane % 16, lane // 16
                kp0 = t * 64 + blk * 16
                base = (n0 // 16) * K * 8 + t * 1024
                assert offs[n0 + row, kp0] == base + lane * 16
                assert all(offs[n0 + row, kp0 + i] == base + lane * 16 + i for i in range(16))


@pytest.mark.parametrize("R,K", [(32, 256), (64, 512), (96, 2048), (40, 320), (3, 64)])
def test_shuffle_scales_matches_view_permute(oracle_mod, R, K):
    rng = np.random.default_rng(R * K)
    nb = K // 32
    s = rng.integers(0, 255, (R, nb), dtype=np.uint8)
    out = oracle_mod.shuffle_scales(s, K, pad=0xAB)
    Rp, S = out.shape
    assert Rp == (R + 31) // 32 * 32 and S == oracle_mod.scale_pad(K)
    padded = np.full((Rp, S), 0xAB, np.uint8)
    padded[:R, :nb] = s
    np.testing.assert_array_equal(out, permute_scales(padded))
    np.testing.assert_array_equal(oracle_mod.unshuffle_scales(out, R, K), s)


def test_scale_dword_per_lane(oracle_mod):
    """Lane L's dword in a 256-byte (32-row x 8-block) group holds
    (row L%16, block L//16), (row+16, block), (row, block+4), (row+16, block+4)."""
    L = oracle_mod.lib()
    snp = 16
    for r0 in (0, 32):
        for g in (0, 1):
            for lane in range(64):
                row, blk = lane % 16, lane // 16
                base = (r0 // 32) * 32 * snp + g * 256 + lane * 4
                assert L.oracle_flat_s(r0 + row, g * 8 + blk, snp) == base + 0
                assert L.oracle_flat_s(r0 + row + 16, g * 8 + blk, snp) == base + 1
                assert L.oracle_flat_s(r0 + row, g * 8 + blk + 4, snp) == base + 2
                assert L.oracle_flat_s(r0 + row + 16, g * 8 + blk + 4, snp) == base + 3


def test_scale_pad_definition(oracle_mod):
    # interface/gemm_a4w4_pybind.cpp:46-48: round_up(ceil(K/32), 8)
    assert oracle_mod.scale_pad(64) == 8
    assert oracle_mod.scale_pad(256) == 8
    assert oracle_mod.scale_pad(320) == 16
    assert oracle_mod.scale_pad(8192) == 256
    assert oracle_mod.scale_pad(7168) == 224
