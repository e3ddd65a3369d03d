"""GPU format kernels against the CPU oracle, bit for bit, through the C ABI:
the quantizer (bf16 -> e2m1 + E8M0, BASELINE configs[0] rule), the B
preshuffle, the scale shuffle, and the dequantizer (the operands of the
reference's dequantize-then-matmul oracle must match bit-exactly)."""
import numpy as np
import pytest

import oracle
from gpu_util import clib, ptr, say, stream_ptr

pytestmark = pytest.mark.gpu


def to_dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def bf16_inputs(rng, R, K):
    """Random finite bf16 bit patterns (all exponents incl. subnormals), plus
    normal data, ties, zero blocks and saturating blocks."""
    bits = rng.integers(0, 2**16, (R, K), dtype=np.uint32).astype(np.uint16)
    exp = (bits >> 7) & 0xFF
    bits[exp == 0xFF] &= 0x807F            # no inf/NaN
    x = (bits.astype(np.uint32) << 16).view(np.float32)
    x[0] = rng.standard_normal(K).astype(np.float32)
    x[1, :32] = 0.0
    x[1, 32:64] = 7.0 * 2.0 ** -20
    if R > 2:
        x[2] = np.tile(np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -5.0], np.float32), K // 8)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("R,K", [(3, 64), (64, 512), (100, 1024), (33, 320)])
def test_quantize_bit_exact(dev, R, K):
    import torch

    rng = np.random.default_rng(R * K)
    xb = bf16_inputs(rng, R, K)
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    ref_p, ref_s = oracle.quantize_mxfp4(xf)
    ref_shuf = oracle.shuffle_scales(ref_s, K, pad=0x5A)
    L = clib()
    x = to_dev(xb)
    packed = torch.empty(R, K // 2, dtype=torch.uint8, device=dev)
    shuf = torch.full(ref_shuf.shape, 0, dtype=torch.uint8, device=dev)
    plain = torch.empty(R, K // 32, dtype=torch.uint8, device=dev)
    say(f"quantize R={R} K={K}")
    assert L.mbs_quantize_mxfp4_bf16(ptr(x), R, K, ptr(packed), ptr(shuf), ptr(plain), 0x5A,
                                     stream_ptr()) == 0
    np.testing.assert_array_equal(host(packed), ref_p)
    np.testing.assert_array_equal(host(plain), ref_s)
    np.testing.assert_array_equal(host(shuf), ref_shuf)


@pytest.mark.parametrize("R,K", [(5, 4128), (7, 96), (4, 32)])
def test_quantize_special_values_and_ragged_grids(dev, R, K):
    """NaN, +-inf, -0, negative values that round to zero and extreme mixes in one
    block, on row counts that are not a multiple of the kernel's 4-row groups and
    chunk counts that leave a partial 64-chunk group (K = 4128: 516 chunks)."""
    import torch

    rng = np.random.default_rng(R + K)
    bits = rng.integers(0, 2**16, (R, K), dtype=np.uint32).astype(np.uint16)
    bits[0, 3] = 0x7FC1                    # NaN: scale 255, block codes 0
    bits[0, 40 % K] = 0xFF80                # -inf (block saturates unless it holds the NaN)
    bits[1, :32] = 0x8000                   # -0 block
    bits[1, 32 % K:(32 % K) + 2] = 0x7F80   # +inf
    bits[2, :32] = 0x8001                   # negative subnormals
    bits[2, 5] = 0x7F7F                     # next to the largest finite value
    if R > 3:
        bits[3, :16] = 0x0001               # tiny positive with a huge one in the block
        bits[3, 16] = 0x7F00
    xf = (bits.astype(np.uint32) << 16).view(np.float32)
    ref_p, ref_s = oracle.quantize_mxfp4(xf)
    ref_shuf = oracle.shuffle_scales(ref_s, K, pad=0x33)
    L = clib()
    x = to_dev(bits)
    packed = torch.empty(R, K // 2, dtype=torch.uint8, device=dev)
    shuf = torch.full(ref_shuf.shape, 0, dtype=torch.uint8, device=dev)
    plain = torch.empty(R, K // 32, dtype=torch.uint8, device=dev)
    say(f"quantize specials R={R} K={K}")
    assert L.mbs_quantize_mxfp4_bf16(ptr(x), R, K, ptr(packed), ptr(shuf), ptr(plain), 0x33,
                                     stream_ptr()) == 0
    np.testing.assert_array_equal(host(packed), ref_p)
    np.testing.assert_array_equal(host(plain), ref_s)
    np.testing.assert_array_equal(host(shuf), ref_shuf)
    assert ref_s[0, 0] == 255 and (K == 32 or ref_s[1, 0] == 0)


@pytest.mark.parametrize("N,K", [(16, 64), (48, 512), (256, 2048)])
def test_shuffles_bit_exact(dev, N, K):
    import torch

    rng = np.random.default_rng(N + K)
    w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s = rng.integers(0, 256, (N, K // 32), dtype=np.uint8)
    L = clib()
    wd, sd = to_dev(w), to_dev(s)
    wo = torch.empty_like(wd)
    so = torch.empty(oracle.round_up(N, 32), oracle.scale_pad(K), dtype=torch.uint8, device=dev)
    say(f"shuffles N={N} K={K}")
    assert L.mbs_shuffle_b(ptr(wd), ptr(wo), N, K, stream_ptr()) == 0
    assert L.mbs_shuffle_scales(ptr(sd), ptr(so), N, K, 0x11, stream_ptr()) == 0
    np.testing.assert_array_equal(host(wo), oracle.shuffle_b(w))
    np.testing.assert_array_equal(host(so), oracle.shuffle_scales(s, K, pad=0x11))


@pytest.mark.parametrize("preshuffled", [False, True])
def test_dequant_bit_exact_all_codes_and_exponents(dev, preshuffled):
    import torch

    R, K = 256, 512
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, (R, K // 2), dtype=np.uint8)
    scales = np.zeros((R, K // 32), np.uint8)
    scales[:, :] = np.arange(256, dtype=np.uint8)[:, None]        # every exponent, one per row
    scales[::7, 3] = rng.integers(0, 256, scales[::7, 3].shape).astype(np.uint8)
    ref = oracle.dequant_mxfp4(packed, scales)
    L = clib()
    src = oracle.shuffle_b(packed) if preshuffled else packed
    pd, sd = to_dev(src), to_dev(oracle.shuffle_scales(scales, K, pad=0))
    out = torch.empty(R, K, dtype=torch.float32, device=dev)
    say(f"dequant preshuffled={preshuffled}")
    assert L.mbs_dequant_mxfp4(ptr(pd), ptr(sd), ptr(out), R, K, int(preshuffled), stream_ptr()) == 0
    got = host(out)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_pybind_format_helpers(dev):
    import torch

    import mbs_amd

    rng = np.random.default_rng(9)
    x = torch.from_numpy(rng.standard_normal((64, 256)).astype(np.float32)).to(torch.bfloat16)
    ref_p, ref_s = oracle.quantize_mxfp4(x.float().numpy())
    say("pybind format helpers")
    p, s = mbs_amd.quantize_mxfp4(x.cuda(), shuffle=False)
    np.testing.assert_array_equal(host(p), ref_p)
    np.testing.assert_array_equal(host(s), ref_s)
    p2, s2 = mbs_amd.quantize_mxfp4(x.cuda(), shuffle=True)
    np.testing.assert_array_equal(host(s2), oracle.shuffle_scales(ref_s, 256, pad=127))
    np.testing.assert_array_equal(host(mbs_amd.shuffle_weight(p)), oracle.shuffle_b(ref_p))
    deq = mbs_amd.dequant_mxfp4(p, s2)
    np.testing.assert_array_equal(host(deq), oracle.dequant_mxfp4(ref_p, ref_s))
