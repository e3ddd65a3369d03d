"""GPU parity of the MBS quantizer (mbs_quantize_mxfp4_mbs_bf16) against the
oracle's restatement (oracle.quantize_mxfp4_mbs), bit for bit: packed codes,
plain and shuffled scales and factor bytes, on ragged shapes and rows whose
maximum is zero, infinite, NaN or subnormal; then the end-to-end MBS GEMM
(both operands MBS-quantized on the GPU, factors undone by the GEMM epilogue)
against the oracle's run_torch with the same factors."""
import ctypes

import numpy as np
import pytest

import oracle
from gpu_util import Case, assert_close, bf16_to_f32, clib, say, stream_ptr

pytestmark = pytest.mark.gpu


def bf16_rows(rng, R, K, spread=3.0):
    x = rng.standard_normal((R, K)) * np.exp(rng.uniform(-spread, spread, (R, 1)))
    bits = (x.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)  # truncate to bf16
    return bits


def run_gpu_mbs(bits):
    import torch

    L = clib()
    L.mbs_quantize_mxfp4_mbs_bf16.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int] + \
        [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p]
    L.mbs_quantize_mxfp4_mbs_bf16.restype = ctypes.c_int
    R, K = bits.shape
    x = torch.from_numpy(bits.view(np.int16)).to("cuda")
    snp = oracle.scale_pad(K)
    packed = torch.empty(R, K // 2, dtype=torch.uint8, device="cuda")
    sshuf = torch.empty(oracle.round_up(R, 32) * snp, dtype=torch.uint8, device="cuda")
    splain = torch.empty(R, K // 32, dtype=torch.uint8, device="cuda")
    fac = torch.empty(R, dtype=torch.uint8, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = L.mbs_quantize_mxfp4_mbs_bf16(P(x), R, K, P(packed), P(sshuf), P(splain), P(fac), 127,
                                       stream_ptr())
    assert st == 0, L.mbs_last_error()
    torch.cuda.synchronize()
    return packed.cpu().numpy(), sshuf.cpu().numpy(), splain.cpu().numpy(), fac.cpu().numpy()


# K = 32768 is the longest row the kernel stages in LDS; K = 32800 takes the
# two-pass (unstaged) form.  Fewer than 256 rows run 1024 threads per row,
# more run 256 (the last two shapes).
@pytest.mark.parametrize("R,K", [(1, 32), (7, 64), (33, 256), (64, 8192), (3, 12288), (7, 32768),
                                 (7, 32800), (300, 1024), (257, 32800)])
def test_mbs_quantizer_bit_exact(dev, R, K):
    rng = np.random.default_rng(R * 131 + K)
    bits = bf16_rows(rng, R, K)
    if R >= 7:
        bits[1] = 0                        # all-zero row: factor 0
        bits[2, 5] = 0x7F80                # +inf: factor 0, block scale 254
        bits[3, K - 1] = 0x7FC1            # NaN: factor 0, NaN block
        bits[4] = (bits[4] & 0x8000) | 0x0001  # subnormal maximum: 6/max overflows
        bits[5, 0] = 0x4200                # 32.0 dominates the row
    say(f"mbs quantizer R={R} K={K}")
    packed, sshuf, splain, fac = run_gpu_mbs(bits)
    x = (bits.astype(np.uint32) << 16).view(np.float32)
    p, s, f = oracle.quantize_mxfp4_mbs(x)
    np.testing.assert_array_equal(fac, f)
    np.testing.assert_array_equal(splain, s)
    np.testing.assert_array_equal(packed, p)
    want = oracle.shuffle_scales(s, K, pad=127).reshape(-1)
    np.testing.assert_array_equal(sshuf, want)


@pytest.mark.parametrize("M,N,K", [(128, 256, 512), (200, 512, 2048), (16, 1024, 4096)])
def test_mbs_gemm_end_to_end(dev, M, N, K):
    import torch

    import mbs_amd

    rng = np.random.default_rng(M + N + K)
    xb = bf16_rows(rng, M, K)
    wb = bf16_rows(rng, N, K, spread=1.0)
    say(f"mbs gemm M={M} N={N} K={K}")
    x = torch.from_numpy(xb.view(np.int16)).to("cuda").view(torch.bfloat16)
    w = torch.from_numpy(wb.view(np.int16)).to("cuda").view(torch.bfloat16)
    A, As, Af = mbs_amd.quantize_mxfp4_mbs(x, shuffle=True)
    Wq, Bs, Bf = mbs_amd.quantize_mxfp4_mbs(w, shuffle=True)
    B = mbs_amd.shuffle_weight(Wq)
    got = bf16_to_f32(mbs_amd.gemm_a4w4(A, B, As, Bs, Af, Bf))[:M]
    xf = (xb.astype(np.uint32) << 16).view(np.float32)
    wf = (wb.astype(np.uint32) << 16).view(np.float32)
    xp, xs, xfac = oracle.quantize_mxfp4_mbs(xf)
    wp, ws, wfac = oracle.quantize_mxfp4_mbs(wf)
    np.testing.assert_array_equal(Af.cpu().numpy(), xfac)
    np.testing.assert_array_equal(Bf.cpu().numpy(), wfac)
    ref = oracle.bf16_bits_to_f32(oracle.run_torch(xp, wp, xs, ws, xfac, wfac))
    assert_close(got, ref, "MBS GEMM vs oracle")
    # the factors undo the multipliers: the result tracks the unquantized product
    exact = xf.astype(np.float64) @ wf.astype(np.float64).T
    rel = np.abs(got - exact).max() / np.abs(exact).max()
    assert rel < 0.25, rel
