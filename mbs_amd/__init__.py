"""mbs_amd -- MI355X (gfx950) MXFP4 A4W4 GEMM.

The product is two in-tree shared objects under ``mbs_amd/lib/`` (build them
with ``python -m mbs_amd._build``):

* ``libmbs_gemm_kernel.so`` -- HIP kernels behind the C ABI declared in
  ``include/mbs_gemm_a4w4.h``;
* ``mbs_gemm_a4w4.*.so`` -- the torch module with the reference's operator
  ``gemm_a4w4(A, B, A_scale, B_scale, A_factor=None, B_factor=None)``.

``import mbs_gemm_a4w4`` works once ``mbs_amd/lib`` is on ``sys.path``
(importing this package puts it there); the names are re-exported here.
Nothing here falls back to a CPU path: if the libraries are missing the
import fails.
"""
from __future__ import annotations

import ctypes
import glob
import importlib
import os
import sys

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
KERNEL_LIB_PATH = os.path.join(LIB_DIR, "libmbs_gemm_kernel.so")

_ext = None
_clib = None


def _load_ext():
    global _ext
    if _ext is None:
        if not glob.glob(os.path.join(LIB_DIR, "mbs_gemm_a4w4*.so")):
            raise ImportError(
                f"mbs_gemm_a4w4 extension not built in {LIB_DIR}; run `python -m mbs_amd._build`")
        import torch  # noqa: F401  (the module links against torch)

        if LIB_DIR not in sys.path:
            sys.path.insert(0, LIB_DIR)
        _ext = importlib.import_module("mbs_gemm_a4w4")
    return _ext


def ext():
    """The ``mbs_gemm_a4w4`` extension module."""
    return _load_ext()


def clib() -> ctypes.CDLL:
    """ctypes handle on ``libmbs_gemm_kernel.so`` (the C ABI).

    torch is imported first: torch ships its own HIP runtime under the same
    soname (libamdhip64.so.7) as the ROCm one this library links against, and
    whichever is loaded first serves the whole process.  Loading torch first
    keeps this library on the runtime that owns torch's memory and streams."""
    global _clib
    if _clib is None:
        if not os.path.exists(KERNEL_LIB_PATH):
            raise ImportError(f"{KERNEL_LIB_PATH} not built; run `python -m mbs_amd._build`")
        import torch  # noqa: F401  (see above)

        _clib = ctypes.CDLL(KERNEL_LIB_PATH)
    return _clib


def gemm_a4w4(A, B, A_scale, B_scale, A_factor=None, B_factor=None, alpha: float = 1.0,
              bias=None):
    """out[M,N] bf16 = dequant(A) @ dequant(B)^T [* f(A_factor)[:,None] * f(B_factor)[None,:]].

    Same contract as the reference's ``mbs_gemm_a4w4.gemm_a4w4``
    (interface/gemm_a4w4_pybind.cpp:19-64): A [M,K/2] fp4x2 row-major, B
    [N,K/2] fp4x2 preshuffled (16,16), shuffled E8M0 scales, optional u8
    factors.  Asynchronous on the current stream.  Beyond the reference: an
    affine epilogue, out = bf16(C * alpha * f(a) * f(b) + bias[n]) with bias a
    bf16 [N] device tensor; the defaults leave the reference's result."""
    return ext().gemm_a4w4(A, B, A_scale, B_scale, A_factor, B_factor, alpha, bias)


def gemm_a4w4_from_bf16(x, B, B_scale, alpha: float = 1.0, bias=None, config: int = -1,
                        splits: int = 0, one_launch=None, B_factor=None):
    """out[M,N] bf16 from a bf16 activation x [M,K]: the reference's decode
    flow, the per_1x32 quantizer then ``gemm_a4w4`` (test_gemm_a4w4.py:134-141,
    bench_one.py:19-30), with the same output bytes as quantizing x with
    ``quantize_mxfp4`` and calling ``gemm_a4w4`` on the result.  It runs in
    one launch (the decode kernel quantizes x in registers) for M <= 8, where
    that is faster, and as the two launches otherwise; ``one_launch=True``
    forces the one-launch form (M <= 32), ``False`` the two launches.
    ``config``/``splits`` force a skinny (decode) configuration of the
    one-launch form.  With ``B_factor`` (the weights' MBS factor bytes) x is
    MBS-quantized instead, as ``quantize_mxfp4_mbs`` does, and both factors
    apply (one launch by default for M <= 4, forced up to M <= 8: the row
    factors are derived in the kernel)."""
    mode = -1 if one_launch is None else int(bool(one_launch))
    return ext().gemm_a4w4_from_bf16(x, B, B_scale, B_factor, alpha, bias, config, splits, mode)


def gemm_a4w4_grouped(A, B, A_scale, B_scale, group_offsets, A_factor=None, B_factor=None,
                      config: int = -1, alpha: float = 1.0, bias=None, validate: bool = False):
    """Grouped (mixture-of-experts) GEMM in one launch.

    Expert e owns rows [group_offsets[e], group_offsets[e+1]) of A and of the
    output, and the e-th [N, K/2] preshuffled block of B (B is [E, N, K/2] or
    [E*N, K/2]), its shuffled scale block and its N factor bytes.  Offsets are
    int32 [E+1]: 0 first, non-decreasing multiples of 32 (pad each expert's
    token block), last <= M.  Each expert's rows equal ``gemm_a4w4`` of that
    expert alone.  Rows past the last offset are not written.  ``alpha`` and
    ``bias`` (bf16 [E, N] or [E*N], expert e's row added to its rows) give the
    affine epilogue of ``gemm_a4w4``.  Host offsets are checked on the host;
    device offsets are read by the kernel unchecked (an expert starting off a
    32-row boundary is skipped, out-of-range offsets are clamped) unless
    ``validate`` asks for a device-side check first (it synchronises)."""
    return ext().gemm_a4w4_grouped(A, B, A_scale, B_scale, group_offsets, A_factor, B_factor,
                                   config, alpha, bias, validate)


def check_groups(group_offsets, M: int):
    """(non-empty experts whose first row is not a multiple of 32, offsets
    outside [0, M] or decreasing) of an int32 device offset vector;
    synchronises the stream."""
    return ext().check_groups(group_offsets, M)


def quantize_mxfp4(x, shuffle: bool = True, pad_byte: int = 127):
    """bf16 [R,K] device tensor -> (packed u8 [R,K/2], E8M0 scales);
    shuffled [round_up(R,32), scaleN_pad] when ``shuffle`` else plain [R,K/32]."""
    return ext().quantize_mxfp4(x, shuffle, pad_byte)


def quantize_mxfp4_mbs(x, shuffle: bool = True, pad_byte: int = 127):
    """MBS quantization: bf16 [R,K] device tensor -> (packed, E8M0 scales,
    factor bytes u8 [R]).  Row r is scaled by 1 + f[r]/256 (f = top 8
    mantissa bits of 6/max|row r|) before quantization; passing the factors
    of A and B to ``gemm_a4w4`` undoes the scaling in the epilogue."""
    return ext().quantize_mxfp4_mbs(x, shuffle, pad_byte)


def shuffle_weight(w):
    """(16,16) preshuffle of packed weights [N,K/2] (out of place)."""
    return ext().shuffle_weight(w)


def shuffle_scales(s, pad_byte: int = 127):
    return ext().shuffle_scales(s, pad_byte)


def dequant_mxfp4(packed, scale, b_preshuffled: bool = False):
    return ext().dequant_mxfp4(packed, scale, b_preshuffled)


def unshuffle_weight(b):
    """Inverse of ``shuffle_weight``: preshuffled [N,K/2] -> plain [N,K/2]."""
    return ext().unshuffle_weight(b)


def unshuffle_scales(s, rows: int, K: int):
    """Shuffled E8M0 buffer -> plain [rows, K/32] (padding dropped)."""
    return ext().unshuffle_scales(s, rows, K)


def check_scales(s, rows: int, K: int, pad_byte: int = 127):
    """(padding bytes != pad_byte, live 0xFF bytes) of a shuffled scale buffer;
    ``pad_byte=-1`` skips the padding check.  Synchronises."""
    return ext().check_scales(s, rows, K, pad_byte)


def scale_pad(K: int) -> int:
    """scaleN_pad = round_up(ceil(K/32), 8)."""
    return ((K + 31) // 32 + 7) // 8 * 8


def round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m
