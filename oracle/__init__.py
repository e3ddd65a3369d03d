"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the MXFP4 A4W4 GEMM path.

A numpy/ctypes front end over ``oracle/mxfp4_oracle.c`` (built into
``oracle/liboracle.so`` by ``make -C oracle``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only to check or time the CPU path; the shipped HIP path
never routes through it.

What each function restates (paths relative to the reference tree):

* ``quantize_mxfp4`` -- the MXFP4 quantizer rule of BASELINE.json configs[0]
  (OCP MX v1.0); the reference delegates quantization to aiter's Triton
  ``per_1x32`` quantizer (``test_gemm_a4w4.py:134-140``), which is absent here,
  so parity with *aiter's* rounding is unpinned -- both the GPU kernel and this
  oracle consume the same bytes, so the GEMM parity does not depend on it.
* ``dequant_mxfp4`` -- ``fp4_utils.mxfp4_to_f32(x) * e8m0_to_f32(scales
  .repeat_interleave(32))`` of ``test_gemm_a4w4.py:33-42``.
* ``shuffle_b`` / ``unshuffle_b`` -- ``shuffle_weight(w, layout=(16,16))``
  decoded as ``flatB`` (``kernel/gemm_a4w4.hip:19-22,84-95``; ``analyze.txt:13-20``).
* ``shuffle_scales`` / ``unshuffle_scales`` -- the quantizer's ``shuffle=True``
  scale layout, decoded as ``flatS`` (``kernel/gemm_a4w4.hip:23-25,97-105``;
  ``analyze.txt:1-10``).
* ``mbs_factor`` -- ``convert_byte_to_float`` (``test_gemm_a4w4.py:47-51``).
* ``run_torch`` / ``run_torch_mbs`` -- ``test_gemm_a4w4.py:28-44`` and ``:54-69``:
  dequantize to fp32, ``torch.mm`` in fp32, optional factor epilogue, bf16.

How each is pinned (tests/test_oracle_*.py): closed forms (OCP tables, exact
rationals), the view/permute algebra of ``analyze.txt`` evaluated with numpy
independently of the closed-form offsets, brute force on small inputs, the
scaled-MFMA known answers of ``kernel/mfma_probe.hip:95-126`` restated at the
GEMM level, and the committed config-0 golden vectors.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

SCALE_GROUP_SIZE = 32  # test_gemm_a4w4.py:21


def lib() -> ctypes.CDLL:
    """Load ``liboracle.so`` (built by ``make -C oracle``); raise if absent."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        L.oracle_e2m1_to_f32.argtypes = [ctypes.c_uint8]
        L.oracle_e2m1_to_f32.restype = ctypes.c_float
        L.oracle_e8m0_to_f32.argtypes = [ctypes.c_uint8]
        L.oracle_e8m0_to_f32.restype = ctypes.c_float
        L.oracle_mbs_factor.argtypes = [ctypes.c_uint8]
        L.oracle_mbs_factor.restype = ctypes.c_float
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_flat_b.argtypes = [I, I, I]
        L.oracle_flat_b.restype = I
        L.oracle_flat_s.argtypes = [I, I, I]
        L.oracle_flat_s.restype = I
        L.oracle_quantize_mxfp4.argtypes = [P, I, I, P, P]
        L.oracle_quantize_mxfp4_mbs.argtypes = [P, I, I, P, P, P]
        L.oracle_quantize_mxfp4_mbs.restype = None
        L.oracle_mbs_factor_byte.argtypes = [ctypes.c_float]
        L.oracle_mbs_factor_byte.restype = ctypes.c_uint8
        L.oracle_dequant_mxfp4.argtypes = [P, P, I, I, P]
        L.oracle_shuffle_b.argtypes = [P, I, I, P]
        L.oracle_unshuffle_b.argtypes = [P, I, I, P]
        L.oracle_shuffle_scales.argtypes = [P, I, I, I, ctypes.c_uint8, P]
        L.oracle_unshuffle_scales.argtypes = [P, I, I, I, P]
        L.oracle_gemm_f32.argtypes = [P, P, I, I, I, P]
        L.oracle_epilogue_bf16.argtypes = [P, I, I, P, P, P]
        for f in ("oracle_quantize_mxfp4", "oracle_dequant_mxfp4", "oracle_shuffle_b",
                  "oracle_unshuffle_b", "oracle_shuffle_scales", "oracle_unshuffle_scales",
                  "oracle_gemm_f32", "oracle_epilogue_bf16"):
            getattr(L, f).restype = None
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a).view(np.uint8) if np.asarray(a).dtype != np.uint8
                                else np.asarray(a))


# ----------------------------------------------------------------- scalars

def e2m1_table() -> np.ndarray:
    """fp32 value of each of the 16 e2m1 codes."""
    L = lib()
    return np.array([L.oracle_e2m1_to_f32(c) for c in range(16)], dtype=np.float32)


def e8m0_table() -> np.ndarray:
    """fp32 value 2^(e-127) of each E8M0 byte (255 -> NaN)."""
    L = lib()
    return np.array([L.oracle_e8m0_to_f32(e) for e in range(256)], dtype=np.float32)


def mbs_factor_table() -> np.ndarray:
    """f(b) = 1/(1+b/256) as fp32 for every factor byte b."""
    L = lib()
    return np.array([L.oracle_mbs_factor(b) for b in range(256)], dtype=np.float32)


def mbs_factor(b) -> np.ndarray:
    return mbs_factor_table()[np.asarray(b, dtype=np.uint8)]


def scale_pad(K: int) -> int:
    """scaleN_pad = round_up(ceil(K/32), 8) (interface/gemm_a4w4_pybind.cpp:46-48)."""
    return ((K + 31) // 32 + 7) // 8 * 8


def round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


# ----------------------------------------------------------- conversions

def quantize_mxfp4(x) -> tuple[np.ndarray, np.ndarray]:
    """fp32/bf16-valued [R, K] -> (packed u8 [R, K/2], plain E8M0 u8 [R, K/32])."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    R, K = x.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    packed = np.empty((R, K // 2), dtype=np.uint8)
    scales = np.empty((R, K // 32), dtype=np.uint8)
    lib().oracle_quantize_mxfp4(_ptr(x), R, K, _ptr(packed), _ptr(scales))
    return packed, scales


def mbs_factor_byte(amax: float) -> int:
    """MBS factor byte of a row maximum: top 8 mantissa bits of 6/amax."""
    return int(lib().oracle_mbs_factor_byte(float(amax)))


def quantize_mxfp4_mbs(x) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """MBS quantization (docs/kernel_advanced.md:120-129 of the reference):
    fp32/bf16-valued [R, K] -> (packed u8 [R, K/2], plain E8M0 u8 [R, K/32],
    factor bytes u8 [R]); row r is quantized after scaling by 1 + f[r]/256."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    R, K = x.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    packed = np.empty((R, K // 2), dtype=np.uint8)
    scales = np.empty((R, K // 32), dtype=np.uint8)
    factors = np.empty((R,), dtype=np.uint8)
    lib().oracle_quantize_mxfp4_mbs(_ptr(x), R, K, _ptr(packed), _ptr(scales), _ptr(factors))
    return packed, scales, factors


def dequant_mxfp4(packed, scales) -> np.ndarray:
    """packed u8 [R, K/2] + plain E8M0 u8 [R, K/32] -> fp32 [R, K]."""
    packed = _u8(packed)
    scales = _u8(scales)
    R, Kp = packed.shape
    K = 2 * Kp
    assert scales.shape[0] >= R and scales.shape[1] >= K // 32
    scales = np.ascontiguousarray(scales[:R, : K // 32])
    out = np.empty((R, K), dtype=np.float32)
    lib().oracle_dequant_mxfp4(_ptr(packed), _ptr(scales), R, K, _ptr(out))
    return out


def shuffle_b(w) -> np.ndarray:
    """Plain packed weights [N, K/2] -> preshuffled (16,16) buffer [N, K/2]."""
    w = _u8(w)
    N, Kp = w.shape
    if N % 16 or Kp % 32:
        raise ValueError("shuffle_b needs N % 16 == 0 and K % 64 == 0")
    out = np.empty_like(w)
    lib().oracle_shuffle_b(_ptr(w), N, Kp, _ptr(out))
    return out


def unshuffle_b(buf) -> np.ndarray:
    buf = _u8(buf)
    N, Kp = buf.shape
    out = np.empty_like(buf)
    lib().oracle_unshuffle_b(_ptr(buf), N, Kp, _ptr(out))
    return out


def shuffle_scales(s, K: int | None = None, pad: int = 127) -> np.ndarray:
    """Plain E8M0 [R, nb] -> shuffled flat buffer of round_up(R,32)*scaleN_pad
    bytes, returned as [round_up(R,32), scaleN_pad].  Padding gets ``pad``."""
    s = _u8(s)
    R, nb = s.shape
    snp = scale_pad(K if K is not None else nb * 32)
    out = np.empty((round_up(R, 32), snp), dtype=np.uint8)
    lib().oracle_shuffle_scales(_ptr(s), R, nb, snp, pad, _ptr(out))
    return out


def unshuffle_scales(buf, rows: int, K: int) -> np.ndarray:
    buf = _u8(buf).reshape(-1)
    nb = K // 32
    snp = scale_pad(K)
    assert buf.size >= round_up(rows, 32) * snp
    out = np.empty((rows, nb), dtype=np.uint8)
    lib().oracle_unshuffle_scales(_ptr(np.ascontiguousarray(buf)), rows, nb, snp, _ptr(out))
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ GEMM

def gemm_f32_small(a, b) -> np.ndarray:
    """c = a . b^T with a sequential fp32 accumulator (C loop; small sizes)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    M, K = a.shape
    N = b.shape[0]
    c = np.empty((M, N), dtype=np.float32)
    lib().oracle_gemm_f32(_ptr(a), _ptr(b), M, N, K, _ptr(c))
    return c


def epilogue_bf16(c, a_factor=None, b_factor=None) -> np.ndarray:
    """run_torch_mbs epilogue: c * (f(a)[m] * f(b)[n]) then bf16 (uint16 bits)."""
    c = np.ascontiguousarray(c, dtype=np.float32)
    M, N = c.shape
    out = np.empty((M, N), dtype=np.uint16)
    if a_factor is None or b_factor is None:
        lib().oracle_epilogue_bf16(_ptr(c), M, N, None, None, _ptr(out))
    else:
        af = np.ascontiguousarray(np.asarray(a_factor, dtype=np.uint8).reshape(-1))
        bf = np.ascontiguousarray(np.asarray(b_factor, dtype=np.uint8).reshape(-1))
        assert af.size == M and bf.size == N
        lib().oracle_epilogue_bf16(_ptr(c), M, N, _ptr(af), _ptr(bf), _ptr(out))
    return out


def epilogue_affine_bf16(c, a_factor=None, b_factor=None, alpha: float = 1.0,
                        bias_bits=None) -> np.ndarray:
    """The affine epilogue (no reference counterpart in its own launcher; the
    aiter GEMM its harness calls next to it takes a bias,
    test_gemm_a4w4.py:95-123): in fp32, c * ((f(a)[m] * alpha) * f(b)[n]),
    plus bias[n] (bf16 bits) when given, then bf16 RNE (uint16 bits).  The
    factors are 1 when absent.  With alpha 1 and no bias this is
    epilogue_bf16."""
    c = np.ascontiguousarray(c, dtype=np.float32)
    M, N = c.shape
    fa = (mbs_factor(np.asarray(a_factor, np.uint8).reshape(-1)) if a_factor is not None
          else np.ones(M, np.float32)).astype(np.float32)
    fb = (mbs_factor(np.asarray(b_factor, np.uint8).reshape(-1)) if b_factor is not None
          else np.ones(N, np.float32)).astype(np.float32)
    sa = (fa * np.float32(alpha)).astype(np.float32)
    v = (c * (sa[:, None] * fb[None, :]).astype(np.float32)).astype(np.float32)
    if bias_bits is not None:
        b = (np.asarray(bias_bits, np.uint16).astype(np.uint32) << 16).view(np.float32)
        v = (v + b[None, :]).astype(np.float32)
    return f32_to_bf16_bits(v)


def run_torch(x_packed, w_packed, x_scales, w_scales, a_factor=None, b_factor=None,
              threads: int | None = None):
    """Restatement of run_torch / run_torch_mbs (test_gemm_a4w4.py:28-44,54-69).

    Inputs are the *plain* layouts the reference oracle reads: packed A [M,K/2],
    packed W [N,K/2], plain scales [>=M, K/32] / [>=N, K/32] (the oracle slices
    ``[:m]``).  Returns the bf16 result as uint16 bits [M, N].  The fp32 matmul
    runs in torch on the CPU, the same library routine the reference oracle
    calls on its device.
    """
    import torch

    if threads:
        torch.set_num_threads(threads)
    xf = dequant_mxfp4(x_packed, x_scales)
    wf = dequant_mxfp4(w_packed, w_scales)
    c = torch.mm(torch.from_numpy(xf), torch.from_numpy(wf).T).numpy()
    return epilogue_bf16(c, a_factor, b_factor)


def reference_from_kernel_inputs(A, B_shuf, A_scale_shuf, B_scale_shuf, M, N, K,
                                 a_factor=None, b_factor=None):
    """Run the oracle on the kernel-layout inputs (plain A, preshuffled B,
    shuffled scales): unshuffle, then ``run_torch``.  Returns bf16 bits [M, N]."""
    B = unshuffle_b(np.asarray(B_shuf).reshape(N, K // 2))
    As = unshuffle_scales(A_scale_shuf, M, K)
    Bs = unshuffle_scales(B_scale_shuf, N, K)
    return run_torch(np.asarray(A).reshape(M, K // 2), B, As, Bs, a_factor, b_factor)
