"""Helpers for the GPU parity tests: C-ABI calls through ctypes (torch only
holds device memory and supplies the stream), operand construction from the
CPU oracle, and the north-star tolerance

    |got - ref| <= 1e-2 * max|ref| + 1 bf16 ulp(ref)      (elementwise)

where ref is the reference oracle's bf16 output (dequantize to fp32, fp32
matmul, optional factors, bf16)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np

import oracle


def say(msg: str) -> None:
    """Name the case before GPU work starts, flushed, so a crash is attributable."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def clib():
    import mbs_amd

    L = mbs_amd.clib()
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.mbs_gemm_a4w4_launch.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, P, S, P]
    L.mbs_gemm_a4w4_launch.restype = I
    L.mbs_gemm_a4w4_launch_config.argtypes = [I, I, P, P, P, P, P, P, P, I, I, I, I, I, P, S, P]
    L.mbs_gemm_a4w4_launch_config.restype = I
    L.mbs_gemm_a4w4_workspace_bytes.argtypes = [I, I, I]
    L.mbs_gemm_a4w4_workspace_bytes.restype = S
    L.mbs_gemm_a4w4_config_workspace_bytes.argtypes = [I, I, I, I, I]
    L.mbs_gemm_a4w4_config_workspace_bytes.restype = S
    L.mbs_gemm_a4w4_config_name.restype = ctypes.c_char_p
    L.mbs_last_error.restype = ctypes.c_char_p
    L.mbs_quantize_mxfp4_bf16.argtypes = [P, I, I, P, P, P, I, P]
    L.mbs_shuffle_b.argtypes = [P, P, I, I, P]
    L.mbs_shuffle_scales.argtypes = [P, P, I, I, I, P]
    L.mbs_dequant_mxfp4.argtypes = [P, P, P, I, I, I, P]
    for f in ("mbs_quantize_mxfp4_bf16", "mbs_shuffle_b", "mbs_shuffle_scales", "mbs_dequant_mxfp4"):
        getattr(L, f).restype = I
    return L


def stream_ptr():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Case:
    """One GEMM problem: oracle-made bytes on the host and on the device."""

    def __init__(self, x_packed, x_scales, w_packed, w_scales, a_factor=None, b_factor=None,
                 dev="cuda:0", scale_pad_byte=127):
        import torch

        self.M, Kp = x_packed.shape
        self.N = w_packed.shape[0]
        self.K = 2 * Kp
        self.Mpad = oracle.round_up(self.M, 32)
        self.snp = oracle.scale_pad(self.K)
        self.x_packed, self.x_scales = x_packed, x_scales
        self.w_packed, self.w_scales = w_packed, w_scales
        self.a_factor, self.b_factor = a_factor, b_factor
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.A = t(x_packed)
        self.B = t(oracle.shuffle_b(w_packed))
        self.As = t(oracle.shuffle_scales(x_scales, self.K, pad=scale_pad_byte))
        self.Bs = t(oracle.shuffle_scales(w_scales, self.K, pad=scale_pad_byte))
        self.Af = None if a_factor is None else t(np.asarray(a_factor, np.uint8).reshape(-1))
        self.Bf = None if b_factor is None else t(np.asarray(b_factor, np.uint8).reshape(-1))

    @classmethod
    def from_bf16(cls, x, w, factors=None, **kw):
        xp, xs = oracle.quantize_mxfp4(x.float().numpy())
        wp, ws = oracle.quantize_mxfp4(w.float().numpy())
        af, bf = (None, None) if factors is None else factors
        return cls(xp, xs, wp, ws, af, bf, **kw)

    def reference(self, rows=None):
        """Oracle bf16 bits for all rows, or for the given row indices."""
        if rows is None:
            return oracle.run_torch(self.x_packed, self.w_packed, self.x_scales, self.w_scales,
                                    self.a_factor, self.b_factor)
        rows = np.asarray(rows)
        af = None if self.a_factor is None else np.asarray(self.a_factor).reshape(-1)[rows]
        return oracle.run_torch(self.x_packed[rows], self.w_packed, self.x_scales[rows],
                                self.w_scales, af, self.b_factor)

    def run(self, config=None, splits=0, out=None, check=True):
        """Launch through the C ABI; returns the full [Mpad, N] bf16 output."""
        import torch

        L = clib()
        if out is None:
            out = torch.empty(self.Mpad, self.N, dtype=torch.bfloat16, device=self.A.device)
        if config is None:
            ws = L.mbs_gemm_a4w4_workspace_bytes(self.M, self.N, self.K)
        else:
            ws = L.mbs_gemm_a4w4_config_workspace_bytes(config, splits, self.M, self.N, self.K)
        wst = torch.empty(max(ws, 1), dtype=torch.uint8, device=self.A.device)
        args = (ptr(self.A), ptr(self.B), ptr(self.As), ptr(self.Bs), ptr(self.Af), ptr(self.Bf),
                ptr(out), self.M, self.N, self.K, self.Mpad, self.snp, ptr(wst), ws, stream_ptr())
        if config is None:
            st = L.mbs_gemm_a4w4_launch(*args)
        else:
            st = L.mbs_gemm_a4w4_launch_config(config, splits, *args)
        if check:
            assert st == 0, (st, L.mbs_last_error())
        return out


def bf16_to_f32(t) -> np.ndarray:
    """bf16 torch tensor (any device) -> float32 numpy."""
    import torch

    return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16).astype(
        np.uint32).__lshift__(16).view(np.float32)


def assert_close(got: np.ndarray, ref: np.ndarray, what: str = "") -> float:
    """North-star tolerance; returns the worst |err| / bound ratio."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    nan_ref = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan_ref), f"{what}: NaN pattern differs"
    g, r = got[~nan_ref], ref[~nan_ref]
    if r.size == 0:
        return 0.0
    scale = np.max(np.abs(r[np.isfinite(r)])) if np.any(np.isfinite(r)) else 0.0
    with np.errstate(divide="ignore"):
        ulp = np.where(r != 0, 2.0 ** (np.floor(np.log2(np.abs(r) + (r == 0))) - 7), 2.0 ** -133)
    bound = 1e-2 * scale + ulp
    err = np.abs(g - r)
    inf = ~np.isfinite(r)
    assert np.array_equal(g[inf], r[inf]), f"{what}: inf mismatch"
    err, bound = err[~inf], bound[~inf]
    bad = err > bound
    assert not bad.any(), (f"{what}: {bad.sum()} elements out of tolerance; "
                           f"max err {err.max():.4g}, scale {scale:.4g}")
    return float((err / bound).max()) if err.size else 0.0
