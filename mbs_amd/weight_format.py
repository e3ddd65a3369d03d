"""Offline weight format: MXFP4 weights as the GEMM consumes them, on disk.

The reference prepares weights at load time with aiter
(``test_gemm_a4w4.py:134-141``: per-1x32 quantization, scale shuffle,
``shuffle_weight(w, layout=(16,16))``) and keeps no on-disk form.  Here the
prepared operand is a file that can be written once and mapped straight into
the GEMM:

* ``weight``        u8 [N, K/2]   e2m1 pairs, (16,16)-preshuffled (``B``)
* ``weight_scale``  u8 [round_up(N,32), scaleN_pad]  shuffled E8M0 (``B_scale``)
* ``weight_factor`` u8 [N]        MBS factor bytes (only for MBS weights)

stored with safetensors (no code runs on load) and metadata ``format``,
``N``, ``K``, ``scale_pad_byte``.  ``unpack_weight`` undoes both shuffles,
``validate_weight`` checks shapes, sizes, the scale padding and NaN scale
bytes on the device.  All conversions run on the GPU through the C ABI;
there is no CPU path.
"""
from __future__ import annotations

import os

FORMAT = "mbs-mxfp4-a4w4-preshuffle16x16-v1"


def _mod():
    from . import ext

    return ext()


def _scale_pad(K: int) -> int:
    return ((K + 31) // 32 + 7) // 8 * 8


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


def prepare_weight(w, mbs: bool = False, pad_byte: int = 127) -> dict:
    """bf16 weights [N, K] on the device -> the GEMM's B operand.

    Returns ``{"weight", "weight_scale", "weight_factor" (MBS only), "N", "K",
    "scale_pad_byte"}``."""
    import torch

    if not (isinstance(w, torch.Tensor) and w.is_cuda and w.dim() == 2 and w.dtype == torch.bfloat16):
        raise TypeError("prepare_weight: w must be a 2D bf16 device tensor")
    N, K = w.shape
    if N % 16 or K % 64:
        raise ValueError(f"prepare_weight: need N % 16 == 0 and K % 64 == 0, got N={N} K={K}")
    m = _mod()
    out = {"N": int(N), "K": int(K), "scale_pad_byte": int(pad_byte)}
    if mbs:
        packed, scale, factor = m.quantize_mxfp4_mbs(w, True, pad_byte)
        out["weight_factor"] = factor
    else:
        packed, scale = m.quantize_mxfp4(w, True, pad_byte)
    out["weight"] = m.shuffle_weight(packed)
    out["weight_scale"] = scale
    return out


def validate_weight(weight, weight_scale, N: int, K: int, weight_factor=None,
                    pad_byte: int | None = 127) -> None:
    """Raise ``ValueError`` listing every way the operand breaks the format.

    Checks dtype, device, shapes, the scale buffer size, the scale padding
    bytes (skipped for ``pad_byte=None``) and E8M0 NaN bytes (0xFF) among the
    live scales, which would make whole blocks of the product NaN."""
    import torch

    problems = []
    for name, t in (("weight", weight), ("weight_scale", weight_scale)):
        if not isinstance(t, torch.Tensor) or t.element_size() != 1:
            problems.append(f"{name}: not a 1-byte tensor")
        elif not t.is_cuda:
            problems.append(f"{name}: not on a GPU")
    if N < 16 or N % 16 or K < 64 or K % 64:
        problems.append(f"N={N}, K={K}: need N % 16 == 0 and K % 64 == 0")
    if problems:
        raise ValueError("; ".join(problems))
    if tuple(weight.shape) != (N, K // 2):
        problems.append(f"weight: shape {tuple(weight.shape)}, expected {(N, K // 2)}")
    need = _round_up(N, 32) * _scale_pad(K)
    if weight_scale.numel() < need:
        problems.append(f"weight_scale: {weight_scale.numel()} bytes, need {need}")
    if weight_factor is not None:
        if not (isinstance(weight_factor, torch.Tensor) and weight_factor.is_cuda
                and weight_factor.element_size() == 1 and weight_factor.numel() == N):
            problems.append(f"weight_factor: need {N} bytes on the GPU")
    if problems:
        raise ValueError("; ".join(problems))
    bad_pad, nan_live = _mod().check_scales(weight_scale, N, K, -1 if pad_byte is None else pad_byte)
    if bad_pad:
        problems.append(f"weight_scale: {bad_pad} padding bytes differ from {pad_byte:#04x}")
    if nan_live:
        problems.append(f"weight_scale: {nan_live} live scale bytes are 0xFF (E8M0 NaN)")
    if problems:
        raise ValueError("; ".join(problems))


def unpack_weight(weight, weight_scale, N: int, K: int):
    """Undo both shuffles: -> (plain packed [N, K/2], plain E8M0 [N, K/32])."""
    m = _mod()
    return m.unshuffle_weight(weight), m.unshuffle_scales(weight_scale, N, K)


def save_weight(path: str | os.PathLike, weight, weight_scale, N: int, K: int,
                weight_factor=None, pad_byte: int = 127, validate: bool = True) -> None:
    """Write the operand to a safetensors file (tensors copied to the host)."""
    from safetensors.torch import save_file

    if validate:
        validate_weight(weight, weight_scale, N, K, weight_factor, pad_byte)
    tensors = {
        "weight": weight.detach().reshape(N, K // 2).cpu().contiguous(),
        "weight_scale": weight_scale.detach().reshape(_round_up(N, 32), _scale_pad(K)).cpu().contiguous(),
    }
    if weight_factor is not None:
        tensors["weight_factor"] = weight_factor.detach().reshape(N).cpu().contiguous()
    meta = {"format": FORMAT, "N": str(N), "K": str(K), "scale_pad_byte": str(pad_byte)}
    save_file(tensors, os.fspath(path), metadata=meta)


def read_weight_file(path: str | os.PathLike) -> dict:
    """Read a weight file into host tensors and its metadata (no validation)."""
    from safetensors import safe_open

    with safe_open(os.fspath(path), framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path}: format {meta.get('format')!r}, expected {FORMAT!r}")
        out = {k: f.get_tensor(k) for k in f.keys()}
    out["N"], out["K"] = int(meta["N"]), int(meta["K"])
    out["scale_pad_byte"] = int(meta["scale_pad_byte"])
    return out


def load_weight(path: str | os.PathLike, device="cuda", validate: bool = True) -> dict:
    """Read a weight file onto ``device`` and (by default) validate it."""
    w = read_weight_file(path)
    for k in ("weight", "weight_scale", "weight_factor"):
        if k in w:
            w[k] = w[k].to(device)
    if validate:
        validate_weight(w["weight"], w["weight_scale"], w["N"], w["K"], w.get("weight_factor"),
                        w["scale_pad_byte"])
    return w
