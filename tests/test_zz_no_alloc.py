"""The allocation-free entry point mbs_gemm_a4w4_launch_noalloc, through the
C ABI: its split-K partials live in the library's static device scratch, so
it must give the bytes of mbs_gemm_a4w4_launch_ex with a caller workspace
on the same plan (same kernels, same fixed reduction order), call after
call -- here a large call followed by smaller ones, which reuse the scratch
the previous call left behind -- and it must refuse a forced split count
whose partials do not fit the scratch."""
import ctypes

import numpy as np
import pytest

import oracle
from gpu_util import Case, assert_close, bf16_to_f32, clib, ptr, say, stream_ptr

FAKE = 0x1000          # never dereferenced: the call is refused before any GPU work
SCRATCH = 32 << 20     # MBS_NOALLOC_SCRATCH_BYTES


def lib():
    L = clib()
    P, I, S, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
    L.mbs_gemm_a4w4_launch_noalloc.argtypes = [I, I, P, P, P, P, P, P, P, I, I, I, I, I, F, P, P]
    L.mbs_gemm_a4w4_launch_noalloc.restype = I
    L.mbs_gemm_a4w4_launch_ex.argtypes = [I, I, P, P, P, P, P, P, P, I, I, I, I, I, F, P, P, S, P]
    L.mbs_gemm_a4w4_launch_ex.restype = I
    L.mbs_gemm_a4w4_config_workspace_bytes.argtypes = [I, I, I, I, I]
    L.mbs_gemm_a4w4_config_workspace_bytes.restype = S
    return L


def config_index(name):
    import mbs_amd

    m = mbs_amd.ext()
    return [m.config_name(c) for c in range(m.num_configs())].index(name)


def test_noalloc_refuses_partials_beyond_scratch():
    L = lib()
    cfg = config_index("bdirect_128x256_w1x4")
    M, N, K = 2048, 4096, 8192
    assert L.mbs_gemm_a4w4_config_workspace_bytes(cfg, 8, M, N, K) > SCRATCH
    st = L.mbs_gemm_a4w4_launch_noalloc(cfg, 8, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, M, N, K,
                                        M, oracle.scale_pad(K), 1.0, None, None)
    assert st == 2  # MBS_ERR_WORKSPACE
    assert b"scratch" in L.mbs_last_error()


def _case(seed, M, N, K, factors):
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    rng = np.random.default_rng(seed)
    f = (rng.integers(0, 256, M, dtype=np.uint8), rng.integers(0, 256, N, dtype=np.uint8)) if factors else None
    return Case.from_bf16(x, w, factors=f)


@pytest.mark.gpu
def test_noalloc_matches_workspace_launch(dev):
    import torch

    L = lib()
    # (M, N, K, config name or None for the heuristic, splits, factors, alpha, bias):
    # a large call, then smaller ones that reuse the scratch it left behind
    steps = [
        (64, 8192, 8192, None, 0, True, 1.0, False),                     # heuristic: 64x64, 4 splits (8 MiB)
        (200, 1024, 4096, "bdirect_64x128_w1x2", 4, False, 0.5, True),   # forced persistent split
        (16, 4096, 4096, "skinny_m16_n32_w8", 4, True, 1.0, False),      # forced decode split
        (40, 512, 2048, "bdirect_64x128_w1x2", 2, True, -2.0, True),     # smaller again
    ]
    for i, (M, N, K, name, splits, factors, alpha, with_bias) in enumerate(steps):
        cfg = -1 if name is None else config_index(name)
        say(f"noalloc step {i}: M={M} N={N} K={K} config={name} splits={splits} factors={factors}")
        c = _case(500 + i, M, N, K, factors)
        bias = None
        if with_bias:
            bias = (torch.randn(N, generator=torch.Generator().manual_seed(i)) * 3).to(torch.bfloat16).to(dev)
        ws = (L.mbs_gemm_a4w4_config_workspace_bytes(cfg, splits, M, N, K) if cfg >= 0
              else clib().mbs_gemm_a4w4_workspace_bytes(M, N, K))
        assert 0 < ws <= SCRATCH, ws   # every step runs a split plan
        wst = torch.empty(ws, dtype=torch.uint8, device=dev)
        want = torch.empty(c.Mpad, N, dtype=torch.bfloat16, device=dev)
        got = torch.empty(c.Mpad, N, dtype=torch.bfloat16, device=dev)
        common = (ptr(c.A), ptr(c.B), ptr(c.As), ptr(c.Bs), ptr(c.Af), ptr(c.Bf))
        st = L.mbs_gemm_a4w4_launch_ex(cfg, splits, *common, ptr(want), M, N, K, c.Mpad, c.snp,
                                       alpha, ptr(bias), ptr(wst), ws, stream_ptr())
        assert st == 0, L.mbs_last_error()
        st = L.mbs_gemm_a4w4_launch_noalloc(cfg, splits, *common, ptr(got), M, N, K, c.Mpad, c.snp,
                                            alpha, ptr(bias), stream_ptr())
        assert st == 0, L.mbs_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got[:M], want[:M]), i
        if alpha == 1.0 and bias is None:
            rows = np.unique(np.linspace(0, M - 1, min(M, 8)).astype(int))
            assert_close(bf16_to_f32(got[torch.from_numpy(rows).to(dev)]),
                         oracle.bf16_bits_to_f32(c.reference(rows)), f"step {i}")
