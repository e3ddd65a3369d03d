"""Cross-check against the reference's own kernel, built from its source into
oracle/_ref/libref_gemm.so (see oracle/Makefile; test infrastructure only).

The reference kernel and this repository's oracle are run on identical
bytes; agreement pins the oracle's reading of the preshuffled-B and
shuffled-scale layouts and of the MBS factor epilogue against the
reference implementation itself (kernel/gemm_a4w4.hip, launcher at
:1044-1146).  The reference kernel is driven only the way its own harness
drives it (test_gemm_a4w4.py:77-83): its workgroup path (K % 1024 == 0, large
tile count) always with factors -- with null factors that path would address
a null buffer -- and its single-wave path (small and decode shapes) without
factors, which it refuses (returns false) as documented at
kernel/gemm_a4w4.h:24-26.

Where both kernels consume the same bytes, this library's output is also
asserted to be the reference kernel's output bit for bit (torch.equal): both
accumulate the same scaled-MFMA partial products over K and apply the
factor product in the same order, so on these seeded operands every bf16
matches."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from gpu_util import Case, assert_close, bf16_to_f32, say

pytestmark = pytest.mark.gpu
REF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                   "libref_gemm.so")
SYM = "_Z22gemm_a4w4_mxfp4_launchPKhS0_S0_S0_S0_S0_PviiiiiS1_"


@pytest.fixture(scope="module")
def ref_launch():
    if not os.path.exists(REF):
        pytest.skip("reference kernel library not built (needs the reference tree at build time)")
    lib = ctypes.CDLL(REF)
    f = getattr(lib, SYM)
    P, I = ctypes.c_void_p, ctypes.c_int
    f.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, P]
    f.restype = ctypes.c_bool
    return f


def run_ref(f, c, factors):
    import torch

    out = torch.zeros(c.Mpad, c.N, dtype=torch.bfloat16, device=c.A.device)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ok = f(p(c.A), p(c.B), p(c.As), p(c.Bs), p(c.Af) if factors else None,
           p(c.Bf) if factors else None, p(out), c.M, c.N, c.K, c.Mpad, c.snp, s)
    torch.cuda.synchronize()
    return ok, out


def make(cfg, M, N, K, factors):
    from mbs_amd import synthetic

    x, w = synthetic.make_operands(cfg, M, N, K)
    f = None
    if factors:
        af, bf = synthetic.make_factors(M, N, 4000 + cfg)
        f = (af.numpy().reshape(-1), bf.numpy().reshape(-1))
    return Case.from_bf16(x, w, factors=f)


def test_single_wave_path_cfg0(dev, ref_launch):
    import torch

    c = make(0, 128, 256, 512, factors=True)
    say("reference kernel cfg0 with factors (single-wave path refuses)")
    ok, _ = run_ref(ref_launch, c, factors=True)
    assert ok is False
    say("reference kernel cfg0 without factors")
    ok, out = run_ref(ref_launch, c, factors=False)
    assert ok is True
    c.a_factor = c.b_factor = None
    c.Af = c.Bf = None
    ref = oracle.bf16_bits_to_f32(c.reference())
    got_ref = bf16_to_f32(out)[: c.M]
    assert_close(got_ref, ref, "reference kernel vs oracle")
    ours_t = c.run()[: c.M]
    ours = bf16_to_f32(ours_t)
    assert_close(ours, ref, "ours vs oracle")
    assert torch.equal(ours_t, out[: c.M]), "ours vs reference kernel: not bit-identical"


@pytest.mark.parametrize("M", [1, 16])
def test_single_wave_path_decode(dev, ref_launch, M):
    import torch

    c = make(2, M, 8192, 8192, factors=False)
    say(f"reference kernel decode M={M}")
    ok, out = run_ref(ref_launch, c, factors=False)
    assert ok is True
    ref = oracle.bf16_bits_to_f32(c.reference())
    got_ref = bf16_to_f32(out)[: c.M]
    assert_close(got_ref, ref, "reference kernel vs oracle")
    ours_t = c.run()[: c.M]
    assert_close(bf16_to_f32(ours_t), got_ref, "ours vs reference kernel")
    assert torch.equal(ours_t, out[: c.M]), "ours vs reference kernel: not bit-identical"


def test_workgroup_path_cfg1_with_factors(dev, ref_launch):
    import torch

    c = make(1, 8192, 8192, 8192, factors=True)
    say("reference kernel cfg1 8192^3 with factors (workgroup path)")
    ok, out = run_ref(ref_launch, c, factors=True)
    assert ok is True
    got_ref = bf16_to_f32(out)[: c.M]
    rows = np.array(sorted({0, 1, 31, 255, 256, 4095, 4096, 8190, 8191} |
                           set(np.random.default_rng(0).integers(0, 8192, 24).tolist())))
    ref_rows = oracle.bf16_bits_to_f32(c.reference(rows))
    assert_close(got_ref[rows], ref_rows, "reference kernel vs oracle (rows)")
    ours_t = c.run()[: c.M]
    ours = bf16_to_f32(ours_t)
    assert_close(ours[rows], ref_rows, "ours vs oracle (rows)")
    assert torch.equal(ours_t, out[: c.M]), "ours vs reference kernel: not bit-identical"
