"""CPU-side checks of the drop-in boundary: the C-ABI library loads and
exports every function include/mbs_gemm_a4w4.h declares; argument validation
returns the documented status codes without touching a GPU; the torch module
raises RuntimeError on bad operands (reference semantics,
interface/gemm_a4w4_pybind.cpp:22-44); plan selection is pure host logic."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "mbs_gemm_a4w4.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mbs_\w+)\s*\(", text)))


def test_header_symbols_exported():
    import mbs_amd

    lib = mbs_amd.clib()
    names = header_functions()
    assert "mbs_gemm_a4w4_launch" in names and len(names) >= 13
    for n in names:
        assert hasattr(lib, n), n


def c_lib():
    import mbs_amd

    L = mbs_amd.clib()
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.mbs_gemm_a4w4_launch.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, P, S, P]
    L.mbs_gemm_a4w4_launch.restype = I
    L.mbs_gemm_a4w4_launch_config.argtypes = [I, I, P, P, P, P, P, P, P, I, I, I, I, I, P, S, P]
    L.mbs_gemm_a4w4_launch_config.restype = I
    L.mbs_status_string.restype = ctypes.c_char_p
    L.mbs_last_error.restype = ctypes.c_char_p
    L.mbs_gemm_a4w4_plan_name.argtypes = [I, I, I, ctypes.c_char_p, S]
    L.mbs_gemm_a4w4_workspace_bytes.argtypes = [I, I, I]
    L.mbs_gemm_a4w4_workspace_bytes.restype = S
    L.mbs_gemm_a4w4_config_name.restype = ctypes.c_char_p
    return L


FAKE = 0x1000  # never dereferenced: validation fails first (or M == 0 returns early)


@pytest.mark.parametrize("M,N,K,Mpad,snp,why", [
    (-1, 256, 512, 0, 16, "M >= 0"),
    (0, 256, 512, 32, 16, "Mpad"),
    (128, 250, 512, 128, 16, "multiple of 16"),
    (128, 256, 480, 128, 16, "multiple of 64"),
    (128, 256, 512, 130, 16, "Mpad"),
    (128, 256, 512, 128, 17, "scaleN_pad"),
])
def test_launch_rejects_bad_shapes(M, N, K, Mpad, snp, why):
    L = c_lib()
    st = L.mbs_gemm_a4w4_launch(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, M, N, K, Mpad, snp,
                                None, 0, None)
    assert st == 1  # MBS_ERR_ARGUMENT
    assert why in L.mbs_last_error().decode()
    assert L.mbs_status_string(st) == b"invalid argument"


def test_empty_batch_is_a_validated_no_op():
    """M == 0: success without a launch (no GPU call is made), null A / out allowed;
    the other arguments are still checked."""
    L = c_lib()
    assert L.mbs_gemm_a4w4_launch(None, FAKE, None, FAKE, None, None, None, 0, 256, 512, 0, 16,
                                  None, 0, None) == 0
    assert L.mbs_gemm_a4w4_launch_config(0, 1, None, FAKE, None, FAKE, None, FAKE, None, 0, 256,
                                         512, 0, 16, None, 0, None) == 0
    # still validated: N, K, Mpad, B pointers and the config index
    assert L.mbs_gemm_a4w4_launch(None, FAKE, None, FAKE, None, None, None, 0, 250, 512, 0, 16,
                                  None, 0, None) == 1
    assert L.mbs_gemm_a4w4_launch(None, None, None, FAKE, None, None, None, 0, 256, 512, 0, 16,
                                  None, 0, None) == 1
    assert L.mbs_gemm_a4w4_launch_config(10**6, 1, None, FAKE, None, FAKE, None, None, None, 0,
                                         256, 512, 0, 16, None, 0, None) == 4
    # M > 0 still needs A and out
    assert L.mbs_gemm_a4w4_launch(None, FAKE, FAKE, FAKE, None, None, FAKE, 32, 256, 512, 32, 16,
                                  None, 0, None) == 1


def test_launch_rejects_null_and_half_factors():
    L = c_lib()
    assert L.mbs_gemm_a4w4_launch(None, FAKE, FAKE, FAKE, None, None, FAKE, 128, 256, 512, 128, 16,
                                  None, 0, None) == 1
    assert L.mbs_gemm_a4w4_launch(FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 128, 256, 512, 128, 16,
                                  None, 0, None) == 1
    assert b"together" in L.mbs_last_error()


@pytest.mark.parametrize("which,off,why", [
    ("A", 8, "16-byte"), ("B", 4, "16-byte"), ("As", 1, "16-byte"), ("Bs", 8, "16-byte"),
    ("out", 2, "16-byte"), ("Af", 2, "4-byte"), ("Bf", 1, "4-byte"),
])
def test_launch_rejects_misaligned_operands(which, off, why):
    """Every kernel moves A, B, the scales and the output in 16-byte units and
    the factor bytes in dwords: a misaligned base is refused before any GPU call."""
    L = c_lib()
    ptrs = dict(A=FAKE, B=FAKE, As=FAKE, Bs=FAKE, Af=FAKE, Bf=FAKE, out=FAKE)
    ptrs[which] += off
    st = L.mbs_gemm_a4w4_launch(ptrs["A"], ptrs["B"], ptrs["As"], ptrs["Bs"], ptrs["Af"], ptrs["Bf"],
                                ptrs["out"], 128, 256, 512, 128, 16, None, 0, None)
    assert st == 1
    assert why in L.mbs_last_error().decode()


def test_format_entry_points_reject_misaligned():
    L = c_lib()
    P, I = ctypes.c_void_p, ctypes.c_int
    L.mbs_shuffle_b.argtypes = [P, P, I, I, P]
    L.mbs_quantize_mxfp4_bf16.argtypes = [P, I, I, P, P, P, I, P]
    L.mbs_dequant_mxfp4.argtypes = [P, P, P, I, I, I, P]
    assert L.mbs_shuffle_b(FAKE + 4, FAKE + 4096, 32, 512, None) == 1
    assert L.mbs_quantize_mxfp4_bf16(FAKE + 2, 4, 64, FAKE, None, None, 127, None) == 1
    assert L.mbs_quantize_mxfp4_bf16(FAKE, 4, 64, FAKE + 1, None, None, 127, None) == 1
    assert L.mbs_dequant_mxfp4(FAKE, FAKE, FAKE + 8, 16, 64, 1, None) == 1
    assert b"aligned" in L.mbs_last_error()


def test_check_groups_validates_arguments():
    L = c_lib()
    P, I = ctypes.c_void_p, ctypes.c_int
    L.mbs_gemm_a4w4_check_groups.argtypes = [P, I, I, P, P]
    assert L.mbs_gemm_a4w4_check_groups(None, 2, 64, FAKE, None) == 1
    assert L.mbs_gemm_a4w4_check_groups(FAKE, 0, 64, FAKE, None) == 1
    assert L.mbs_gemm_a4w4_check_groups(FAKE, 2, -1, FAKE, None) == 1
    assert L.mbs_gemm_a4w4_check_groups(FAKE + 2, 2, 64, FAKE, None) == 1


def test_plans_cover_every_config_shape():
    from mbs_amd import synthetic

    L = c_lib()
    buf = ctypes.create_string_buffer(256)
    for cfg in range(5):
        for (M, N, K) in synthetic.config_shapes(cfg):
            assert L.mbs_gemm_a4w4_plan_name(M, N, K, buf, 256) == 0
            name = buf.value.decode()
            if M <= 32:
                assert name.startswith("skinny"), (M, N, K, name)
            else:
                assert name.startswith("bdirect"), (M, N, K, name)
    L.mbs_gemm_a4w4_plan_name(8192, 8192, 8192, buf, 256)
    assert "_256x256_" in buf.value.decode()
    assert L.mbs_gemm_a4w4_workspace_bytes(8192, 8192, 8192) == 0


def test_format_entry_points_validate():
    L = c_lib()
    P, I = ctypes.c_void_p, ctypes.c_int
    L.mbs_shuffle_b.argtypes = [P, P, I, I, P]
    L.mbs_quantize_mxfp4_bf16.argtypes = [P, I, I, P, P, P, I, P]
    L.mbs_dequant_mxfp4.argtypes = [P, P, P, I, I, I, P]
    assert L.mbs_shuffle_b(FAKE, FAKE + 64, 24, 512, None) == 1      # N % 16
    assert L.mbs_shuffle_b(FAKE, FAKE, 32, 512, None) == 1           # in place
    assert L.mbs_quantize_mxfp4_bf16(FAKE, 4, 48, FAKE, None, None, 127, None) == 1
    assert L.mbs_quantize_mxfp4_bf16(FAKE, 4, 64, FAKE, None, None, 300, None) == 1
    assert L.mbs_dequant_mxfp4(FAKE, FAKE, FAKE, 8, 64, 1, None) == 1  # rows % 16 for B


def test_torch_module_rejects_host_tensors_and_bad_shapes():
    import torch

    import mbs_amd

    m = mbs_amd.ext()
    A = torch.zeros(128, 256, dtype=torch.uint8)
    B = torch.zeros(256, 256, dtype=torch.uint8)
    s = torch.zeros(256 * 16, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="on device"):
        m.gemm_a4w4(A, B, s, s)
    with pytest.raises(RuntimeError, match="on device"):
        m.gemm_a4w4(A, B, s, s, torch.zeros(128, 1, dtype=torch.uint8), torch.zeros(256, 1, dtype=torch.uint8))
    with pytest.raises(RuntimeError):
        m.quantize_mxfp4(torch.zeros(4, 64, dtype=torch.bfloat16))
    assert m.num_configs() >= 8
    assert all(m.config_name(c).startswith(("bdirect", "skinny")) for c in range(m.num_configs()))
    assert "skinny" in m.plan_name(1, 8192, 8192)


def test_whole_k_tiles_refuse_k_tails_and_splits():
    """The 32x32x64-MFMA tiles (configs named *_m32) run whole-K (K % 512 == 0),
    single-split plans only: forced onto a K tail or K splits they return
    MBS_ERR_CONFIG before any launch."""
    L = c_lib()
    names = [L.mbs_gemm_a4w4_config_name(i).decode() for i in range(L.mbs_gemm_a4w4_num_configs())]
    m32 = [i for i, n in enumerate(names) if n.endswith("_m32")]
    assert len(m32) == 5
    for c in m32:
        for K, splits in [(448, 1), (1536 + 64, 1), (1024, 2), (2048, 3)]:
            snp = ((K // 32) + 7) // 8 * 8
            st = L.mbs_gemm_a4w4_launch_config(c, splits, FAKE, FAKE, FAKE, FAKE, None, None, FAKE,
                                               256, 256, K, 256, snp, None, 0, None)
            assert st == 4, (names[c], K, splits)
            assert b"cannot run" in L.mbs_last_error()


def test_grouped_whole_k_tiles_refuse_k_tails():
    """The grouped launch's 32x32x64-MFMA configurations refuse K % 512 != 0
    with MBS_ERR_CONFIG before any launch (the offsets are never read)."""
    L = c_lib()
    P, I = ctypes.c_void_p, ctypes.c_int
    L.mbs_gemm_a4w4_grouped_launch_ex.argtypes = [P, P, P, P, P, P, P, I, P, I, I, I, I, I,
                                                  ctypes.c_float, P, I, P]
    L.mbs_gemm_a4w4_grouped_launch_ex.restype = I
    L.mbs_gemm_a4w4_grouped_config_name.restype = ctypes.c_char_p
    names = [L.mbs_gemm_a4w4_grouped_config_name(i).decode()
             for i in range(L.mbs_gemm_a4w4_grouped_num_configs())]
    m32 = [i for i, n in enumerate(names) if n.endswith("_m32")]
    assert len(m32) == 2
    for c in m32:
        for K in (448, 1536 + 64, 1024 + 128):
            snp = ((K // 32) + 7) // 8 * 8
            st = L.mbs_gemm_a4w4_grouped_launch_ex(FAKE, FAKE, FAKE, FAKE, None, None, FAKE, 4, FAKE,
                                                   256, 256, K, 256, snp, 1.0, None, c, None)
            assert st == 4, (names[c], K)
            assert b"cannot run" in L.mbs_last_error()


def from_bf16_lib():
    L = c_lib()
    P, I, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    L.mbs_gemm_a4w4_from_bf16_launch.argtypes = [I, I, P, P, P, P, P, I, I, I, I, I,
                                                 ctypes.c_float, P, P, S, P]
    L.mbs_gemm_a4w4_from_bf16_launch.restype = I
    L.mbs_gemm_a4w4_from_bf16_workspace_bytes.argtypes = [I, I, I]
    L.mbs_gemm_a4w4_from_bf16_workspace_bytes.restype = S
    return L


def test_from_bf16_entry_validates_before_launch():
    """The bf16-activation decode entry: M > 32, a non-decode configuration,
    a misaligned or null activation, a NaN alpha and bad shapes return their
    status before any launch; M == 0 is a validated no-op."""
    L = from_bf16_lib()
    names = [L.mbs_gemm_a4w4_config_name(i).decode() for i in range(L.mbs_gemm_a4w4_num_configs())]
    skinny = [i for i, n in enumerate(names) if n.startswith("skinny")]
    other = [i for i, n in enumerate(names) if not n.startswith("skinny")]
    assert len(skinny) == 7 and other
    K, snp = 512, 16
    go = lambda cfg, x, M, N=256, K=K, Mpad=None, snp=snp, alpha=1.0, bf=None, splits=0: \
        L.mbs_gemm_a4w4_from_bf16_launch(
            cfg, splits, x, FAKE, FAKE, bf, FAKE, M, N, K,
            (M + 31) // 32 * 32 if Mpad is None else Mpad, snp, alpha, None, None, 0, None)
    assert go(-1, FAKE, 33) == 1 and b"M <= 32" in L.mbs_last_error()
    assert go(-1, None, 4) == 1 and b"null" in L.mbs_last_error()
    assert go(-1, FAKE + 8, 4) == 1 and b"aligned" in L.mbs_last_error()
    assert go(-1, FAKE, 4, alpha=float("nan")) == 1
    assert go(-1, FAKE, 4, N=250) == 1
    assert go(-1, FAKE, 4, K=480, snp=16) == 1
    assert go(-1, FAKE, 4, Mpad=64) == 1
    for c in other:
        assert go(c, FAKE, 4) == 4, names[c]
        assert b"not a decode" in L.mbs_last_error()
    assert go(len(names), FAKE, 4) == 4
    # a 16-row decode config cannot take 17 rows
    m16 = [i for i in skinny if "_m16_" in names[i]]
    assert m16 and all(go(c, FAKE, 17) == 4 for c in m16)
    assert go(-1, None, 0, Mpad=0) == 0   # empty batch: nothing launched
    # MBS activations (B factors given): M <= 8, aligned factors, 16-row
    # decode configurations without K splits
    assert go(-1, FAKE, 9, bf=FAKE) == 1 and b"M <= 8" in L.mbs_last_error()
    assert go(-1, FAKE, 4, bf=FAKE + 2) == 1 and b"aligned" in L.mbs_last_error()
    m32 = [i for i in skinny if "_m32_" in names[i]]
    assert m32 and all(go(c, FAKE, 4, bf=FAKE) == 4 for c in m32)
    assert all(go(c, FAKE, 4, bf=FAKE, splits=2) == 4 for c in m16)
    assert L.mbs_gemm_a4w4_from_bf16_workspace_bytes(33, 256, 512) == 0
    assert L.mbs_gemm_a4w4_from_bf16_workspace_bytes(1, 8192, 8192) == 0   # no split at this size


def test_from_bf16_plan_is_the_decode_plan():
    """For decode shapes whose heuristic plan is a skinny one, the
    bf16-activation entry's plan (skinny configurations only) is that same
    plan, so both paths give the same bytes."""
    L = from_bf16_lib()
    buf = ctypes.create_string_buffer(256)
    for M, N, K in [(1, 8192, 8192), (4, 8192, 8192), (16, 8192, 8192), (32, 8192, 8192),
                    (8, 4096, 4096), (32, 2112, 7168), (1, 256, 512)]:
        assert L.mbs_gemm_a4w4_plan_name(M, N, K, buf, 256) == 0
        plan = buf.value.decode()
        if plan.startswith("skinny"):
            assert (L.mbs_gemm_a4w4_from_bf16_workspace_bytes(M, N, K)
                    == L.mbs_gemm_a4w4_workspace_bytes(M, N, K)), (M, N, K, plan)


@pytest.mark.parametrize("passes", [1, 2])
def test_compact_bf16_lane_map_is_a_bijection(passes):
    """The compact one-launch decode form (gemm_skinny_kernel, XBF = 2/3):
    in pass q lane j quantizes block (row 4q + j/16, stage (j/4)%4, K-block
    j%4) of a 4-stage batch, and MFMA lane l of stage u reads pass (l%16)/4,
    lane 16*((l%16)%4) + 4u + l/16.  Every MFMA lane of a live row must read
    exactly the block its operand layout wants (row l%16, K-block l/16), and
    every quantized block is read exactly once."""
    produced = {}
    for q in range(passes):
        for j in range(64):
            produced[(q, j)] = (4 * q + j // 16, (j // 4) % 4, j % 4)   # (row, stage, kblock)
    seen = []
    for u in range(4):
        for lane in range(64):
            r = lane % 16
            if r >= 4 * passes:
                continue   # rows past the compact form's reach read zeros
            src = (r % 4) * 16 + 4 * u + lane // 16
            got = produced[(r // 4, src)]
            assert got == (r, u, lane // 16), (passes, u, lane, got)
            seen.append(got)
    assert sorted(seen) == sorted(produced.values())
