"""Build the gfx950 libraries in-tree.

Products (under ``mbs_amd/lib/``):

* ``libmbs_gemm_kernel.so`` -- the torch-free HIP library with the C ABI of
  ``include/mbs_gemm_a4w4.h`` (GEMM + format kernels), built with hipcc for
  gfx950 only.
* ``libmbs_probe.so`` -- a measurement tool: the streaming-read floor of a
  decode GEMM (``include/mbs_probe.h``).
* ``mbs_gemm_a4w4<EXT_SUFFIX>.so`` -- the torch/pybind11 module that is the
  drop-in for the reference's ``mbs_gemm_a4w4`` extension; host-only C++
  (built with g++), linked against the library above with an ``$ORIGIN``
  rpath so the pair travels together.

Run ``python -m mbs_amd._build`` (or ``__graft_entry__.build()``).  Every call
rebuilds.  ``python -m mbs_amd._build --phase-timer`` builds
``libmbs_gemm_phase.so`` instead: the same kernels with the in-kernel phase
timer (``MBS_PHASE_TIMER=1``, ``include/mbs_phase_timer.h``), a measurement
tool.  ``--incremental`` keeps object files newer than every source and
header (development builds; ``build()`` always rebuilds everything).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# The GEMM kernel families are instantiated in separate translation units
# (gemm_inst_*.hip) so that they compile in parallel.
HIP_SOURCES = [
    "gemm_inst_bdirect_c.hip", "gemm_inst_bdirect_d.hip", "gemm_inst_bdirect_e.hip", "gemm_inst_bdirect_a.hip",
    "gemm_inst_bdirect_b.hip", "gemm_inst_grouped.hip", "gemm_inst_grouped_m.hip",
    "gemm_inst_skinny.hip",
    "gemm_a4w4.hip", "mxfp4_format.hip",
]
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed-fp32 VALU ops are kept out of the generated code on purpose
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-warning-option",
    f"-I{INCLUDE}", f"-I{CSRC}",
]

KERNEL_LIB = os.path.join(LIB, "libmbs_gemm_kernel.so")
# Measurement tool beside the GEMM library: the streaming-read floor of a
# decode GEMM (include/mbs_probe.h; bench.py loads it).
PROBE_LIB = os.path.join(LIB, "libmbs_probe.so")
# The same kernels with the in-kernel phase timer compiled in (a measurement
# tool: bench.py --phase-split and the sclk figure of the bench line).
PHASE_LIB = os.path.join(LIB, "libmbs_gemm_phase.so")
MODULE = os.path.join(LIB, "mbs_gemm_a4w4" + sysconfig.get_config_var("EXT_SUFFIX"))


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {os.path.basename(cmd[0])} -> {cmd[-1]}")


def _newest_input(src: str) -> float:
    heads = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    heads += [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    return max(os.path.getmtime(p) for p in [os.path.join(CSRC, src), *heads])


INCREMENTAL = False   # --incremental: keep objects newer than every source and header


def _hip_object(src: str, phase_timer: bool = False) -> str:
    sub = "_obj_phase" if phase_timer else "_obj"
    obj = os.path.join(LIB, sub, os.path.splitext(src)[0] + ".o")
    os.makedirs(os.path.dirname(obj), exist_ok=True)
    if INCREMENTAL and os.path.exists(obj) and os.path.getmtime(obj) > _newest_input(src):
        return obj
    extra = ["-DMBS_PHASE_TIMER=1"] if phase_timer else []
    _run([HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_kernel_lib(phase_timer: bool = False) -> str:
    """The C-ABI library; with phase_timer, its timer build (PHASE_LIB)."""
    os.makedirs(LIB, exist_ok=True)
    out = PHASE_LIB if phase_timer else KERNEL_LIB
    workers = max(1, min(len(HIP_SOURCES), os.cpu_count() or 1, 16))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda src: _hip_object(src, phase_timer), HIP_SOURCES))
    tmp = out + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_probe_lib() -> str:
    os.makedirs(LIB, exist_ok=True)
    _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, "stream_probe.hip"), "-o", PROBE_LIB + ".tmp"])
    os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    return PROBE_LIB


def build_module() -> str:
    import torch
    import torch.utils.cpp_extension as ce

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    py_inc = sysconfig.get_paths()["include"]
    import pybind11

    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=mbs_gemm_a4w4", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        *[f"-I{p}" for p in ce.include_paths()],
        f"-I{pybind11.get_include()}", f"-I{py_inc}", f"-I{ROCM}/include", f"-I{INCLUDE}",
        os.path.join(CSRC, "gemm_a4w4_pybind.cpp"),
        f"-L{LIB}", "-lmbs_gemm_kernel", "-Wl,-rpath,$ORIGIN",
        f"-L{torch_lib}", f"-Wl,-rpath,{torch_lib}",
        "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10", "-lc10_hip", "-ltorch_hip",
        f"-L{ROCM}/lib", "-lamdhip64",
        "-o", MODULE + ".tmp",
    ]
    _run(cmd)
    os.replace(MODULE + ".tmp", MODULE)
    return MODULE


def build_oracle() -> None:
    """TEST INFRASTRUCTURE: the CPU oracle (and the reference build under
    oracle/_ref when the reference tree is mounted) -- the checkers, not the
    product."""
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle")])
    if os.path.isdir("/root/reference/kernel"):
        _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref"])


def build_all(with_oracle: bool = True) -> None:
    build_kernel_lib()
    build_module()
    build_probe_lib()
    if with_oracle:
        build_oracle()


if __name__ == "__main__":
    INCREMENTAL = "--incremental" in sys.argv[1:]
    if "--phase-timer" in sys.argv[1:]:
        print("built", build_kernel_lib(phase_timer=True))
    else:
        build_all()
        print("built", KERNEL_LIB, MODULE)
