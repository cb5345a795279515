"""Build the native parts in-tree.

* ``tcc_amd/libtcc_swtcf.so`` — the HIP kernels for gfx950 and the C-ABI
  (``include/tcc_swtcf.h``, ``include/tcc_spmm_cnic.h``), no torch dependency.
* ``tcc_amd/spmm_cnic*.so`` — the ``spmm_cnic`` PyTorch extension (pybind11,
  C++), a thin layer over the C-ABI (see ``csrc/spmm_cnic_ext.cpp``).

Run ``python -m tcc_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(ROOT, "_build", "tcc_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("TCC_OFFLOAD_ARCH", "gfx950")

LIB_SOURCES = ["swtcf_convert.hip", "swtcf_spmm.hip", "swtcf_plan.hip", "bcsr_spmm.hip", "bcsr_build.hip",
               "hub_tiles.hip", "dense_tn.hip",
               "errors.cpp"]
LIB_NAME = "libtcc_swtcf.so"

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
# -munsafe-fp-atomics: hardware global_atomic_add_f32 instead of CAS loops.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]

# Per-source device flags.  hub_tiles.hip: MFMA accumulators in arch VGPRs.
# In the default AGPR form the register allocator gives most MFMAs of the
# split tile kernel a destination other than their accumulator and copies the
# accumulators around the loop (~150 v_accvgpr moves per 128 MFMAs, 392
# registers); in the VGPR form every MFMA accumulates in place, with no
# copies, in 244 registers.
SOURCE_FLAGS = {
    "hub_tiles.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build_library(jobs: int = 8) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs = []

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        path = os.path.join(CSRC, src)
        if src.endswith(".hip"):
            cmd = [HIPCC, "-x", "hip", *DEVICE_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", path, "-o", obj]
        else:
            cmd = [HIPCC, "-O3", "-std=c++17", "-fPIC", "-Wall", "-c", path, "-o", obj]
        _run(cmd)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, LIB_SOURCES))
    out = os.path.join(PKG, LIB_NAME)
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_extension() -> str:
    """Compile the spmm_cnic pybind11 module against libtcc_swtcf.so."""
    import pybind11
    import torch.utils.cpp_extension as cpp

    os.makedirs(BUILD, exist_ok=True)
    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "spmm_cnic" + suffix)
    tmp = out + ".tmp"
    torch_lib = os.path.join(os.path.dirname(cpp.__file__), "..", "lib")
    torch_lib = os.path.abspath(torch_lib)
    inc = [f"-I{p}" for p in cpp.include_paths()] + [
        f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}",
        f"-I{os.path.join(ROOT, 'include')}", "-I/opt/rocm/include",
    ]
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
        "-DTORCH_EXTENSION_NAME=spmm_cnic", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D_GLIBCXX_USE_CXX11_ABI=1", *inc,
        os.path.join(CSRC, "spmm_cnic_ext.cpp"), "-o", tmp,
        f"-L{PKG}", "-ltcc_swtcf", f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu",
        "-ltorch_python", "-lc10_hip", "-ltorch_hip", "-L/opt/rocm/lib", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}", "-Wl,-rpath,/opt/rocm/lib",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


CLI_SOURCES = ["swtcf_convert_run.cpp", "swtcf_spmm_run.cpp"]


def build_cli() -> list:
    """The command-line drivers (tcc_amd/bin/swtcf_convert_run, swtcf_spmm_run):
    host C++ over include/tcc_swtcf.hpp, linked against libtcc_swtcf.so."""
    bindir = os.path.join(PKG, "bin")
    os.makedirs(bindir, exist_ok=True)
    outs = []
    for src in CLI_SOURCES:
        out = os.path.join(bindir, os.path.splitext(src)[0])
        tmp = out + ".tmp"
        _run(["g++", "-O2", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__=1", f"-I{os.path.join(ROOT, 'include')}",
              "-I/opt/rocm/include", os.path.join(PKG, "cli", src), "-o", tmp, f"-L{PKG}", "-ltcc_swtcf",
              "-Wl,-rpath,$ORIGIN/..", "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"])
        os.replace(tmp, out)
        outs.append(out)
    return outs


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    print("building", build_library(), flush=True)
    for out in build_cli():
        print("building", out, flush=True)
    if "--no-ext" not in argv:
        print("building", build_extension(), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
