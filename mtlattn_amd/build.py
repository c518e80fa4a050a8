"""Build the gfx950 kernels and the torch binding in-tree.

    python -m mtlattn_amd.build            # or __graft_entry__.build()

Produces, next to this file:
  * libmtlattn_hip.so   -- the C-ABI library (include/mtlattn_capi.h), built
                           by hipcc from csrc/*.hip for --offload-arch=gfx950;
  * _C<EXT_SUFFIX>      -- the pybind11 torch extension (csrc/torch_ext.cpp),
                           built by g++ against torch's headers and linked to
                           libmtlattn_hip.so through an $ORIGIN rpath;
  * libmtlattn_calib.so -- measured-ceiling kernels (csrc/calib.hip) that
                           bench.py divides by; not part of the C ABI.
Object files go to _build/ (git-ignored). Always recompiles.
"""

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmtlattn_hip.so")
EXT = os.path.join(HERE, "_C" + sysconfig.get_config_var("EXT_SUFFIX"))
CALIB = os.path.join(HERE, "libmtlattn_calib.so")
HIP_SOURCES = ["fwd.hip", "bwd.hip", "bwd_wide.hip", "decode.hip", "generic.hip", "f32mfma.hip", "pad.hip", "capi.hip"]
# Per-source flags. bwd_wide.hip pins its accumulators to the AGPRs by inline
# asm and needs the compiler's own MFMA results in VGPRs, where the VALU reads
# them.
SOURCE_FLAGS = {"bwd_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = os.environ.get("MTLATTN_ARCH", "gfx950")
# Packed fp32 VALU ops are disabled for all device code.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build_lib(verbose=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(HIP_SOURCES), max(1, (os.cpu_count() or 2) // 2))

    def compile_one(src):
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        _run([HIPCC, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj], verbose)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


def build_ext(verbose=False):
    import torch
    from torch.utils import cpp_extension

    incs = cpp_extension.include_paths()
    libdirs = cpp_extension.library_paths()
    py_inc = sysconfig.get_paths()["include"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    obj = os.path.join(BUILD, "torch_ext.o")
    os.makedirs(BUILD, exist_ok=True)
    cflags = ["-O2", "-std=c++17", "-fPIC", "-w", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
              "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
              "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              *[f"-I{d}" for d in incs], f"-I{py_inc}", f"-I{ROCM}/include"]
    _run(["g++", *cflags, "-c", os.path.join(CSRC, "torch_ext.cpp"), "-o", obj], verbose)
    tmp = EXT + ".tmp"
    _run(["g++", "-shared", obj, "-o", tmp, f"-L{HERE}", "-lmtlattn_hip", "-Wl,-rpath,$ORIGIN",
          *[f"-L{d}" for d in libdirs], *[f"-Wl,-rpath,{d}" for d in libdirs],
          "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip"], verbose)
    os.replace(tmp, EXT)
    return EXT


def build_calib(verbose=False):
    tmp = CALIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(CSRC, "calib.hip"), "-o", tmp], verbose)
    os.replace(tmp, CALIB)
    return CALIB


def build(verbose=False):
    build_lib(verbose)
    build_ext(verbose)
    build_calib(verbose)
    return LIB, EXT, CALIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
