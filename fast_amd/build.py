"""In-tree build of the gfx950 kernel library and the ``fastAgg`` torch binding.

Outputs (git-ignored, shipped with the tree):
  fast_amd/lib/libfastagg_hip.so                   C ABI of include/fastagg.h (hipcc, gfx950)
  fast_amd/fastAgg<EXT_SUFFIX>                     pybind11 torch extension over that ABI

The kernels are compiled for gfx950 only, with packed-FP32 instruction selection turned off.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(PKG, "_build")

HIP_SOURCES = ["capi.hip", "bookkeeping.hip", "softmax.hip", "aggregate.hip", "fused_attn.hip",
               "tgat_attn.hip", "epilogue.hip", "head_gemm.hip", "layer_params.hip", "memory.hip"]
ARCH = "gfx950"
LIB_NAME = "libfastagg_hip.so"
EXT_NAME = "fastAgg"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the ROCm toolchain is required to build fast_amd")


HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n"
                           f"{res.stdout}\n{res.stderr}")
    noisy = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if verbose and noisy:
        print("\n".join(noisy), flush=True)


def lib_path() -> str:
    return os.path.join(LIBDIR, LIB_NAME)


def ext_path() -> str:
    return os.path.join(PKG, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_hip_library(verbose: bool = False, jobs: int = 8) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(OBJDIR, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([cc, *HIP_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, src),
                     "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    out = lib_path()
    tmp = out + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


def build_torch_extension(verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension

    tinc = cpp_extension.include_paths()
    tlib = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    pyinc = sysconfig.get_paths()["include"]
    out = ext_path()
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *[f"-I{p}" for p in tinc], f"-I{pyinc}", "-I/opt/rocm/include", f"-I{INCLUDE}",
           os.path.join(CSRC, "fastagg_torch.cpp"),
           *[f"-L{p}" for p in tlib], f"-L{LIBDIR}",
           "-lfastagg_hip", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-ltorch_python",
           "-Wl,-rpath,$ORIGIN/lib", *[f"-Wl,-rpath,{p}" for p in tlib],
           "-o", tmp]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    build_hip_library(verbose=verbose)
    build_torch_extension(verbose=verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", lib_path(), ext_path())
