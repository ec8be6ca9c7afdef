"""In-tree build of the native parts of mi355x_sampler.

  libmxs_sampler.so   HIP kernels + C ABI (include/mxs_sampler.h), hipcc for gfx950
  _mxs_ext*.so        thin torch extension over that C ABI (g++ against torch headers)

Both land in mi355x_sampler/_lib/.  Each kernel instance (csrc/k_*.hip) and
the C-ABI file compile as separate objects, in parallel, into _build/, and
are then linked into the library.  Run `python llm-inference-scheduler_amd/build.py`
or call build() (which __graft_entry__.build() does).
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIBDIR = os.path.join(PKG_ROOT, "mi355x_sampler", "_lib")
OBJDIR = os.path.join(PKG_ROOT, "_build")
LIB = os.path.join(LIBDIR, "libmxs_sampler.so")
EXT = os.path.join(LIBDIR, "_mxs_ext" + sysconfig.get_config_var("EXT_SUFFIX"))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

# -ffp-contract=off: the kernels' only fused multiply-adds are explicit fmaf
# calls, matching the CPU oracle bit for bit; IEEE division stays the default.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", f"-I{INCLUDE}", f"-I{CSRC}",
]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(os.path.basename(src))[0] + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    return obj


def build_library() -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def build_extension() -> str:
    import torch
    from torch.utils import cpp_extension

    os.makedirs(LIBDIR, exist_ok=True)
    inc = cpp_extension.include_paths()
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    py_inc = sysconfig.get_paths()["include"]
    tmp = EXT + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-DTORCH_EXTENSION_NAME=_mxs_ext", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-I{INCLUDE}", f"-I{ROCM}/include", *[f"-isystem{p}" for p in inc], f"-isystem{py_inc}",
           os.path.join(CSRC, "sampler_ext.cpp"), "-o", tmp,
           f"-L{LIBDIR}", "-lmxs_sampler", "-Wl,-rpath,$ORIGIN",
           f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-ltorch_python"]
    _run(cmd)
    os.replace(tmp, EXT)
    return EXT


def build() -> None:
    build_library()
    build_extension()


if __name__ == "__main__":
    build()
    sys.exit(0)
