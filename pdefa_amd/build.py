"""Builds pdefa_amd/lib/libpdefa_native.so (HIP kernels + C++ runtime + C ABI)
for gfx950 with hipcc, in-tree.

    python -m pdefa_amd.build            # or: python pdefa_amd/build.py
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libpdefa_native.so")
ARCH = os.environ.get("PDEFA_OFFLOAD_ARCH", "gfx950")

SOURCES = [
    "kernels/conv_mfma.hip",
    "kernels/conv_mfma_tiles_a.hip",
    "kernels/conv_mfma_tiles_b.hip",
    "kernels/conv_mfma_tiles_c.hip",
    "kernels/conv_mfma_tiles_d.hip",
    "kernels/conv_mfma_tiles_e.hip",
    "kernels/conv_wino.hip",
    "kernels/conv_wino_strip.hip",
    "kernels/ops.hip",
    "kernels/yolo_decode.hip",
    "kernels/noalloc.hip",
    "model.cpp",
    "planner.cpp",
    "runtime.cpp",
    "conv_tune.cpp",
    "engine_api.cpp",
    "host_ops.cpp",
    "pdefa_api.cpp",
]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
          "-I" + os.path.join(ROOT, "include")]
# Device code is compiled without packed-fp32 instruction selection.
DEVICE = ["--offload-arch=" + ARCH, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def rocm() -> str:
    return os.environ.get("ROCM_PATH", "/opt/rocm")


def host_cxx() -> str:
    c = os.path.join(rocm(), "lib", "llvm", "bin", "clang++")
    return c if os.path.exists(c) else "g++"


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src.replace("/", "_") + ".o")
    if src.endswith(".hip"):
        cmd = [hipcc()] + COMMON + DEVICE + ["-x", "hip"]
    else:
        # host-only translation units: plain C++ against the HIP runtime headers
        cmd = [host_cxx(), "-x", "c++"] + COMMON + ["-D__HIP_PLATFORM_AMD__",
                                                    "-I" + os.path.join(rocm(), "include")]
    cmd += ["-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    jobs = min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs + [
        "-Wl,--no-undefined", "-Wl,-soname,libpdefa_native.so"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
