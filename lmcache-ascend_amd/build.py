"""Builds liblmcache_amd.so (the gfx950 kernels plus the C ABI) in-tree.

    python lmcache-ascend_amd/build.py [--jobs N]

Each source under csrc/ is compiled by hipcc for gfx950 into _build/, then
linked into lmcache_amd/liblmcache_amd.so, where the Python package loads it.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "lmcache_amd", "liblmcache_amd.so")
SOURCES = ["kv_transfer.hip", "kv_noalloc.hip", "kv_direct.hip", "kv_sparse_graph.hip", "indexer_c8.hip", "cachegen.hip", "rope.hip",
           "host_mem.cpp", "host_shm.cpp", "dma_copy.hip", "blend.hip"]
ARCH = "gfx950"

# Packed-FP32 instructions are kept out of every code object.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO, "include"),
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; a ROCm toolchain is required")
    return found


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


EXT_SRC = "torch_binding.cpp"


def build_torch_binding(verbose: bool = False) -> str:
    """Compiles the pybind11 binding (host code only, g++) against torch."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(HERE, "lmcache_amd", "_c_ops_ext" + suffix)
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    incs = ce.include_paths() + [sysconfig.get_paths()["include"], os.path.join(rocm, "include"),
                                 os.path.join(REPO, "include")]
    libdirs = ce.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_c_ops_ext",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-DUSE_ROCM=1", "-D__HIP_PLATFORM_AMD__=1",
           *[f"-I{i}" for i in incs], os.path.join(CSRC, EXT_SRC), "-o", out + ".tmp",
           *[f"-L{d}" for d in libdirs], *[f"-Wl,-rpath,{d}" for d in libdirs],
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch binding build failed:\n{res.stderr[-4000:]}")
    os.replace(out + ".tmp", out)
    if verbose:
        print(f"built {out}")
    return out


def build(jobs: int = 4, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    build_torch_binding(verbose)
    return OUT


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
