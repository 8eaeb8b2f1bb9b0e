"""Builds libd2sd.so (the C-ABI library) in-tree with hipcc for gfx950, and
libd2sd_torch.so (torch.ops.d2sd.*, host C++ over that C ABI) with g++.

    python d2-sd_amd/d2sd/_build.py     (or __graft_entry__.build())

Every call compiles from source; objects go to d2-sd_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent          # d2-sd_amd/d2sd
ROOT = PKG_DIR.parent                               # d2-sd_amd
CSRC = ROOT / "csrc"
OBJ_DIR = ROOT / "_build"
LIB_PATH = PKG_DIR / "libd2sd.so"
TORCH_LIB_PATH = PKG_DIR / "libd2sd_torch.so"
INCLUDE = ROOT.parent / "include"

ARCH = "gfx950"
SOURCES = ["attention.hip", "verify_attention.hip", "kv_append.hip", "accept.hip", "qk_rope.hip", "tree_build.hip",
           "plan.cpp", "capi.cpp"]

COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function", f"-I{INCLUDE}", f"-I{CSRC}"]
# Device code: never let the compiler emit packed-fp32 VALU forms.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-ffp-contract=fast"]
# Per-source extras.  verify_attention.hip runs one wave per SIMD with up to
# 512 registers; MFMA results in VGPRs (not AGPRs) keep the accumulators out
# of per-tile AGPR<->VGPR copies.  Its inputs are NaN-free by contract (scores
# use -inf, never NaN): without NaN semantics the row maxima need no
# canonicalising v_max x, x of every MFMA result (one VALU op per score).
# The work-list pointer is the kernels' first argument (and the attention
# kernel's run-time prefix lengths its second): preloaded into SGPRs at wave
# launch, so a workgroup's first loads (its item, request 0's prefix length)
# depend on nothing.
EXTRA = {"verify_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans",
                                  "-mllvm", "-amdgpu-kernarg-preload-count=4"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libd2sd.so)")


def _compile(src: str) -> Path:
    path = CSRC / src
    obj = OBJ_DIR / (path.stem + ".o")
    cmd = [hipcc(), *COMMON]
    if path.suffix == ".hip":
        cmd += DEVICE + EXTRA.get(src, [])
    else:
        cmd += ["-x", "c++", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]
    cmd += ["-c", str(path), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libd2sd.so", *map(str, objs),
           "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    build_torch_ops(verbose)
    return LIB_PATH


def build_torch_ops(verbose: bool = False) -> Path:
    """torch_ops.cpp -> libd2sd_torch.so: the TORCH_LIBRARY(d2sd, ...)
    registrations, linked against libd2sd.so (found next to it, by soname)."""
    import torch
    from torch.utils import cpp_extension as ce
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    tmp = TORCH_LIB_PATH.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-Wno-unused-function",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
           *[f"-I{p}" for p in ce.include_paths()], f"-I{INCLUDE}", "-I/opt/rocm/include",
           str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
           f"-L{torch_lib}", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip",
           f"-L{PKG_DIR}", "-ld2sd", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch ops build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, TORCH_LIB_PATH)
    if verbose:
        print(f"built {TORCH_LIB_PATH}")
    return TORCH_LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
