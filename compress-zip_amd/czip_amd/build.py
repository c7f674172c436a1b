"""Build recipe of libczip_hip.so (gfx950) -- in-tree, no JIT cache.

Every HIP translation unit is compiled with hipcc for gfx950 only, with the
packed-FP32 instructions disabled, then linked into one shared library that
exports the C-ABI of include/czip_hip.h.  The benchmark's ceiling probes (a
copy kernel and an int8 MFMA loop) go into a library of their own,
libczip_ceiling.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT, "csrc")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_PATH = os.path.join(ROOT, "libczip_hip.so")
CEILING_SOURCE = "czip_ceiling.hip"
CEILING_LIB_PATH = os.path.join(ROOT, "libczip_ceiling.so")

SOURCES = ["czip_rows.hip", "czip_gemm.hip", "czip_head.hip", "czip_attention.hip", "czip_decode.hip", "czip_ffn.hip",
           "czip_api.cpp",
           "czm_loader.cpp", "czip_tokenizer.cpp", "czip_container.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-result", "-I", os.path.join(ROOT, "..", "include")]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def _link(objs, path: str):
    tmp = path + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, path)


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as ex:
        objs = list(ex.map(_compile, SOURCES + [CEILING_SOURCE]))
    _link(objs[:-1], LIB_PATH)
    _link(objs[-1:], CEILING_LIB_PATH)
    if verbose:
        print("built", LIB_PATH, "and", CEILING_LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
