"""Builds libinferd_amd.so (the HIP kernels + the C ABI of include/inferd_qmm.h) for gfx950 with hipcc, in-tree.

Usage: python -m inferd_amd.build   (or inferd_amd.build.build()). Every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libinferd_amd.so")
# the operator-level MoE timer bench.py runs (Qwen35::encode_moe over this library)
MOE_BENCH_SRC = os.path.join(HERE, "csrc", "encode_moe_bench.cpp")
MOE_BENCH = os.path.join(HERE, "encode_moe_bench")
OBJ = os.path.join(HERE, "_build")

SOURCES = ["qmv.hip", "qmm.hip", "w4a8.hip", "moe.hip", "t64.hip", "gemm_t64.hip", "gemm_sk.hip", "gemm_t8.hip",
           "w4a8_t64.hip", "w8a8_t64.hip", "fused.hip", "moe_dec.hip", "moe_t64.hip", "capi.hip", "workspace.hip",
           "probe.hip", "noalloc.hip"]

# Packed-fp32 VALU forms are kept out of every code object; hipcc's host pass warns that it does not know the
# feature, which is harmless.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-lambda-capture",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if p and (os.path.sep not in p or os.path.exists(p)):
            return p
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    missing = [s for s in SOURCES if not os.path.exists(os.path.join(CSRC, s))]
    if missing:
        raise RuntimeError(f"sources missing from {CSRC}: {missing}")
    srcs = list(SOURCES)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [_hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    cmd = [_hipcc(), "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wall",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(os.path.dirname(HERE), "include"), "-I", CSRC, MOE_BENCH_SRC, "-o", MOE_BENCH,
           "-L", HERE, "-linferd_amd", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"encode_moe_bench failed to build:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {OUT} and {MOE_BENCH}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
