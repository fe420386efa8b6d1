"""Build the C++ test programs: the operator-shim test (qwen35_ops_test) against the in-tree libinferd_amd.so and the
oracle, and the checkpoint-loader test (ckpt_test, host only, g++).

Run after inferd_amd.build and oracle's build (``__graft_entry__.build()`` does all three). qwen35_ops_test finds both
libraries through its RUNPATH, so it runs from any working directory.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
SRC = os.path.join(HERE, "qwen35_ops_test.cpp")
BIN = os.path.join(HERE, "qwen35_ops_test")
CKPT_SRC = os.path.join(HERE, "ckpt_test.cpp")
CKPT_BIN = os.path.join(HERE, "ckpt_test")


def build_ckpt(verbose: bool = False) -> str:
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-I", os.path.join(ROOT, "inferd_amd", "csrc"),
           CKPT_SRC, "-o", CKPT_BIN]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return CKPT_BIN


def build(verbose: bool = False) -> str:
    hipcc = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    cmd = [hipcc, "-O2", "-std=c++17", "-Wall", "--offload-arch=gfx950",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "inferd_amd", "csrc"),
           SRC, "-o", BIN,
           "-L", os.path.join(ROOT, "inferd_amd"), "-linferd_amd",
           "-L", os.path.join(ROOT, "oracle"), "-loracle",
           "-Wl,-rpath,$ORIGIN/../../inferd_amd", "-Wl,-rpath,$ORIGIN/../../oracle"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    build_ckpt(verbose)
    return BIN


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
