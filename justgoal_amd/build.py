"""Builds ``libjustgoal_moe.so`` (all HIP kernels + the C ABI) in-tree for gfx950.

``python -m justgoal_amd.build`` or ``justgoal_amd.build.build()``. hipcc cross-compiles, so
this runs on a machine without a GPU.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB_NAME = "libjustgoal_moe.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["moe_api.hip", "moe_routing.hip", "moe_gemm.hip", "moe_stream.hip", "moe_tile.hip", "moe_big.hip", "moe_quant.hip"]
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed-FP32 VALU ops are kept out of the generated code on purpose
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results straight into VGPRs: the block-scale FMAs that follow every MFMA then need
    # no accumulator-register reads
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-result",
]


def build(verbose: bool = False, out: str = LIB_PATH) -> str:
    """Compile every source into one shared library; returns its path."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = out + f".{os.getpid()}.tmp"
    cmd = [HIPCC, *FLAGS, f"-I{INCLUDE}", "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {LIB_NAME}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
