"""Builds libetmoe.so (gfx950) in-tree with hipcc.

Flags: -O3, -ffp-contract=off (every fused multiply-add in the kernels is an
explicit fma, so results match their written definition bit for bit), and the
packed-fp32 feature switched off for device code.
"""
from __future__ import annotations

import os
import subprocess
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)
SOURCES = ["et_abi.hip", "et_route.hip", "et_rows.hip", "et_threshold.hip", "et_router.hip", "et_router_bwd.hip",
           "et_expert_gemm.hip", "et_swiglu.hip"]
OUT = os.path.join(_HERE, "libetmoe.so")
ARCH = os.environ.get("ET_OFFLOAD_ARCH", "gfx950")


def hipcc_command(out: str = OUT) -> list[str]:
    hipcc = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    return [hipcc, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-ffp-contract=off",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", os.path.join(_ROOT, "include"),
            "-o", out] + [os.path.join(_HERE, "csrc", s) for s in SOURCES]


def build_library(verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    cmd = hipcc_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with status {res.returncode}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build_library(verbose=True))
