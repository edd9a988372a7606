"""Builds libetmoe.so (gfx950) in-tree with hipcc.

Flags: -O3, -ffp-contract=off (every fused multiply-add in the kernels is an
explicit fma, so results match their written definition bit for bit), and the
packed-fp32 feature switched off for device code.

Each source is compiled to its own object in parallel (a source holds its
kernels and their host launchers, so no device code crosses files), then the
objects are linked into the shared library.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
import tempfile

_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)
SOURCES = ["et_abi.hip", "et_route.hip", "et_rows.hip", "et_threshold.hip", "et_router.hip", "et_router_bwd.hip",
           "et_expert_gemm.hip", "et_swiglu.hip"]
OUT = os.path.join(_HERE, "libetmoe.so")
ARCH = os.environ.get("ET_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    return os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")


def _flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            "-ffp-contract=off",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", os.path.join(_ROOT, "include")]


def hipcc_command(out: str = OUT) -> list[str]:
    """One hipcc line that builds the whole library (or, with its sources
    replaced, any other shared object with the library's flags)."""
    return [_hipcc()] + _flags() + ["-shared", "-o", out] + [os.path.join(_HERE, "csrc", s) for s in SOURCES]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with status {res.returncode}: {' '.join(cmd[-3:])}")


def build_library(verbose: bool = False, jobs: int | None = None) -> str:
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with tempfile.TemporaryDirectory(prefix="etmoe_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[_hipcc()] + _flags() + ["-c", "-o", o, os.path.join(_HERE, "csrc", s)]
                for s, o in zip(SOURCES, objs)]
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp = OUT + ".tmp"
        _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build_library(verbose=True))
