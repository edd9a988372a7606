"""Loader for libetmoe.so, the C-ABI HIP library of the Expert-Threshold MoE path.

torch is imported first on purpose: the library links libamdhip64 by soname, so
when torch's own HIP runtime is already mapped the library binds to it and
shares its device context and streams (one HIP runtime per process).

There is no fallback: if the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch  # noqa: F401  (see module docstring: must be loaded before the library)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libetmoe.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "etmoe.h")

ET_DTYPE_F32 = 0
ET_DTYPE_BF16 = 1
ET_MAX_EXPERTS = 1024
ET_MAX_ROUTER_EXPERTS = 256
ET_GEMM_PLAIN, ET_GEMM_ROW_SCALE, ET_GEMM_SWIGLU = 0, 1, 2


class ETMoEError(RuntimeError):
    """A libetmoe.so entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.fn = fn
        self.code = code


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t
_f = ctypes.c_float

_SIGNATURES = {
    "et_abi_version": (_int, []),
    "et_last_error": (ctypes.c_char_p, []),
    "et_route_workspace_bytes": (_sz, [_i64, _i64]),
    "et_route": (_int, [_p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _sz, _p]),
    "et_route_noalloc": (_int, [_p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "et_dispatch_fwd": (_int, [_p, _i64, _i64, _int, _p, _p, _i64, _p, _p]),
    "et_combine_fwd": (_int, [_p, _p, _p, _p, _i64, _i64, _int, _i64, _p, _p]),
    "et_combine_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _int]),
    "et_combine_bwd": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _i64, _p, _p, _p, _p, _sz,
                              _p]),
    "et_dispatch_bwd": (_int, [_p, _p, _p, _i64, _i64, _int, _i64, _p, _p]),
    "et_threshold_workspace_bytes": (_sz, [_i64, _i64]),
    "et_threshold_update": (_int, [_p, _p, _i64, _i64, _i64, _f, _p, _p, _sz, _p]),
    "et_route_update": (_int, [_p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _sz, _i64, _f, _p, _p, _sz, _p]),
    "et_router_logits": (_int, [_p, _p, _i64, _i64, _i64, _p, _p]),
    "et_router_route_workspace_bytes": (_sz, [_i64, _i64]),
    "et_router_route": (_int, [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _sz, _p]),
    "et_dispatch_bwd_router_workspace_bytes": (_sz, [_i64]),
    "et_dispatch_bwd_router": (_int, [_p, _p, _p, _i64, _i64, _int, _i64, _p, _p, _p, _i64, _p, _p, _p, _sz, _p]),
    "et_router_wgrad_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "et_router_wgrad": (_int, [_p, _p, _i64, _i64, _i64, _p, _p, _sz, _p]),
    "et_expert_gemm": (_int, [_p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _int, _p, _p, _p]),
    "et_expert_gemm_fp8": (_int, [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _int, _p, _p]),
    "et_expert_weight_transpose": (_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "et_expert_wgrad": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "et_swiglu_fwd": (_int, [_p, _i64, _p, _i64, _i64, _p, _p]),
    "et_swiglu_bwd": (_int, [_p, _p, _i64, _p, _i64, _i64, _p, _p]),
}

_lib = None


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of the functions declared in include/etmoe.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(et_[a-z_0-9]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(there is no CPU fallback for this path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, rc: int) -> None:
    if rc != 0:
        msg = lib().et_last_error()
        raise ETMoEError(fn, rc, msg.decode() if msg else "")
