"""The kernels' f32 -> bf16 packing (one v_cvt_pk_bf16_f32 per two values) equals
the specified round-to-nearest-even rule with the oracle's NaN rule, checked
exhaustively over all 2^32 binary32 inputs on the GPU by
tests/gpu_checks/bf16_pack_check.hip.  (The oracle's own conversion is pinned
to torch's bf16 cast in tests/test_oracle.py.)"""
import ctypes
import os

import pytest

from conftest import ROOT

HELPER = os.path.join(ROOT, "tests", "gpu_checks", "libbf16check.so")


def _helper():
    # torch first: the helper links libamdhip64 by soname, and only with torch's
    # HIP runtime already mapped does it bind to that runtime (one per process)
    import torch  # noqa: F401
    if not os.path.exists(HELPER):
        raise RuntimeError(f"{HELPER} is not built; run __graft_entry__.build()")
    L = ctypes.CDLL(HELPER)
    L.bf16_pack_check.restype = ctypes.c_int
    L.bf16_pack_check.argtypes = [ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_uint)]
    return L


def test_helper_is_built_and_exports_the_check():
    assert hasattr(_helper(), "bf16_pack_check")


@pytest.mark.gpu
def test_hardware_bf16_pack_equals_rule_on_all_inputs(dev):
    import torch
    torch.cuda.synchronize()
    mis, first = ctypes.c_ulonglong(7), ctypes.c_uint(0)
    rc = _helper().bf16_pack_check(ctypes.byref(mis), ctypes.byref(first))
    assert rc == 0
    assert mis.value == 0, f"{mis.value} mismatching pairs, first input {first.value:#010x}"
    assert first.value == 0xFFFFFFFF
