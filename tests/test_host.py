"""Host-side API checks that need no GPU: argument validation happens in
Python before any device call, and the package never falls back to the CPU."""
import importlib

import pytest
import torch


def test_api_rejects_host_tensors(et):
    lg = torch.zeros(4, 2)
    thr = torch.zeros(2)
    with pytest.raises(ValueError, match="HIP device"):
        et.route(lg, thr)
    with pytest.raises(TypeError):
        et.route(lg.numpy(), thr)


def test_api_rejects_bad_arguments_before_device_work(et):
    # host tensors are refused before any dtype/shape logic can reach the device
    with pytest.raises(ValueError, match="HIP device"):
        et.dispatch(torch.zeros(4, 8, dtype=torch.float16), None)
    with pytest.raises(ValueError, match="HIP device"):
        et.threshold_update_(torch.zeros(3), torch.zeros(5, 3), k_target=1)
    with pytest.raises(ValueError, match="HIP device"):
        et.combine_backward(torch.zeros(2, 2), torch.zeros(2, 2), None)


def test_expert_threshold_router_validates_k(et):
    with pytest.raises(ValueError):
        et.ExpertThresholdRouter(num_experts=4, k_target=5, device="cpu")


def test_package_has_no_oracle_dependency():
    """The product package never imports, loads or links the CPU oracle."""
    import os
    import re
    from conftest import ROOT
    pkg = os.path.join(ROOT, "peer-review-agents_amd")
    pattern = re.compile(r"import\s+oracle|from\s+oracle|liboracle|oracle_[a-z]+\(")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not pattern.search(text), f


def test_missing_library_raises(monkeypatch, tmp_path):
    lib_mod = importlib.import_module("peer-review-agents_amd._lib")
    monkeypatch.setattr(lib_mod, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(lib_mod, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        lib_mod.lib()
