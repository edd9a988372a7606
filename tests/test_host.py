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


def test_expert_gemm_fp8_checks_shapes_like_bf16(et):
    """The fp8 grouped GEMM validates what the bf16 one does, in Python and
    before any device call (fake HIP tensors: shapes only): a gather operand
    shorter than the token count, K off the 16-element step, N off the
    8-element step (16 for SwiGLU)."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    f8 = torch.float8_e4m3fn
    with FakeTensorMode():
        T, E, K, N = 64, 4, 128, 64
        i32 = dict(dtype=torch.int32, device="cuda")
        plan = et.RoutingPlan(torch.empty(E, **i32), torch.empty(E + 1, **i32), torch.empty(T + 1, **i32),
                              torch.empty(100, **i32), torch.empty(100, device="cuda"), torch.empty(100, **i32),
                              T, E, 100, 100)

        def call(a_rows=T, k=K, n=N, epilogue="none", gather=True):
            a = torch.empty(a_rows, k, dtype=f8, device="cuda")
            w = torch.empty(E, n, k, dtype=f8, device="cuda")
            return et.expert_gemm_fp8(a, torch.empty(a_rows, device="cuda"), w, torch.empty(E, n, device="cuda"),
                                      plan, gather=gather, epilogue=epilogue)

        with pytest.raises(ValueError, match="tokens"):
            call(a_rows=T - 1)
        with pytest.raises(ValueError, match="K must"):
            call(k=120)
        with pytest.raises(ValueError, match="N must"):
            call(n=60)
        with pytest.raises(ValueError, match="N must"):
            call(n=72, epilogue="swiglu")
        with pytest.raises(ValueError, match="slot-major"):
            call(a_rows=99, gather=False)
