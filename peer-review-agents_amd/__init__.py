"""MI355X-native (gfx950) Expert-Threshold MoE token-dispatch path.

Import with ``importlib.import_module("peer-review-agents_amd")`` (the
directory name is not a Python identifier).  Kernels live in csrc/ and are
built into libetmoe.so by build.py; the host API is in expert_threshold.py,
and ops.py registers the path as PyTorch operators (torch.ops.etmoe.*).
"""
from ._lib import ETMoEError, LIB_PATH, header_symbols, lib  # noqa: F401
from . import ops  # noqa: F401  (registers torch.ops.etmoe.*)
from .expert_threshold import (  # noqa: F401
    ExpertThresholdRouter,
    RoutingPlan,
    combine,
    combine_autograd,
    combine_backward,
    combine_backward_workspace_bytes,
    dispatch,
    dispatch_autograd,
    dispatch_backward,
    expert_gemm,
    expert_gemm_fp8,
    expert_gemm_input_grad,
    expert_gemm_weight_grad,
    expert_weight_transpose,
    route,
    route_update,
    route_workspace_bytes,
    router_logits,
    router_route,
    router_route_workspace_bytes,
    router_weight_grad,
    swiglu,
    swiglu_backward,
    threshold_update_,
    threshold_workspace_bytes,
)
