"""Host-side API of the Expert-Threshold MoE token-dispatch path.

Every function validates its arguments in Python (raising ValueError or
TypeError before anything reaches the device), allocates outputs with torch's
caching allocator, and calls one entry point of libetmoe.so on torch's current
HIP stream.  torch is only plumbing here -- device memory and streams; all
arithmetic runs in the HIP kernels.  There is no CPU fallback: without the
library every call raises.

The reference tree (bat0001/peer-review-agents) has no operator for this path
(it is an agent-launcher CLI; its only plug-in points are the backend registry
at cli/reva/backends.py:28-131 and the translator table at
cli/reva/translators/__init__.py:33-53), so the names and signatures below are
this package's own.

Data layout after routing (all int32 except slot_gate):
    counts[E], expert_offsets[E+1]      CSR of slots by expert
    token_offsets[T+1], token_slot[S]   CSR of slots by token (ascending expert)
    sorted_token[S], slot_gate[S]       slot -> token id, slot -> gate (score)
Slots are ordered by (expert, token id).  Slot-major activations (Xp, Yp, dYp,
dXp) have one row per slot.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from ._lib import (ET_DTYPE_BF16, ET_DTYPE_F32, ET_GEMM_PLAIN, ET_GEMM_ROW_SCALE, ET_GEMM_SWIGLU,
                   ET_MAX_EXPERTS, ET_MAX_ROUTER_EXPERTS, check, lib)

_ACT_DTYPES = {torch.float32: ET_DTYPE_F32, torch.bfloat16: ET_DTYPE_BF16}


# --------------------------------------------------------------------------- #
# helpers
# --------------------------------------------------------------------------- #

def _vp(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_device(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a HIP device, got {t.device}")


def _require(t: torch.Tensor, name: str, dtype, ndim: int, device=None) -> None:
    _require_device(t, name)
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _act_dtype(t: torch.Tensor, name: str) -> int:
    if t.dtype not in _ACT_DTYPES:
        raise TypeError(f"{name} must be float32 or bfloat16, got {t.dtype}")
    return _ACT_DTYPES[t.dtype]


def _require_act(t: torch.Tensor, name: str, device=None) -> int:
    _require_device(t, name)
    dt = _act_dtype(t, name)
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D [rows, d], got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    return dt


# --------------------------------------------------------------------------- #
# routing
# --------------------------------------------------------------------------- #

@dataclass
class RoutingPlan:
    """Result of :func:`route`.

    ``num_slots`` is the host-side slot count S when routing synchronised to
    read it (the default); the slot arrays are then exactly S long.  With an
    explicit ``slot_capacity`` routing does not synchronise, ``num_slots`` is
    None and the slot arrays have ``capacity`` entries of which the first
    ``expert_offsets[E]`` are valid.
    """

    counts: torch.Tensor
    expert_offsets: torch.Tensor
    token_offsets: torch.Tensor
    sorted_token: torch.Tensor
    slot_gate: torch.Tensor
    token_slot: torch.Tensor
    num_tokens: int
    num_experts: int
    capacity: int
    num_slots: Optional[int] = None

    @property
    def rows(self) -> int:
        """Rows of a slot-major activation buffer for this plan."""
        return self.num_slots if self.num_slots is not None else self.capacity

    @property
    def device(self) -> torch.device:
        return self.token_offsets.device


def route_workspace_bytes(num_tokens: int, num_experts: int) -> int:
    return int(lib().et_route_workspace_bytes(num_tokens, num_experts))


def route(logits: torch.Tensor, thr: torch.Tensor, *, slot_capacity: Optional[int] = None,
          workspace: Optional[torch.Tensor] = None) -> RoutingPlan:
    """Threshold routing + CSR + stable permutation indices.

    logits: float32 [T, E] router logits (score = sigmoid(logit)).
    thr:    float32 [E] per-expert thresholds.
    (t, e) is routed iff score >= thr[e]; a token with no expert goes to its
    argmax expert.  Deterministic: identical inputs give identical bits.
    """
    _require(logits, "logits", torch.float32, 2)
    dev = logits.device
    T, E = logits.shape
    _require(thr, "thr", torch.float32, 1, dev)
    if thr.shape[0] != E:
        raise ValueError(f"thr has {thr.shape[0]} entries, logits has {E} experts")
    if not 1 <= E <= ET_MAX_EXPERTS:
        raise ValueError(f"num_experts must be in [1, {ET_MAX_EXPERTS}], got {E}")
    if T * E >= 2 ** 31:
        raise ValueError("num_tokens * num_experts must be < 2^31 (int32 slot indices)")
    sync = slot_capacity is None
    cap = T * E if sync else int(slot_capacity)
    if cap < 0:
        raise ValueError("slot_capacity must be >= 0")
    i32 = dict(dtype=torch.int32, device=dev)
    counts = torch.empty(E, **i32)
    eo = torch.empty(E + 1, **i32)
    to = torch.empty(T + 1, **i32)
    st = torch.empty(cap, **i32)
    sg = torch.empty(cap, dtype=torch.float32, device=dev)
    ts = torch.empty(cap, **i32)
    wsb = route_workspace_bytes(T, E)
    if workspace is None:
        workspace = torch.empty(wsb, dtype=torch.uint8, device=dev)
    elif workspace.device != dev or workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace must hold {wsb} bytes on {dev}")
    with torch.cuda.device(dev):
        rc = lib().et_route(_vp(logits), _vp(thr), T, E, _vp(counts), _vp(eo), _vp(to), _vp(st),
                            _vp(sg), _vp(ts), cap, _vp(workspace), wsb, _stream(dev))
    check("et_route", rc)
    plan = RoutingPlan(counts, eo, to, st, sg, ts, T, E, cap)
    if sync:
        _shrink(plan, int(eo[E].item()))
    return plan


def _shrink(plan: RoutingPlan, S: int) -> None:
    """Exactly-sized copies of the slot arrays of a plan routed at capacity
    T*E, so the T*E buffers are released (a plan held until a backward pass
    then pins 12 bytes per slot, not per token-expert pair)."""
    plan.num_slots = S
    plan.sorted_token = plan.sorted_token[:S].clone()
    plan.slot_gate = plan.slot_gate[:S].clone()
    plan.token_slot = plan.token_slot[:S].clone()
    plan.capacity = S


# --------------------------------------------------------------------------- #
# dispatch / combine
# --------------------------------------------------------------------------- #

def _out_or_new(out, shape, dtype, dev, name):
    if out is None:
        return torch.empty(shape, dtype=dtype, device=dev)
    _require(out, name, dtype, len(shape), dev)
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(out.shape)}")
    return out


def _check_plan(plan: RoutingPlan, dev: torch.device) -> None:
    if plan.device != dev:
        raise ValueError(f"plan is on {plan.device}, tensors are on {dev}")


def dispatch(x: torch.Tensor, plan: RoutingPlan, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Permute (scatter): Xp[slot] = X[token(slot)].  x: [T, d] f32/bf16."""
    dt = _require_act(x, "x")
    dev = x.device
    _check_plan(plan, dev)
    T, d = x.shape
    if T != plan.num_tokens:
        raise ValueError(f"x has {T} tokens, plan has {plan.num_tokens}")
    xp = _out_or_new(out, (plan.rows, d), x.dtype, dev, "out")
    with torch.cuda.device(dev):
        rc = lib().et_dispatch_fwd(_vp(x), T, d, dt, _vp(plan.token_offsets), _vp(plan.token_slot),
                                   plan.rows, _vp(xp), _stream(dev))
    check("et_dispatch_fwd", rc)
    return xp


def combine(yp: torch.Tensor, plan: RoutingPlan, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Un-permute with gate-weighted combine: Y[t] = sum_s gate[s] * Yp[s]."""
    dt = _require_act(yp, "yp")
    dev = yp.device
    _check_plan(plan, dev)
    if yp.shape[0] != plan.rows:
        raise ValueError(f"yp has {yp.shape[0]} rows, plan has {plan.rows} slots")
    T, d = plan.num_tokens, yp.shape[1]
    y = _out_or_new(out, (T, d), yp.dtype, dev, "out")
    with torch.cuda.device(dev):
        rc = lib().et_combine_fwd(_vp(yp), _vp(plan.slot_gate), _vp(plan.token_offsets),
                                  _vp(plan.token_slot), T, d, dt, plan.rows, _vp(y), _stream(dev))
    check("et_combine_fwd", rc)
    return y


def combine_backward_workspace_bytes(num_tokens: int, slot_capacity: int, d: int,
                                     dtype: torch.dtype) -> int:
    return int(lib().et_combine_bwd_workspace_bytes(num_tokens, slot_capacity, d,
                                                    _ACT_DTYPES[dtype]))


def combine_backward(dy: torch.Tensor, yp: torch.Tensor, plan: RoutingPlan, *,
                     need_dlogits: bool = False, out_dyp: Optional[torch.Tensor] = None,
                     out_dgate: Optional[torch.Tensor] = None,
                     out_dlogits: Optional[torch.Tensor] = None,
                     workspace: Optional[torch.Tensor] = None):
    """Fused backward of combine.

    Returns (dYp [S, d], dgate f32 [S], dlogits f32 [T, E] or None) with
    dYp[s] = gate[s] * dY[t], dgate[s] = <dY[t], Yp[s]>,
    dlogits[t, e] = dgate[s] * gate[s] * (1 - gate[s]) (0 where not routed).
    """
    dt = _require_act(dy, "dy")
    dev = dy.device
    if _require_act(yp, "yp", dev) != dt:
        raise TypeError("dy and yp must have the same dtype")
    _check_plan(plan, dev)
    T, d = dy.shape
    if T != plan.num_tokens:
        raise ValueError(f"dy has {T} tokens, plan has {plan.num_tokens}")
    if tuple(yp.shape) != (plan.rows, d):
        raise ValueError(f"yp must have shape {(plan.rows, d)}, got {tuple(yp.shape)}")
    E = plan.num_experts
    dyp = _out_or_new(out_dyp, (plan.rows, d), dy.dtype, dev, "out_dyp")
    dgate = _out_or_new(out_dgate, (plan.rows,), torch.float32, dev, "out_dgate")
    dl = None
    if need_dlogits or out_dlogits is not None:
        dl = _out_or_new(out_dlogits, (T, E), torch.float32, dev, "out_dlogits")
    wsb = combine_backward_workspace_bytes(T, plan.rows, d, dy.dtype)
    if workspace is None:
        workspace = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    elif workspace.device != dev or workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace must hold {wsb} bytes on {dev}")
    with torch.cuda.device(dev):
        rc = lib().et_combine_bwd(_vp(dy), _vp(yp), _vp(plan.slot_gate), _vp(plan.sorted_token),
                                  _vp(plan.token_offsets), _vp(plan.token_slot),
                                  _vp(plan.expert_offsets), T, E, d, dt,
                                  plan.rows, _vp(dyp), _vp(dgate), _vp(dl), _vp(workspace),
                                  workspace.numel() * workspace.element_size(), _stream(dev))
    check("et_combine_bwd", rc)
    return dyp, dgate, dl


def dispatch_backward(dxp: torch.Tensor, plan: RoutingPlan, out: Optional[torch.Tensor] = None, *,
                      router_weight: Optional[torch.Tensor] = None, dgate: Optional[torch.Tensor] = None,
                      workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Backward of dispatch: dX[t] = sum of dXp over t's slots (ascending expert).

    With ``router_weight`` (W [E, d], the dtype of dxp) and ``dgate`` (from
    :func:`combine_backward`), the router's input gradient through the routed
    logits is added in the same pass: per slot s of expert e,
    dX[t] += dl(s) * W[e] with dl(s) = dgate[s] * g * (1 - g), the dlogits
    entry of combine_backward -- i.e. dX + dlogits @ W.
    """
    dt = _require_act(dxp, "dxp")
    dev = dxp.device
    _check_plan(plan, dev)
    if dxp.shape[0] != plan.rows:
        raise ValueError(f"dxp has {dxp.shape[0]} rows, plan has {plan.rows} slots")
    T, d = plan.num_tokens, dxp.shape[1]
    dx = _out_or_new(out, (T, d), dxp.dtype, dev, "out")
    if (router_weight is None) != (dgate is None):
        raise ValueError("router_weight and dgate go together")
    if router_weight is None:
        with torch.cuda.device(dev):
            rc = lib().et_dispatch_bwd(_vp(dxp), _vp(plan.token_offsets), _vp(plan.token_slot), T, d, dt,
                                       plan.rows, _vp(dx), _stream(dev))
        check("et_dispatch_bwd", rc)
        return dx
    E = plan.num_experts
    _require(router_weight, "router_weight", dxp.dtype, 2, dev)
    if tuple(router_weight.shape) != (E, d):
        raise ValueError(f"router_weight must have shape {(E, d)}, got {tuple(router_weight.shape)}")
    _require(dgate, "dgate", torch.float32, 1, dev)
    if dgate.shape[0] != plan.rows:
        raise ValueError(f"dgate has {dgate.shape[0]} entries, plan has {plan.rows} slots")
    wsb = int(lib().et_dispatch_bwd_router_workspace_bytes(plan.rows))
    if workspace is None:
        workspace = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    elif workspace.device != dev or workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace must hold {wsb} bytes on {dev}")
    with torch.cuda.device(dev):
        rc = lib().et_dispatch_bwd_router(_vp(dxp), _vp(plan.token_offsets), _vp(plan.token_slot), T, d, dt,
                                          plan.rows, _vp(plan.slot_gate), _vp(dgate), _vp(plan.expert_offsets), E,
                                          _vp(router_weight), _vp(dx), _vp(workspace), wsb, _stream(dev))
    check("et_dispatch_bwd_router", rc)
    return dx


def router_weight_grad(dlogits: torch.Tensor, x: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                       workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Router weight gradient dW = dlogits^T X (float32 [E, d]) from the f32
    router-logit gradient [T, E] and the bf16 router input [T, d]."""
    _require(dlogits, "dlogits", torch.float32, 2)
    dev = dlogits.device
    _require(x, "x", torch.bfloat16, 2, dev)
    T, E = dlogits.shape
    if x.shape[0] != T:
        raise ValueError(f"x has {x.shape[0]} tokens, dlogits has {T}")
    d = x.shape[1]
    if not 1 <= E <= ET_MAX_ROUTER_EXPERTS:
        raise ValueError(f"num_experts must be in [1, {ET_MAX_ROUTER_EXPERTS}], got {E}")
    if d < 8 or d % 8 or d >= 1 << 22:
        raise ValueError(f"d must be a positive multiple of 8 below 2^22, got {d}")
    if T * d >= 1 << 30 or T * E >= 1 << 29:
        raise ValueError("x must be below 2^30 elements and dlogits below 2^29")
    dw = _out_or_new(out, (E, d), torch.float32, dev, "out")
    if x.data_ptr() % 16 or dw.data_ptr() % 16:
        raise ValueError("x and out must be 16-byte aligned")
    wsb = int(lib().et_router_wgrad_workspace_bytes(T, d, E))
    if workspace is None:
        workspace = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    elif workspace.device != dev or workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace must hold {wsb} bytes on {dev}")
    with torch.cuda.device(dev):
        rc = lib().et_router_wgrad(_vp(dlogits), _vp(x), T, d, E, _vp(dw), _vp(workspace), wsb, _stream(dev))
    check("et_router_wgrad", rc)
    return dw


# --------------------------------------------------------------------------- #
# expert grouped GEMM
# --------------------------------------------------------------------------- #

_EPILOGUES = {"none": ET_GEMM_PLAIN, "row_scale": ET_GEMM_ROW_SCALE, "swiglu": ET_GEMM_SWIGLU}


def expert_gemm(a: torch.Tensor, w: torch.Tensor, plan: RoutingPlan, *, gather: bool = True,
                epilogue: str = "none", row_scale: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Grouped expert GEMM over the plan's slot blocks (bf16, binary32 accumulation).

    p[s] = A[row(s)] @ W[e(s)]^T for every routed slot s, e(s) its expert, then
    the epilogue, rounded once to bf16:
      "none"       out[s] = p[s]                                   [rows, N]
      "row_scale"  out[s] = row_scale[s] * p[s]  (e.g. slot_gate)  [rows, N]
      "swiglu"     out[s, f] = silu(p[s, f]) * p[s, F + f], F = N/2 [rows, F]
                   (W holds each expert's gate rows, then its up rows)
    gather=True: ``a`` is the token matrix X [T, K] and row(s) = the slot's token
    (the dispatch fused into the GEMM: Xp is never materialised).
    gather=False: ``a`` is slot-major [rows, K] (e.g. dispatch(X) or an
    activation of the previous projection) and row(s) = s.
    ``w`` is [E, N, K], each expert's weight in nn.Linear layout.  Rows of
    ``out`` past the routed slots are left as they were.
    """
    _require(a, "a", torch.bfloat16, 2)
    dev = a.device
    _require(w, "w", torch.bfloat16, 3, dev)
    _check_plan(plan, dev)
    if epilogue not in _EPILOGUES:
        raise ValueError(f"epilogue must be one of {sorted(_EPILOGUES)}, got {epilogue!r}")
    E, N, K = w.shape
    if E != plan.num_experts:
        raise ValueError(f"w has {E} experts, plan has {plan.num_experts}")
    if a.shape[1] != K:
        raise ValueError(f"a has row length {a.shape[1]}, w has K = {K}")
    if K < 8 or K % 8 or K >= 1 << 22:
        raise ValueError(f"K must be a positive multiple of 8 below 2^22, got {K}")
    if N < 8 or N % 8 or (epilogue == "swiglu" and N % 16):
        raise ValueError(f"N must be a positive multiple of 8 (16 for swiglu), got {N}")
    if N * K * 2 >= 1 << 31:
        raise ValueError("one expert's weight must be below 2 GiB")
    if gather:
        if a.shape[0] != plan.num_tokens:
            raise ValueError(f"a has {a.shape[0]} rows, plan has {plan.num_tokens} tokens")
        if a.shape[0] * K * 2 >= 1 << 31:
            raise ValueError("in gather mode the token matrix must be below 2 GiB")
    elif a.shape[0] != plan.rows:
        raise ValueError(f"a has {a.shape[0]} rows, plan has {plan.rows} slots")
    if epilogue == "row_scale":
        if row_scale is None:
            raise ValueError("the row_scale epilogue needs row_scale")
        _require(row_scale, "row_scale", torch.float32, 1, dev)
        if row_scale.shape[0] < plan.rows:
            raise ValueError(f"row_scale has {row_scale.shape[0]} entries, plan has {plan.rows} slots")
    ncols = N // 2 if epilogue == "swiglu" else N
    c = _out_or_new(out, (plan.rows, ncols), torch.bfloat16, dev, "out")
    if a.data_ptr() % 16 or w.data_ptr() % 16 or c.data_ptr() % 16:
        raise ValueError("a, w and out must be 16-byte aligned")
    with torch.cuda.device(dev):
        rc = lib().et_expert_gemm(_vp(a), a.shape[0], _vp(plan.sorted_token) if gather else None, _vp(w),
                                  _vp(plan.expert_offsets), E, K, N, plan.rows, _EPILOGUES[epilogue],
                                  _vp(row_scale) if epilogue == "row_scale" else None, _vp(c), _stream(dev))
    check("et_expert_gemm", rc)
    return c


def expert_gemm_fp8(a: torch.Tensor, a_scale: torch.Tensor, w: torch.Tensor, w_scale: torch.Tensor,
                    plan: RoutingPlan, *, gather: bool = True, epilogue: str = "none",
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The expert grouped GEMM on fp8 e4m3 operands (``torch.float8_e4m3fn``):
    c[s] = ((A[row(s)] @ W[e(s)]^T) * a_scale[row(s)]) * w_scale[e(s)], bf16
    [rows, N] (or [rows, N / 2] with ``epilogue="swiglu"``).  a [T or rows, K],
    a_scale f32 [a rows], w [E, N, K], w_scale f32 [E, N]; row(s) as in
    :func:`expert_gemm`.  K a multiple of 16."""
    if a.dtype != torch.float8_e4m3fn or w.dtype != torch.float8_e4m3fn:
        raise TypeError("a and w must be torch.float8_e4m3fn")
    dev = a.device
    _require_device(a, "a")
    if a.dim() != 2 or not a.is_contiguous():
        raise ValueError("a must be a contiguous 2-D tensor")
    if w.dim() != 3 or not w.is_contiguous() or w.device != dev:
        raise ValueError("w must be a contiguous [E, N, K] tensor on a's device")
    _check_plan(plan, dev)
    E, N, K = w.shape
    if E != plan.num_experts or a.shape[1] != K:
        raise ValueError(f"w must be [{plan.num_experts}, N, {a.shape[1]}]")
    _require(a_scale, "a_scale", torch.float32, 1, dev)
    _require(w_scale, "w_scale", torch.float32, 2, dev)
    if a_scale.shape[0] != a.shape[0] or tuple(w_scale.shape) != (E, N):
        raise ValueError("a_scale must be [a rows] and w_scale [E, N]")
    epi = {"none": ET_GEMM_PLAIN, "swiglu": ET_GEMM_SWIGLU}.get(epilogue)
    if epi is None:
        raise ValueError(f"unknown epilogue {epilogue!r} (the fp8 GEMM has 'none' and 'swiglu')")
    if K < 16 or K % 16 or K >= 1 << 22:
        raise ValueError(f"K must be a positive multiple of 16 below 2^22, got {K}")
    if N < 8 or N % 8 or (epi == ET_GEMM_SWIGLU and N % 16):
        raise ValueError(f"N must be a positive multiple of 8 (16 for swiglu), got {N}")
    if N * K >= 1 << 31:
        raise ValueError("one expert's weight must be below 2 GiB")
    if gather:
        if a.shape[0] != plan.num_tokens:
            raise ValueError(f"a has {a.shape[0]} rows, plan has {plan.num_tokens} tokens")
        if a.shape[0] * K >= 1 << 31:
            raise ValueError("in gather mode the token matrix must be below 2 GiB")
    elif a.shape[0] != plan.rows:
        raise ValueError(f"slot-major a must have {plan.rows} rows")
    ncol = N // 2 if epi == ET_GEMM_SWIGLU else N
    c = _out_or_new(out, (plan.rows, ncol), torch.bfloat16, dev, "out")
    if a.data_ptr() % 16 or w.data_ptr() % 16 or c.data_ptr() % 16:
        raise ValueError("a, w and out must be 16-byte aligned")
    if a_scale.data_ptr() % 4 or w_scale.data_ptr() % 4:
        raise ValueError("a_scale and w_scale must be 4-byte aligned")
    with torch.cuda.device(dev):
        rc = lib().et_expert_gemm_fp8(_vp(a), a.shape[0], _vp(a_scale), _vp(plan.sorted_token) if gather else None,
                                      _vp(w), _vp(w_scale), _vp(plan.expert_offsets), E, K, N, plan.rows, epi,
                                      _vp(c), _stream(dev))
    check("et_expert_gemm_fp8", rc)
    return c


def expert_weight_transpose(w: torch.Tensor, plan: RoutingPlan, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """wt[e] = w[e]^T ([E, K, N] bf16) for the plan's experts with slots (the
    other experts' blocks of ``out`` are left as they were)."""
    _require(w, "w", torch.bfloat16, 3)
    dev = w.device
    _check_plan(plan, dev)
    E, N, K = w.shape
    if E != plan.num_experts:
        raise ValueError(f"w has {E} experts, plan has {plan.num_experts}")
    if N % 8 or K % 8 or N * K >= 1 << 31:
        raise ValueError("N and K must be multiples of 8 with N * K < 2^31")
    wt = _out_or_new(out, (E, K, N), torch.bfloat16, dev, "out")
    with torch.cuda.device(dev):
        rc = lib().et_expert_weight_transpose(_vp(w), _vp(plan.expert_offsets), E, N, K, plan.rows, _vp(wt),
                                              _stream(dev))
    check("et_expert_weight_transpose", rc)
    return wt


def expert_gemm_input_grad(dc: torch.Tensor, w: torch.Tensor, plan: RoutingPlan, *, gather: bool = False,
                           row_scale: Optional[torch.Tensor] = None, wt: Optional[torch.Tensor] = None,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Input gradient of :func:`expert_gemm`: da[s] = dC[row(s)] @ W[e(s)]
    ([rows, K] bf16), through the transposed weights of the experts with slots
    and the grouped GEMM.

    gather=True takes dC from a token matrix [T, N] at row(s) = token(s), and
    ``row_scale`` multiplies each slot's row: with dC = dY and row_scale =
    slot_gate this is the backward of the down projection fused with the
    combine backward (dYp = gate * dY[token] is never written).
    """
    wt = expert_weight_transpose(w, plan, out=wt)
    return expert_gemm(dc, wt, plan, gather=gather, epilogue="row_scale" if row_scale is not None else "none",
                       row_scale=row_scale, out=out)


def expert_gemm_weight_grad(dc: torch.Tensor, a: torch.Tensor, plan: RoutingPlan,
                            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Weight gradient of :func:`expert_gemm`: dw[e] = dC_e^T @ A_e over e's
    slots (f32 [E, N, K]; zeros for experts without slots).  dc [rows, N] and
    a [rows, K] are slot-major bf16 (a = dispatch(X) for a gathered forward)."""
    _require(dc, "dc", torch.bfloat16, 2)
    dev = dc.device
    _require(a, "a", torch.bfloat16, 2, dev)
    _check_plan(plan, dev)
    if dc.shape[0] != plan.rows or a.shape[0] != plan.rows:
        raise ValueError(f"dc and a must have {plan.rows} rows")
    N, K, E = dc.shape[1], a.shape[1], plan.num_experts
    if N % 8 or K % 8 or N * K * 4 >= 1 << 31:
        raise ValueError("N and K must be multiples of 8 with N * K * 4 < 2^31")
    dw = _out_or_new(out, (E, N, K), torch.float32, dev, "out")
    if dc.data_ptr() % 16 or a.data_ptr() % 16:
        raise ValueError("dc and a must be 16-byte aligned")
    with torch.cuda.device(dev):
        rc = lib().et_expert_wgrad(_vp(dc), _vp(a), _vp(plan.expert_offsets), E, N, K, plan.rows, _vp(dw),
                                   _stream(dev))
    check("et_expert_wgrad", rc)
    return dw


def _swiglu_args(gu: torch.Tensor, plan: RoutingPlan) -> int:
    _require(gu, "gu", torch.bfloat16, 2)
    _check_plan(plan, gu.device)
    if gu.shape[0] != plan.rows:
        raise ValueError(f"gu must have {plan.rows} rows (the plan's slot capacity)")
    if gu.shape[1] % 16:
        raise ValueError("gu must have 2F columns with F a multiple of 8")
    return gu.shape[1] // 2


def swiglu(gu: torch.Tensor, plan: RoutingPlan, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """SwiGLU of the expert FFN for training: h[s, j] = silu(g) * u with g =
    gu[s, j], u = gu[s, F + j] (gu = expert_gemm(...) without epilogue, kept for
    :func:`swiglu_backward`), bf16 [rows, F].  Same bits as the GEMM's
    ``epilogue="swiglu"`` applied to the rounded gu.  Rows past the routed slots
    are left as they were."""
    F = _swiglu_args(gu, plan)
    dev = gu.device
    h = _out_or_new(out, (plan.rows, F), torch.bfloat16, dev, "out")
    if gu.data_ptr() % 16 or h.data_ptr() % 16:
        raise ValueError("gu and out must be 16-byte aligned")
    with torch.cuda.device(dev):
        rc = lib().et_swiglu_fwd(_vp(gu), F, _vp(plan.expert_offsets), plan.num_experts, plan.rows, _vp(h),
                                 _stream(dev))
    check("et_swiglu_fwd", rc)
    return h


def swiglu_backward(gu: torch.Tensor, dh: torch.Tensor, plan: RoutingPlan,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Backward of :func:`swiglu`: dgu = [dh * u * silu'(g) | dh * silu(g)],
    bf16 [rows, 2F] (the gate/up projection's output gradient, ready for
    :func:`expert_gemm_input_grad` and :func:`expert_gemm_weight_grad`)."""
    F = _swiglu_args(gu, plan)
    dev = gu.device
    _require(dh, "dh", torch.bfloat16, 2, dev)
    if tuple(dh.shape) != (plan.rows, F):
        raise ValueError(f"dh must be [{plan.rows}, {F}]")
    dgu = _out_or_new(out, (plan.rows, 2 * F), torch.bfloat16, dev, "out")
    if gu.data_ptr() % 16 or dh.data_ptr() % 16 or dgu.data_ptr() % 16:
        raise ValueError("gu, dh and out must be 16-byte aligned")
    with torch.cuda.device(dev):
        rc = lib().et_swiglu_bwd(_vp(gu), _vp(dh), F, _vp(plan.expert_offsets), plan.num_experts, plan.rows,
                                 _vp(dgu), _stream(dev))
    check("et_swiglu_bwd", rc)
    return dgu


# --------------------------------------------------------------------------- #
# EMA threshold update
# --------------------------------------------------------------------------- #

def threshold_workspace_bytes(num_tokens: int, num_experts: int) -> int:
    return int(lib().et_threshold_workspace_bytes(num_tokens, num_experts))


def threshold_update_(thr: torch.Tensor, logits: torch.Tensor, k_target: int,
                      momentum: float = 0.99, *, stat: Optional[torch.Tensor] = None,
                      workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """In-place EMA update of thr from this batch; returns the statistic.

    stat[e] = c-th largest score of expert e, c = ceil(T * k_target / E);
    thr[e]  = fma(momentum, thr[e], (1 - momentum) * stat[e]).
    """
    _require(logits, "logits", torch.float32, 2)
    dev = logits.device
    T, E = logits.shape
    _require(thr, "thr", torch.float32, 1, dev)
    if thr.shape[0] != E:
        raise ValueError(f"thr has {thr.shape[0]} entries, logits has {E} experts")
    if not 1 <= E <= ET_MAX_EXPERTS:
        raise ValueError(f"num_experts must be in [1, {ET_MAX_EXPERTS}], got {E}")
    if not 1 <= int(k_target) <= E:
        raise ValueError(f"k_target must be in [1, {E}], got {k_target}")
    if not 0.0 <= float(momentum) <= 1.0:
        raise ValueError(f"momentum must be in [0, 1], got {momentum}")
    stat = _out_or_new(stat, (E,), torch.float32, dev, "stat")
    wsb = threshold_workspace_bytes(T, E)
    if workspace is None:
        workspace = torch.empty(wsb, dtype=torch.uint8, device=dev)
    elif workspace.device != dev or workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace must hold {wsb} bytes on {dev}")
    with torch.cuda.device(dev):
        rc = lib().et_threshold_update(_vp(logits), _vp(thr), T, E, int(k_target), float(momentum),
                                       _vp(stat), _vp(workspace), wsb, _stream(dev))
    check("et_threshold_update", rc)
    return stat


def route_update(logits: torch.Tensor, thr: torch.Tensor, k_target: int, momentum: float = 0.99, *,
                 slot_capacity: Optional[int] = None, stat: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None,
                 thr_workspace: Optional[torch.Tensor] = None) -> RoutingPlan:
    """Routing with the current thresholds, then the EMA update of thr from
    the same batch, in one call: the same results as :func:`route` followed by
    :func:`threshold_update_` (et_route_update), with every kernel on the
    current stream and the update's small passes in the routing's launches."""
    _require(logits, "logits", torch.float32, 2)
    dev = logits.device
    T, E = logits.shape
    _require(thr, "thr", torch.float32, 1, dev)
    if thr.shape[0] != E:
        raise ValueError(f"thr has {thr.shape[0]} entries, logits has {E} experts")
    if not 1 <= E <= ET_MAX_EXPERTS:
        raise ValueError(f"num_experts must be in [1, {ET_MAX_EXPERTS}], got {E}")
    if T * E >= 2 ** 31:
        raise ValueError("num_tokens * num_experts must be < 2^31 (int32 slot indices)")
    if not 1 <= int(k_target) <= E:
        raise ValueError(f"k_target must be in [1, {E}], got {k_target}")
    if not 0.0 <= float(momentum) <= 1.0:
        raise ValueError(f"momentum must be in [0, 1], got {momentum}")
    sync = slot_capacity is None
    cap = T * E if sync else int(slot_capacity)
    if cap < 0:
        raise ValueError("slot_capacity must be >= 0")
    if stat is not None:
        _out_or_new(stat, (E,), torch.float32, dev, "stat")
    i32 = dict(dtype=torch.int32, device=dev)
    counts = torch.empty(E, **i32)
    eo = torch.empty(E + 1, **i32)
    to = torch.empty(T + 1, **i32)
    st = torch.empty(cap, **i32)
    sg = torch.empty(cap, dtype=torch.float32, device=dev)
    ts = torch.empty(cap, **i32)
    rwsb, twsb = route_workspace_bytes(T, E), threshold_workspace_bytes(T, E)
    if workspace is None:
        workspace = torch.empty(rwsb, dtype=torch.uint8, device=dev)
    elif workspace.device != dev or workspace.numel() * workspace.element_size() < rwsb:
        raise ValueError(f"workspace must hold {rwsb} bytes on {dev}")
    if thr_workspace is None:
        thr_workspace = torch.empty(twsb, dtype=torch.uint8, device=dev)
    elif thr_workspace.device != dev or thr_workspace.numel() * thr_workspace.element_size() < twsb:
        raise ValueError(f"thr_workspace must hold {twsb} bytes on {dev}")
    a, b = workspace.data_ptr(), thr_workspace.data_ptr()
    if a < b + twsb and b < a + rwsb:
        raise ValueError("workspace and thr_workspace must not overlap")
    with torch.cuda.device(dev):
        rc = lib().et_route_update(_vp(logits), _vp(thr), T, E, _vp(counts), _vp(eo), _vp(to), _vp(st), _vp(sg),
                                   _vp(ts), cap, _vp(workspace), rwsb, int(k_target), float(momentum),
                                   _vp(stat) if stat is not None else None, _vp(thr_workspace), twsb,
                                   _stream(dev))
    check("et_route_update", rc)
    plan = RoutingPlan(counts, eo, to, st, sg, ts, T, E, cap)
    if sync:
        _shrink(plan, int(eo[E].item()))
    return plan


# --------------------------------------------------------------------------- #
# router producer
# --------------------------------------------------------------------------- #

def router_logits(x: torch.Tensor, w: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Router logits L = X W^T in float32 from bf16 X [T, d] and W [E, d].

    W is the router weight in nn.Linear layout.  Binary32 accumulation in a
    fixed order on the matrix cores (k-steps of 16 ascending from
    k0 = (t // 256 % 4) * 64 * (d // 256), wrapping to 0): repeated calls give
    identical bits.
    """
    _require(x, "x", torch.bfloat16, 2)
    dev = x.device
    _require(w, "w", torch.bfloat16, 2, dev)
    T, d = x.shape
    E, dw = w.shape
    if dw != d:
        raise ValueError(f"w has row length {dw}, x has {d}")
    if not 1 <= E <= ET_MAX_ROUTER_EXPERTS:
        raise ValueError(f"num_experts must be in [1, {ET_MAX_ROUTER_EXPERTS}], got {E}")
    if d < 8 or d % 8 or d >= 1 << 22:
        raise ValueError(f"d must be a positive multiple of 8 below 2^22, got {d}")
    if x.data_ptr() % 16 or w.data_ptr() % 16:
        raise ValueError("x and w must be 16-byte aligned")
    L = _out_or_new(out, (T, E), torch.float32, dev, "out")
    with torch.cuda.device(dev):
        rc = lib().et_router_logits(_vp(x), _vp(w), T, d, E, _vp(L), _stream(dev))
    check("et_router_logits", rc)
    return L


def router_route_workspace_bytes(num_tokens: int, num_experts: int) -> int:
    return int(lib().et_router_route_workspace_bytes(num_tokens, num_experts))


def router_route(x: torch.Tensor, w: torch.Tensor, thr: torch.Tensor, *, slot_capacity: Optional[int] = None,
                 return_logits: bool = False, logits_out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None):
    """Router GEMM fused with routing: ``route(router_logits(x, w), thr)``
    without writing the [T, E] scores.  Bit-identical to that composition.

    Returns the RoutingPlan, or (plan, logits) when ``return_logits`` is set or
    ``logits_out`` is given (the logits are then written too, e.g. for
    :func:`threshold_update_` on this batch).
    """
    _require(x, "x", torch.bfloat16, 2)
    dev = x.device
    _require(w, "w", torch.bfloat16, 2, dev)
    T, d = x.shape
    E, dw = w.shape
    if dw != d:
        raise ValueError(f"w has row length {dw}, x has {d}")
    if not 1 <= E <= ET_MAX_ROUTER_EXPERTS:
        raise ValueError(f"num_experts must be in [1, {ET_MAX_ROUTER_EXPERTS}], got {E}")
    if d < 8 or d % 8 or d >= 1 << 22:
        raise ValueError(f"d must be a positive multiple of 8 below 2^22, got {d}")
    if x.data_ptr() % 16 or w.data_ptr() % 16:
        raise ValueError("x and w must be 16-byte aligned")
    _require(thr, "thr", torch.float32, 1, dev)
    if thr.shape[0] != E:
        raise ValueError(f"thr has {thr.shape[0]} entries, w has {E} experts")
    if T * E >= 2 ** 31:
        raise ValueError("num_tokens * num_experts must be < 2^31 (int32 slot indices)")
    sync = slot_capacity is None
    cap = T * E if sync else int(slot_capacity)
    if cap < 0:
        raise ValueError("slot_capacity must be >= 0")
    want_logits = return_logits or logits_out is not None
    L = _out_or_new(logits_out, (T, E), torch.float32, dev, "logits_out") if want_logits else None
    i32 = dict(dtype=torch.int32, device=dev)
    counts = torch.empty(E, **i32)
    eo = torch.empty(E + 1, **i32)
    to = torch.empty(T + 1, **i32)
    st = torch.empty(cap, **i32)
    sg = torch.empty(cap, dtype=torch.float32, device=dev)
    ts = torch.empty(cap, **i32)
    wsb = router_route_workspace_bytes(T, E)
    if workspace is None:
        workspace = torch.empty(wsb, dtype=torch.uint8, device=dev)
    elif workspace.device != dev or workspace.numel() * workspace.element_size() < wsb:
        raise ValueError(f"workspace must hold {wsb} bytes on {dev}")
    with torch.cuda.device(dev):
        rc = lib().et_router_route(_vp(x), _vp(w), _vp(thr), T, d, E, _vp(counts), _vp(eo), _vp(to), _vp(st),
                                   _vp(sg), _vp(ts), cap, _vp(L), _vp(workspace), wsb, _stream(dev))
    check("et_router_route", rc)
    plan = RoutingPlan(counts, eo, to, st, sg, ts, T, E, cap)
    if sync:
        _shrink(plan, int(eo[E].item()))
    return (plan, L) if want_logits else plan


# --------------------------------------------------------------------------- #
# autograd wrappers
# --------------------------------------------------------------------------- #

class _DispatchFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, plan):
        ctx.plan = plan
        return dispatch(x, plan)

    @staticmethod
    def backward(ctx, dxp):
        return dispatch_backward(dxp.contiguous(), ctx.plan), None


class _CombineFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, yp, logits, plan):
        ctx.plan = plan
        ctx.save_for_backward(yp)
        return combine(yp, plan)

    @staticmethod
    def backward(ctx, dy):
        (yp,) = ctx.saved_tensors
        dyp, _dgate, dl = combine_backward(dy.contiguous(), yp, ctx.plan,
                                           need_dlogits=ctx.needs_input_grad[1])
        return dyp, dl, None


def dispatch_autograd(x: torch.Tensor, plan: RoutingPlan) -> torch.Tensor:
    """dispatch() with a backward that runs dispatch_backward()."""
    return _DispatchFn.apply(x, plan)


def combine_autograd(yp: torch.Tensor, logits: torch.Tensor, plan: RoutingPlan) -> torch.Tensor:
    """combine() differentiable in yp and in the router logits (through the
    gates, which are sigmoid(logits) at the routed pairs; the routing mask
    itself is piecewise constant and has no gradient)."""
    return _CombineFn.apply(yp, logits, plan)


class ExpertThresholdRouter(torch.nn.Module):
    """Per-expert thresholds with the EMA update applied after each training
    batch (route with the current thresholds, then update them from the batch),
    the way batch statistics are kept in a running buffer.  In training mode
    both go through :func:`route_update` (one call, the same bits as
    :func:`route` then :func:`threshold_update_`); in eval mode it only routes."""

    def __init__(self, num_experts: int, k_target: int, momentum: float = 0.99,
                 init_threshold: float = 0.5, device=None):
        super().__init__()
        if not 1 <= k_target <= num_experts:
            raise ValueError("k_target must be in [1, num_experts]")
        self.k_target = int(k_target)
        self.momentum = float(momentum)
        self.register_buffer("thr", torch.full((num_experts,), float(init_threshold),
                                               dtype=torch.float32, device=device))

    def forward(self, logits: torch.Tensor, *, slot_capacity: Optional[int] = None) -> RoutingPlan:
        if self.training:
            return route_update(logits.detach(), self.thr, self.k_target, self.momentum,
                                slot_capacity=slot_capacity)
        return route(logits.detach(), self.thr, slot_capacity=slot_capacity)
