"""The path as PyTorch custom operators (namespace ``etmoe``).

Registered with ``torch.library.custom_op``, each with a fake (meta) kernel for
tracing and, where the operation has a gradient, ``register_autograd``.  So
``torch.compile(fullgraph=True)`` and ``torch.export`` see one opaque node per
operation instead of breaking the graph at a ctypes call.  The routing plan
travels as a tuple of tensors:

    (counts[E], expert_offsets[E+1], token_offsets[T+1],
     sorted_token[S], slot_gate[S], token_slot[S])

S, the routed slot count, is data-dependent: the fake kernel of ``route``
returns it as an unbacked symbolic size.  ``route_with_capacity`` fixes the
slot arrays at a caller-chosen capacity instead (no host synchronisation;
rows past expert_offsets[E] are then unused).

Every eager kernel calls the C ABI of libetmoe.so through the functions of
``expert_threshold`` (argument checks there); there is no CPU kernel.

    torch.ops.etmoe.route(logits, thr)                          -> plan tuple
    torch.ops.etmoe.route_with_capacity(logits, thr, capacity)  -> plan tuple
    torch.ops.etmoe.dispatch(x, token_offsets, token_slot)      -> Xp [rows, d]
    torch.ops.etmoe.combine(yp, logits, slot_gate, sorted_token, token_offsets,
                            token_slot, expert_offsets)         -> Y [T, d]
    torch.ops.etmoe.combine_backward(dy, yp, slot_gate, sorted_token,
                            token_offsets, token_slot, expert_offsets,
                            need_dlogits)                       -> (dYp, dgate, dlogits)
    torch.ops.etmoe.dispatch_backward(dxp, token_offsets, token_slot) -> dX [T, d]
    torch.ops.etmoe.threshold_update_(thr, logits, k_target, momentum) -> stat (thr updated in place)

Gradients: dispatch -> dispatch_backward; combine -> combine_backward, with
respect to yp, to the router logits (through the gates, which are the
sigmoid scores at the routed pairs: dlogits) and to slot_gate (dgate).  The
routing itself is piecewise constant and has no gradient.
"""
from typing import Tuple

import torch
from torch import Tensor

from . import expert_threshold as _et

Plan = Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]


def plan_tensors(plan: _et.RoutingPlan) -> Plan:
    """A RoutingPlan as the tuple the operators take."""
    return (plan.counts, plan.expert_offsets, plan.token_offsets, plan.sorted_token, plan.slot_gate,
            plan.token_slot)


# --------------------------------------------------------------------------- #
# routing
# --------------------------------------------------------------------------- #

@torch.library.custom_op("etmoe::route", mutates_args=())
def route(logits: Tensor, thr: Tensor) -> Plan:
    """Threshold routing with exactly-sized slot arrays (one host
    synchronisation to read S)."""
    p = _et.route(logits, thr)
    return (p.counts, p.expert_offsets, p.token_offsets, p.sorted_token, p.slot_gate, p.token_slot)


@route.register_fake
def _route_fake(logits, thr):
    T, E = logits.shape
    S = torch.library.get_ctx().new_dynamic_size()
    i32 = dict(dtype=torch.int32, device=logits.device)
    return (logits.new_empty(E, **i32), logits.new_empty(E + 1, **i32), logits.new_empty(T + 1, **i32),
            logits.new_empty(S, **i32), logits.new_empty(S, dtype=torch.float32), logits.new_empty(S, **i32))


@torch.library.custom_op("etmoe::route_with_capacity", mutates_args=())
def route_with_capacity(logits: Tensor, thr: Tensor, slot_capacity: int) -> Plan:
    """Threshold routing into slot arrays of `slot_capacity` entries (no host
    synchronisation); the first expert_offsets[E] entries are the slots."""
    p = _et.route(logits, thr, slot_capacity=slot_capacity)
    return (p.counts, p.expert_offsets, p.token_offsets, p.sorted_token, p.slot_gate, p.token_slot)


@route_with_capacity.register_fake
def _route_cap_fake(logits, thr, slot_capacity):
    T, E = logits.shape
    i32 = dict(dtype=torch.int32, device=logits.device)
    cap = slot_capacity
    return (logits.new_empty(E, **i32), logits.new_empty(E + 1, **i32), logits.new_empty(T + 1, **i32),
            logits.new_empty(cap, **i32), logits.new_empty(cap, dtype=torch.float32), logits.new_empty(cap, **i32))


@torch.library.custom_op("etmoe::threshold_update_", mutates_args=("thr",))
def threshold_update_(thr: Tensor, logits: Tensor, k_target: int, momentum: float) -> Tensor:
    """EMA threshold update in place on thr; returns the per-expert statistic."""
    return _et.threshold_update_(thr, logits, k_target, momentum)


@threshold_update_.register_fake
def _threshold_update_fake(thr, logits, k_target, momentum):
    return thr.new_empty(thr.shape)


# --------------------------------------------------------------------------- #
# dispatch / combine and their backward
# --------------------------------------------------------------------------- #

def _rows_plan(token_offsets, token_slot, slot_gate=None, sorted_token=None, expert_offsets=None, counts=None):
    """A RoutingPlan over the given plan tensors (dispatch and its backward
    need only the token-major lists)."""
    T = token_offsets.shape[0] - 1
    E = expert_offsets.shape[0] - 1 if expert_offsets is not None else 0
    rows = token_slot.shape[0]
    return _et.RoutingPlan(counts, expert_offsets, token_offsets, sorted_token, slot_gate, token_slot, T, E, rows,
                           rows)


@torch.library.custom_op("etmoe::dispatch", mutates_args=())
def dispatch(x: Tensor, token_offsets: Tensor, token_slot: Tensor) -> Tensor:
    """Xp[slot] = X[token(slot)], one row per entry of token_slot."""
    return _et.dispatch(x, _rows_plan(token_offsets, token_slot))


@dispatch.register_fake
def _dispatch_fake(x, token_offsets, token_slot):
    return x.new_empty(token_slot.shape[0], x.shape[1])


@torch.library.custom_op("etmoe::dispatch_backward", mutates_args=())
def dispatch_backward(dxp: Tensor, token_offsets: Tensor, token_slot: Tensor) -> Tensor:
    """dX[t] = the sum of dXp over t's slots in ascending expert order."""
    return _et.dispatch_backward(dxp, _rows_plan(token_offsets, token_slot))


@dispatch_backward.register_fake
def _dispatch_backward_fake(dxp, token_offsets, token_slot):
    return dxp.new_empty(token_offsets.shape[0] - 1, dxp.shape[1])


@torch.library.custom_op("etmoe::combine", mutates_args=())
def combine(yp: Tensor, logits: Tensor, slot_gate: Tensor, sorted_token: Tensor, token_offsets: Tensor,
            token_slot: Tensor, expert_offsets: Tensor) -> Tensor:
    """Y[t] = sum over t's slots of slot_gate * Yp (fma chain, ascending
    expert).  `logits` is not read: it is the input the gradient through the
    gates flows to."""
    return _et.combine(yp, _rows_plan(token_offsets, token_slot, slot_gate, sorted_token, expert_offsets))


@combine.register_fake
def _combine_fake(yp, logits, slot_gate, sorted_token, token_offsets, token_slot, expert_offsets):
    return yp.new_empty(token_offsets.shape[0] - 1, yp.shape[1])


@torch.library.custom_op("etmoe::combine_backward", mutates_args=())
def combine_backward(dy: Tensor, yp: Tensor, slot_gate: Tensor, sorted_token: Tensor, token_offsets: Tensor,
                     token_slot: Tensor, expert_offsets: Tensor, need_dlogits: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """(dYp, dgate, dlogits): dYp = gate * dY[token], dgate = <dY, Yp> in
    binary64 rounded once, dlogits [T, E] (or [0, E] when not requested)."""
    plan = _rows_plan(token_offsets, token_slot, slot_gate, sorted_token, expert_offsets)
    dyp, dgate, dl = _et.combine_backward(dy, yp, plan, need_dlogits=need_dlogits)
    if dl is None:
        dl = dy.new_empty(0, plan.num_experts, dtype=torch.float32)
    return dyp, dgate, dl


@combine_backward.register_fake
def _combine_backward_fake(dy, yp, slot_gate, sorted_token, token_offsets, token_slot, expert_offsets,
                           need_dlogits):
    T = token_offsets.shape[0] - 1
    E = expert_offsets.shape[0] - 1
    return (yp.new_empty(yp.shape), yp.new_empty(yp.shape[0], dtype=torch.float32),
            dy.new_empty(T if need_dlogits else 0, E, dtype=torch.float32))


# --------------------------------------------------------------------------- #
# autograd
# --------------------------------------------------------------------------- #

def _dispatch_setup(ctx, inputs, output):
    _x, token_offsets, token_slot = inputs
    ctx.save_for_backward(token_offsets, token_slot)


def _dispatch_grad(ctx, dxp):
    token_offsets, token_slot = ctx.saved_tensors
    return torch.ops.etmoe.dispatch_backward(dxp.contiguous(), token_offsets, token_slot), None, None


torch.library.register_autograd("etmoe::dispatch", _dispatch_grad, setup_context=_dispatch_setup)


def _combine_setup(ctx, inputs, output):
    yp, _logits, slot_gate, sorted_token, token_offsets, token_slot, expert_offsets = inputs
    ctx.save_for_backward(yp, slot_gate, sorted_token, token_offsets, token_slot, expert_offsets)


def _combine_grad(ctx, dy):
    yp, slot_gate, sorted_token, token_offsets, token_slot, expert_offsets = ctx.saved_tensors
    need_dl = bool(ctx.needs_input_grad[1])
    dyp, dgate, dl = torch.ops.etmoe.combine_backward(dy.contiguous(), yp, slot_gate, sorted_token, token_offsets,
                                                      token_slot, expert_offsets, need_dl)
    return dyp, (dl if need_dl else None), dgate, None, None, None, None


torch.library.register_autograd("etmoe::combine", _combine_grad, setup_context=_combine_setup)
