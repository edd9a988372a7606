"""The torch.library operators (namespace etmoe) without a GPU: every operator
of the path is registered with the schema the C ABI needs, the fake kernels
give the shapes the eager kernels produce (the routed slot count S as an
unbacked symbolic size), and a forward pass over the operators traces into
one graph with one node per operator.  Their eager results and gradients, and
torch.compile(fullgraph=True) over them, are checked on the GPU in
tests/test_gpu_ops.py."""
import importlib

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx
from torch.fx.experimental.symbolic_shapes import ShapeEnv

importlib.import_module("peer-review-agents_amd.ops")

SCHEMAS = {
    "route": "etmoe::route(Tensor logits, Tensor thr) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    "route_with_capacity": "etmoe::route_with_capacity(Tensor logits, Tensor thr, SymInt slot_capacity) -> "
                           "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    "dispatch": "etmoe::dispatch(Tensor x, Tensor token_offsets, Tensor token_slot) -> Tensor",
    "dispatch_backward": "etmoe::dispatch_backward(Tensor dxp, Tensor token_offsets, Tensor token_slot) -> Tensor",
    "combine": "etmoe::combine(Tensor yp, Tensor logits, Tensor slot_gate, Tensor sorted_token, "
               "Tensor token_offsets, Tensor token_slot, Tensor expert_offsets) -> Tensor",
    "combine_backward": "etmoe::combine_backward(Tensor dy, Tensor yp, Tensor slot_gate, Tensor sorted_token, "
                        "Tensor token_offsets, Tensor token_slot, Tensor expert_offsets, bool need_dlogits) -> "
                        "(Tensor, Tensor, Tensor)",
    "threshold_update_": "etmoe::threshold_update_(Tensor(a0!) thr, Tensor logits, SymInt k_target, "
                         "float momentum) -> Tensor",
}


@pytest.mark.parametrize("name", sorted(SCHEMAS))
def test_operator_schema(name):
    assert str(getattr(torch.ops.etmoe, name).default._schema) == SCHEMAS[name]


def _fake():
    return FakeTensorMode(shape_env=ShapeEnv())


def test_fake_shapes_follow_the_plan():
    with _fake():
        T, E, d = 100, 8, 64
        lg = torch.empty(T, E, device="cuda")
        thr = torch.empty(E, device="cuda")
        counts, eo, to, st, sg, ts = torch.ops.etmoe.route(lg, thr)
        assert (counts.shape, eo.shape, to.shape) == ((E,), (E + 1,), (T + 1,))
        S = st.shape[0]
        assert isinstance(S, torch.SymInt) and sg.shape == (S,) and ts.shape == (S,)
        assert (counts.dtype, sg.dtype, ts.dtype) == (torch.int32, torch.float32, torch.int32)
        x = torch.empty(T, d, device="cuda", dtype=torch.bfloat16)
        xp = torch.ops.etmoe.dispatch(x, to, ts)
        assert xp.shape == (S, d) and xp.dtype == torch.bfloat16
        y = torch.ops.etmoe.combine(xp, lg, sg, st, to, ts, eo)
        assert y.shape == (T, d) and y.dtype == torch.bfloat16
        dyp, dgate, dl = torch.ops.etmoe.combine_backward(y, xp, sg, st, to, ts, eo, True)
        assert dyp.shape == (S, d) and dgate.shape == (S,) and dl.shape == (T, E) and dl.dtype == torch.float32
        assert torch.ops.etmoe.combine_backward(y, xp, sg, st, to, ts, eo, False)[2].shape == (0, E)
        assert torch.ops.etmoe.dispatch_backward(xp, to, ts).shape == (T, d)
        cap = torch.ops.etmoe.route_with_capacity(lg, thr, 333)
        assert [tuple(t.shape) for t in cap[3:]] == [(333,)] * 3
        assert torch.ops.etmoe.threshold_update_(thr, lg, 2, 0.99).shape == (E,)


def test_forward_traces_into_one_graph():
    def layer(x, logits, thr, scale):
        counts, eo, to, st, sg, ts = torch.ops.etmoe.route(logits, thr)
        xp = torch.ops.etmoe.dispatch(x, to, ts)
        return torch.ops.etmoe.combine(torch.tanh(xp) * scale, logits, sg, st, to, ts, eo)

    with _fake():
        args = (torch.empty(64, 32, device="cuda"), torch.empty(64, 4, device="cuda"),
                torch.empty(4, device="cuda"), torch.empty(32, device="cuda"))
        gm = make_fx(layer, tracing_mode="real")(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    for op in ("etmoe.route.default", "etmoe.dispatch.default", "etmoe.combine.default"):
        assert targets.count(op) == 1, targets
