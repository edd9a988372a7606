"""End-to-end use of the path inside a small Expert-Threshold MoE layer, the way
a model uses it: router Linear -> ExpertThresholdRouter (routing + EMA) ->
dispatch_autograd -> per-expert FFNs over the CSR blocks -> combine_autograd,
then backward into the input, the router weight and the expert weights.

The check is a float64 torch restatement of the same layer on the CPU: the
routed pairs are taken from the plan (selection is piecewise constant and has
no gradient), the gates are sigmoid(logits) at those pairs, and
y = sum over routed (t, e) of gate * FFN_e(x_t).  Outputs and every gradient
must agree within float32 rounding (relative to the magnitudes involved)."""
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


class TinyETMoE(torch.nn.Module):
    def __init__(self, et, d, E, h, k_target, dev):
        super().__init__()
        g = torch.Generator().manual_seed(3)
        self.et = et
        self.router = torch.nn.Linear(d, E, bias=False).to(dev)
        with torch.no_grad():
            self.router.weight.copy_(torch.randn(E, d, generator=g) * 0.3)
        self.w1 = torch.nn.Parameter((torch.randn(E, d, h, generator=g) * d ** -0.5).to(dev))
        self.w2 = torch.nn.Parameter((torch.randn(E, h, d, generator=g) * h ** -0.5).to(dev))
        self.thr = et.ExpertThresholdRouter(E, k_target, momentum=0.9, init_threshold=0.6, device=dev)

    def forward(self, x):
        logits = self.router(x)
        plan = self.thr(logits.detach().float().contiguous())
        xp = self.et.dispatch_autograd(x, plan)
        eo = plan.expert_offsets.tolist()
        outs = []
        for e in range(len(eo) - 1):
            rows = xp[eo[e]:eo[e + 1]]
            outs.append(torch.relu(rows @ self.w1[e]) @ self.w2[e])
        yp = torch.cat(outs).contiguous()
        return self.et.combine_autograd(yp, logits.float().contiguous(), plan), plan, logits


def reference(x, wr, w1, w2, plan):
    """float64 CPU restatement with the same routed pairs."""
    st = plan.sorted_token.long().cpu()
    ee = torch.repeat_interleave(torch.arange(len(plan.counts)), plan.counts.long().cpu())
    logits = x @ wr.T
    gate = torch.sigmoid(logits[st, ee])
    xs = x[st]
    hidden = torch.relu(torch.einsum("sd,sdh->sh", xs, w1[ee]))
    ys = torch.einsum("sh,shd->sd", hidden, w2[ee])
    return torch.zeros_like(x).index_add(0, st, gate[:, None] * ys)


@pytest.mark.parametrize("T,d,E,h,k", [(256, 64, 8, 32, 2), (300, 128, 16, 48, 4)])
def test_moe_layer_forward_backward_matches_float64(dev, T, d, E, h, k):
    et = importlib.import_module("peer-review-agents_amd")
    torch.manual_seed(0)
    layer = TinyETMoE(et, d, E, h, k, dev)
    layer.thr.eval()                               # fixed thresholds for this check
    x = torch.randn(T, d, device=dev, requires_grad=True)
    y, plan, _ = layer(x)
    dy = torch.randn(T, d, device=dev)
    y.backward(dy)

    xr = x.detach().cpu().double().requires_grad_(True)
    wr = layer.router.weight.detach().cpu().double().requires_grad_(True)
    w1 = layer.w1.detach().cpu().double().requires_grad_(True)
    w2 = layer.w2.detach().cpu().double().requires_grad_(True)
    yr = reference(xr, wr, w1, w2, plan)
    yr.backward(dy.cpu().double())

    def close(a, b, name):
        a = a.detach().cpu().double()
        scale = b.abs().max().item() + 1e-12
        err = (a - b.detach()).abs().max().item()
        assert err <= 2e-5 * scale, f"{name}: max error {err:.3e} vs scale {scale:.3e}"

    close(y, yr, "y")
    close(x.grad, xr.grad, "dX")
    close(layer.router.weight.grad, wr.grad, "dW_router")
    close(layer.w1.grad, w1.grad, "dW1")
    close(layer.w2.grad, w2.grad, "dW2")


def test_moe_layer_trains_with_ema_thresholds(dev):
    """A few SGD steps: the EMA moves the thresholds toward the k_target-th
    score, every token keeps at least one expert, and the loss is finite."""
    et = importlib.import_module("peer-review-agents_amd")
    T, d, E, h, k = 512, 64, 8, 32, 2
    layer = TinyETMoE(et, d, E, h, k, dev)
    layer.train()
    opt = torch.optim.SGD(layer.parameters(), lr=1e-2)
    g = torch.Generator(device=dev).manual_seed(1)
    thr0 = layer.thr.thr.clone()
    for step in range(5):
        x = torch.randn(T, d, device=dev, generator=g)
        y, plan, _ = layer(x)
        loss = (y.float() ** 2).mean()
        opt.zero_grad()
        loss.backward()
        opt.step()
        assert torch.isfinite(loss)
        assert int(torch.diff(plan.token_offsets).min()) >= 1
    assert not torch.equal(thr0, layer.thr.thr)
    assert bool(((layer.thr.thr > 0) & (layer.thr.thr < 1)).all())
