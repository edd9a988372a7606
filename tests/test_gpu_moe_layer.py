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


def test_manual_bf16_training_step_with_router_kernels(dev):
    """A bf16 training step with the router on this library's kernels, the way a
    fused training loop calls them (no autograd through the path):
      router_logits -> route -> dispatch -> expert FFNs (torch) -> combine;
      combine_backward -> FFN backward (torch) -> dispatch_backward with the
      router's input gradient -> router_weight_grad.
    Output, dX and dW_router against a float64 restatement with the same routed
    pairs; the bar is the bf16 one (each bf16 rounding on the path is 2^-9)."""
    et = importlib.import_module("peer-review-agents_amd")
    T, d, E, h = 512, 128, 16, 64
    g = torch.Generator().manual_seed(7)
    bf = torch.bfloat16
    X = (torch.randn(T, d, generator=g)).to(bf).to(dev)
    Wr = (torch.randn(E, d, generator=g) * d ** -0.5).to(bf).to(dev)
    w1 = (torch.randn(E, d, h, generator=g) * d ** -0.5).to(dev)
    w2 = (torch.randn(E, h, d, generator=g) * h ** -0.5).to(dev)
    dy = (torch.randn(T, d, generator=g) * 0.1).to(bf).to(dev)

    logits = et.router_logits(X, Wr)
    thr = torch.quantile(torch.sigmoid(logits.double()), 0.8, dim=0).float().contiguous()
    plan = et.route(logits, thr)
    xp = et.dispatch(X, plan)
    eo = plan.expert_offsets.tolist()
    xpf = xp.float().requires_grad_(True)
    yp_parts = [torch.relu(xpf[eo[e]:eo[e + 1]] @ w1[e]) @ w2[e] for e in range(E)]
    ypf = torch.cat(yp_parts)
    yp = ypf.detach().to(bf).contiguous()
    y = et.combine(yp, plan)
    dyp, dgate, dlogits = et.combine_backward(dy, yp, plan, need_dlogits=True)
    (dxpf,) = torch.autograd.grad(ypf, xpf, grad_outputs=dyp.float())
    dx = et.dispatch_backward(dxpf.to(bf).contiguous(), plan, router_weight=Wr, dgate=dgate)
    dwr = et.router_weight_grad(dlogits, X)

    # float64 restatement on the bf16 inputs, same routed pairs
    st = plan.sorted_token.long().cpu()
    ee = torch.repeat_interleave(torch.arange(E), plan.counts.long().cpu())
    xr = X.cpu().double().requires_grad_(True)
    wr = Wr.cpu().double().requires_grad_(True)
    lg = xr @ wr.T
    gate = torch.sigmoid(lg[st, ee])
    xs = xr[st]
    hid = torch.relu(torch.einsum("sd,sdh->sh", xs, w1.cpu().double()[ee]))
    ys = torch.einsum("sh,shd->sd", hid, w2.cpu().double()[ee])
    yr = torch.zeros(T, d, dtype=torch.float64).index_add(0, st, gate[:, None] * ys)
    yr.backward(dy.cpu().double())

    def close(a, b, name, rel):
        a = a.detach().cpu().double()
        scale = b.abs().max().item() + 1e-12
        err = (a - b.detach()).abs().max().item()
        assert err <= rel * scale, f"{name}: max error {err:.3e} vs scale {scale:.3e}"

    close(y, yr, "y", 2e-2)
    close(dx, xr.grad, "dX", 3e-2)
    close(dwr, wr.grad, "dW_router", 3e-2)


def test_bf16_moe_layer_entirely_on_library_kernels(dev):
    """A bf16 SwiGLU-expert MoE layer with every GEMM and data movement on this
    library's kernels, the way a fused training step would run it:
      forward:  router_logits -> route -> expert_gemm(X, W1) gathered (the
                dispatch fused) -> SwiGLU -> expert_gemm(., W2) -> combine;
      backward: combine_backward (dgate, dlogits, dYp) ->
                expert_gemm_input_grad(dY, W2) gathered, rows times the slot
                gate (the down projection's input gradient fused with the
                combine backward) -> swiglu_backward on the kept gu ->
                expert_gemm_input_grad(dGU, W1) -> dispatch_backward with the
                router's input gradient; expert_gemm_weight_grad for W1 and W2
                (the gathered operand dispatched once), router_weight_grad.
    Output and every gradient against a float64 restatement with the same
    routed pairs, at the bf16 bar (several bf16 roundings on the path)."""
    et = importlib.import_module("peer-review-agents_amd")
    T, d, E, F = 1024, 256, 16, 128
    g = torch.Generator().manual_seed(11)
    bf = torch.bfloat16
    X = torch.randn(T, d, generator=g).to(bf).to(dev)
    Wr = (torch.randn(E, d, generator=g) * d ** -0.5).to(bf).to(dev)
    W1 = (torch.randn(E, 2 * F, d, generator=g) * d ** -0.5).to(bf).to(dev)     # gate rows, then up rows
    W2 = (torch.randn(E, d, F, generator=g) * F ** -0.5).to(bf).to(dev)
    dy = (torch.randn(T, d, generator=g) * 0.1).to(bf).to(dev)

    logits = et.router_logits(X, Wr)
    thr = torch.quantile(torch.sigmoid(logits.double()), 0.8, dim=0).float().contiguous()
    plan = et.route(logits, thr)
    gu = et.expert_gemm(X, W1, plan)                       # [S, 2F] pre-activations
    hact = et.expert_gemm(X, W1, plan, epilogue="swiglu")   # [S, F], fused activation
    yp = et.expert_gemm(hact, W2, plan, gather=False)
    y = et.combine(yp, plan)

    dyp, dgate, dlogits = et.combine_backward(dy, yp, plan, need_dlogits=True)
    dh = et.expert_gemm_input_grad(dy, W2, plan, gather=True, row_scale=plan.slot_gate)
    dgu = et.swiglu_backward(gu, dh, plan)
    # the training forward's activation (from the kept, rounded gu) is within
    # one bf16 rounding of the fused epilogue's (from the binary32 accumulators)
    htrain = et.swiglu(gu, plan).float()
    assert (htrain - hact.float()).abs().max().item() <= 2 ** -7 * hact.float().abs().max().item()
    dxp = et.expert_gemm_input_grad(dgu, W1, plan)
    dx = et.dispatch_backward(dxp, plan, router_weight=Wr, dgate=dgate)
    dW1 = et.expert_gemm_weight_grad(dgu, et.dispatch(X, plan), plan)
    dW2 = et.expert_gemm_weight_grad(dyp, hact, plan)
    dWr = et.router_weight_grad(dlogits, X)

    st = plan.sorted_token.long().cpu()
    ee = torch.repeat_interleave(torch.arange(E), plan.counts.long().cpu())
    xr = X.cpu().double().requires_grad_(True)
    wr = Wr.cpu().double().requires_grad_(True)
    w1 = W1.cpu().double().requires_grad_(True)
    w2 = W2.cpu().double().requires_grad_(True)
    gate = torch.sigmoid((xr @ wr.T)[st, ee])
    pre = torch.bmm(w1[ee], xr[st].unsqueeze(2)).squeeze(2)                  # [S, 2F]
    act = torch.nn.functional.silu(pre[:, :F]) * pre[:, F:]
    ys = torch.bmm(w2[ee], act.unsqueeze(2)).squeeze(2)                     # [S, d]
    yr = torch.zeros(T, d, dtype=torch.float64).index_add(0, st, gate[:, None] * ys)
    yr.backward(dy.cpu().double())

    def close(a, b, name, rel):
        a = a.detach().cpu().double()
        scale = b.abs().max().item() + 1e-12
        err = (a - b.detach()).abs().max().item()
        assert err <= rel * scale, f"{name}: max error {err:.3e} vs scale {scale:.3e}"

    close(y, yr, "y", 2e-2)
    close(dx, xr.grad, "dX", 3e-2)
    close(dW1, w1.grad, "dW1", 3e-2)
    close(dW2, w2.grad, "dW2", 3e-2)
    close(dWr, wr.grad, "dW_router", 3e-2)
