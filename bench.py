"""Benchmark: fwd+bwd Expert-Threshold MoE dispatch/combine on one MI355X.

One step = one pass of the path over one batch of synthetic input, inputs
resident in HBM before timing starts:
    route            threshold routing + CSR + permutation (3 kernels)
    dispatch_fwd     Xp = permute(X)
    combine_fwd      Y  = sum_s gate[s] * Yp[s]
    combine_bwd      dYp = gate * dY[token], dgate = <dY, Yp>, dlogits (router grad)
    dispatch_bwd     dX = sum_s dXp[s]
The router producer (router logits GEMM, fused producer + routing) and its
backward (dispatch backward with the router input gradient, router weight
gradient) are measured separately after the timed steps and reported in
"router_producer" and "router_backward"; so is the expert grouped GEMM that
consumes the dispatch ("expert_gemm": the gate/up projection with the dispatch
fused into its operand load, also on fp8 e4m3 operands, the down projection,
the backward, and torch's grouped GEMM on the same shapes).
Yp and dXp are separate resident buffers standing in for the expert FFN's
output and input-gradient (the FFN itself is not part of the path).

Metric: routed token-slots per second, and the step's algorithmic HBM bytes
per second as a fraction of MI355X's 8 TB/s.  Workload: C3 (T=65536, d=4096,
E=128, bf16, Zipf-skewed expert popularity) unless --workload says otherwise.

Prints ONE JSON line on stdout (rank 0); a readable breakdown goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12   # MI355X HBM3E, bytes/s
METRIC = "routed token-slots/sec fwd+bwd dispatch+combine; % of HBM peak (8 TB/s)"
STAGES = ["route", "dispatch_fwd", "combine_fwd", "combine_bwd", "dispatch_bwd"]


def algorithmic_bytes(T: int, E: int, S: int, d: int, b: int) -> dict:
    """Minimum HBM bytes each stage must move (each element read or written once)."""
    idx = 4
    return {
        # read logits once; write counts/offsets, token_offsets, 3 slot arrays
        "route": T * E * 4 + (2 * E + 1) * idx + (T + 1) * idx + 3 * S * idx,
        # read X, token_offsets, token_slot; write Xp
        "dispatch_fwd": T * d * b + S * d * b + (T + 1) * idx + S * idx,
        # read Yp, gates, token_offsets, token_slot; write Y
        "combine_fwd": S * d * b + T * d * b + S * 4 + (T + 1) * idx + S * idx,
        # read dY, Yp, gates, offsets, token_slot, expert_offsets; write dYp, dgate, dlogits
        "combine_bwd": T * d * b + 2 * S * d * b + 2 * S * 4 + (T + 1) * idx + S * idx
                       + (E + 1) * idx + T * E * 4,
        # read dXp, offsets, token_slot; write dX
        "dispatch_bwd": S * d * b + T * d * b + (T + 1) * idx + S * idx,
    }


def read_traffic(workload: str):
    """Measured HBM bytes of one et_combine_bwd call (its kernels), from the
    committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, calibrated), if
    one exists for the workload."""
    path = os.path.join(ROOT, "profiles", f"pmc_combine_bwd_{workload}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def copy_ceiling(dev, stream, nbytes: int = 1 << 30, reps: int = 5) -> dict:
    """Bandwidth of a plain streaming kernel on this GPU, measured in the same
    run: torch's elementwise ``x * 1`` over ``nbytes`` of int32 in and ``nbytes``
    out (each byte read once and written once), timed with events on ``stream``.
    It is also the known-size kernel that calibrates the FETCH_SIZE and
    WRITE_SIZE counters in a ``rocprofv3 --pmc`` run of this script."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    torch.mul(src, 1, out=dst)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(reps):
        torch.mul(src, 1, out=dst)
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    del src, dst
    return {"kernel": "torch elementwise x*1 (int32)", "bytes": 2 * nbytes, "ms": round(ms, 4),
            "GB/s": round(2 * nbytes / (ms * 1e-3) / 1e9, 1),
            "frac": round(2 * nbytes / (ms * 1e-3) / HBM_PEAK, 4)}


def threshold_dynamics(et, W, dev, stream, workload: str, seed: int) -> dict:
    """Routing-only loop of a workload whose thresholds follow the EMA (C5):
    per step, route a fresh logits batch with the current thresholds (fixed
    slot capacity, no host sync) and apply the EMA update.  Logits are
    generated on the device beforehand; the step count is the workload's."""
    import torch
    cfg = W.CONFIGS[workload]
    T, E, steps = cfg["T"], cfg["E"], cfg["steps"]
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 17)
    logits = [torch.randn(T, E, device=dev, generator=g) for _ in range(steps)]
    thr = torch.full((E,), cfg["thr0"], dtype=torch.float32, device=dev)
    cap = T * E
    rws = torch.empty(et.route_workspace_bytes(T, E), dtype=torch.uint8, device=dev)
    tws = torch.empty(et.threshold_workspace_bytes(T, E), dtype=torch.uint8, device=dev)
    stat = torch.empty(E, dtype=torch.float32, device=dev)
    plan = et.route(logits[0], thr, slot_capacity=cap, workspace=rws)       # warm-up
    et.threshold_update_(thr.clone(), logits[0], cfg["k_target"], cfg["momentum"], stat=stat, workspace=tws)
    # Events on the stream, no host synchronisation inside the loop (the host
    # runs ahead, so each interval is the kernels' own time on the GPU).
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    slots = []
    for i in range(steps):
        ev[i][0].record(stream)
        plan = et.route(logits[i], thr, slot_capacity=cap, workspace=rws)
        ev[i][1].record(stream)
        et.threshold_update_(thr, logits[i], cfg["k_target"], cfg["momentum"], stat=stat, workspace=tws)
        ev[i][2].record(stream)
        slots.append(plan.expert_offsets[E:E + 1])
    torch.cuda.synchronize()
    r_ms = sum(e[0].elapsed_time(e[1]) for e in ev)
    u_ms = sum(e[1].elapsed_time(e[2]) for e in ev)
    k = [int(x) / T for x in slots]
    thr_eager = thr.clone()
    # All steps captured in one HIP graph and replayed once from the start
    # thresholds: the final thresholds must equal the eager loop's bit for bit.
    thr.fill_(cfg["thr0"])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            et.route(logits[i], thr, slot_capacity=cap, workspace=rws)
            et.threshold_update_(thr, logits[i], cfg["k_target"], cfg["momentum"], stat=stat, workspace=tws)
    thr.fill_(cfg["thr0"])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    g_ms = (time.perf_counter() - t0) * 1e3 / steps
    if not torch.equal(thr, thr_eager):
        raise RuntimeError("graph-replayed threshold dynamics differ from the eager loop")
    del graph
    # The same loop through et_route_update (routing, then the EMA update, in
    # one call).
    def combined():
        for i in range(steps):
            et.route_update(logits[i], thr, cfg["k_target"], cfg["momentum"], slot_capacity=cap, stat=stat,
                            workspace=rws, thr_workspace=tws)
    thr.fill_(cfg["thr0"])
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    combined()
    b.record(stream)
    torch.cuda.synchronize()
    c_ms = a.elapsed_time(b) / steps
    if not torch.equal(thr, thr_eager):
        raise RuntimeError("route_update threshold dynamics differ from the eager loop")
    thr.fill_(cfg["thr0"])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        combined()
    thr.fill_(cfg["thr0"])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    cg_ms = (time.perf_counter() - t0) * 1e3 / steps
    if not torch.equal(thr, thr_eager):
        raise RuntimeError("graph-replayed route_update dynamics differ from the eager loop")
    del graph
    return {"steps": steps, "T": T, "E": E, "route_ms": round(r_ms / steps, 4),
            "ema_update_ms": round(u_ms / steps, 4), "mean_k_first_step": round(k[0], 4),
            "mean_k_last_step": round(k[-1], 4), "k_target": cfg["k_target"],
            "graph_replay_ms_per_step": round(g_ms, 4), "route_update_ms": round(c_ms, 4),
            "route_update_graph_replay_ms_per_step": round(cg_ms, 4)}


def router_producer(et, dev, stream, X, E: int, reps: int = 10) -> dict:
    """The router producer on the workload's resident activations X (bf16):
    logits = X W^T (router_logits_kernel), the fused producer + routing
    (et_router_route, scores never written) against router_logits followed by
    et_route, and torch's bf16 linear as a library reference.  Measured with
    HIP events on the stream the kernels run on, outside the timed step."""
    import torch
    T, d = X.shape
    g = torch.Generator(device=dev)
    g.manual_seed(4242)
    Wr = (torch.randn(E, d, device=dev, generator=g) * d ** -0.5).to(torch.bfloat16)
    L = et.router_logits(X, Wr)
    q = max(0.0, 1.0 - 8.0 / E)
    thr = torch.quantile(torch.sigmoid(L[:8192].double()), q, dim=0).float().contiguous()
    cap = et.route(L, thr).num_slots + 4096
    rws = torch.empty(et.route_workspace_bytes(T, E), dtype=torch.uint8, device=dev)
    fws = torch.empty(et.router_route_workspace_bytes(T, E), dtype=torch.uint8, device=dev)

    def timed(fn):
        for _ in range(2):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    t_gemm = timed(lambda: et.router_logits(X, Wr, out=L))
    t_route = timed(lambda: et.route(L, thr, slot_capacity=cap, workspace=rws))
    t_fused = timed(lambda: et.router_route(X, Wr, thr, slot_capacity=cap, workspace=fws))
    t_torch = timed(lambda: torch.nn.functional.linear(X, Wr))
    nbytes = T * d * 2 + E * d * 2 + T * E * 4
    gbs = nbytes / (t_gemm * 1e-6) / 1e9
    return {"kernel": "router_logits_kernel", "T": T, "d": d, "E": E, "us": round(t_gemm, 2),
            "algorithmic_bytes": nbytes, "GB/s": round(gbs, 1), "frac": round(gbs * 1e9 / HBM_PEAK, 4),
            "TFLOP/s": round(2.0 * T * d * E / (t_gemm * 1e-6) / 1e12, 1),
            "fused_route_us": round(t_fused, 2), "logits_then_route_us": round(t_gemm + t_route, 2),
            "torch_linear_bf16_us": round(t_torch, 2)}


def router_backward(et, dev, stream, plan, X, DXP, DGATE, DL, reps: int = 10) -> dict:
    """The router producer's backward on the workload's step buffers: the
    dispatch backward with the router's input gradient fused in (against the
    plain dispatch backward), and the router weight gradient dW = dlogits^T X
    (against torch's float32 matmul).  Measured after the timed step."""
    import torch
    T, d = X.shape
    E = plan.num_experts
    g = torch.Generator(device=dev)
    g.manual_seed(4243)
    Wr = (torch.randn(E, d, device=dev, generator=g) * d ** -0.5).to(X.dtype)
    dx = torch.empty(T, d, dtype=X.dtype, device=dev)
    ws = torch.empty(max(1, int(et.lib().et_dispatch_bwd_router_workspace_bytes(plan.rows))), dtype=torch.uint8,
                     device=dev)
    dw = torch.empty(E, d, dtype=torch.float32, device=dev)
    wws = torch.empty(max(16, int(et.lib().et_router_wgrad_workspace_bytes(T, d, E))), dtype=torch.uint8,
                      device=dev)

    def timed(fn):
        for _ in range(2):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    t_plain = timed(lambda: et.dispatch_backward(DXP, plan, out=dx))
    t_fused = timed(lambda: et.dispatch_backward(DXP, plan, out=dx, router_weight=Wr, dgate=DGATE, workspace=ws))
    out = {"dispatch_bwd_us": round(t_plain, 2), "dispatch_bwd_router_us": round(t_fused, 2)}
    if X.dtype == torch.bfloat16 and E <= 256:
        t_wg = timed(lambda: et.router_weight_grad(DL, X, out=dw, workspace=wws))
        t_torch = timed(lambda: torch.mm(DL.t(), X.float()))
        nbytes = T * d * 2 + T * E * 4 + E * d * 4
        gbs = nbytes / (t_wg * 1e-6) / 1e9
        out.update({"router_wgrad_us": round(t_wg, 2), "router_wgrad_GB/s": round(gbs, 1),
                    "router_wgrad_frac": round(gbs * 1e9 / HBM_PEAK, 4),
                    "torch_mm_f32_wgrad_us": round(t_torch, 2)})
    return out


EXPERT_FFN = 1536          # expert FFN width of the gate/up and down projections (Qwen3-MoE's, d = 4096, E = 128)
MFMA_BF16_PEAK = 2.5e15   # MI355X dense bf16 matrix peak, FLOP/s
MFMA_FP8_PEAK = 5.0e15    # MI355X dense fp8 matrix peak, FLOP/s


def expert_gemm_leg(et, dev, stream, plan, X, reps: int = 3) -> dict:
    """The expert grouped GEMM on the workload's routing: the gate/up projection
    (K = d, N = 2 * EXPERT_FFN) straight from X with the dispatch fused into the
    operand load, and the down projection (K = EXPERT_FFN, N = d) on a
    slot-major operand, each against torch's grouped GEMM (hipBLASLt) -- which
    needs the dispatched Xp, so the dispatch is timed beside it.  The gate/up
    projection is also timed with the SwiGLU epilogue (half the output), and
    the backward of both projections: the input gradients (the down one fused
    with the combine backward) and the f32 weight gradients, and the
    element-wise SwiGLU for training (forward and backward).  Random-init
    expert weights of that shape; measured after the timed step with HIP events
    on the stream the kernels run on."""
    import torch
    T, d = X.shape
    E, S, F = plan.num_experts, plan.rows, EXPERT_FFN
    g = torch.Generator(device=dev)
    g.manual_seed(4244)
    w1 = (torch.randn(E, 2 * F, d, device=dev, generator=g) * d ** -0.5).to(torch.bfloat16)
    w2 = (torch.randn(E, d, F, device=dev, generator=g) * F ** -0.5).to(torch.bfloat16)
    h = torch.empty(S, 2 * F, dtype=torch.bfloat16, device=dev)
    a2 = torch.randn(S, F, device=dev, generator=g).to(torch.bfloat16)
    y = torch.empty(S, d, dtype=torch.bfloat16, device=dev)
    xp = et.dispatch(X, plan)
    offs = plan.expert_offsets[1:].contiguous()

    def timed(fn):
        fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    t_up = timed(lambda: et.expert_gemm(X, w1, plan, out=h))
    hs = torch.empty(S, F, dtype=torch.bfloat16, device=dev)
    t_up_swiglu = timed(lambda: et.expert_gemm(X, w1, plan, epilogue="swiglu", out=hs))
    del hs
    # the same projection on fp8 e4m3 operands, each row of X and of the
    # weight scaled by its amax / 448 (the binary32 scales are applied in the
    # epilogue); its distance from the bf16 product is the quantization's
    xsc = X.float().abs().amax(1).clamp_min(1e-30) / 448.0
    xq = (X.float() / xsc[:, None]).to(torch.float8_e4m3fn)
    w1sc = torch.empty(E, 2 * F, dtype=torch.float32, device=dev)
    w1q = torch.empty(E, 2 * F, d, dtype=torch.float8_e4m3fn, device=dev)
    for e in range(E):
        we = w1[e].float()
        w1sc[e] = we.abs().amax(1).clamp_min(1e-30) / 448.0
        w1q[e] = (we / w1sc[e][:, None]).to(torch.float8_e4m3fn)
        del we
    h8 = torch.empty(S, 2 * F, dtype=torch.bfloat16, device=dev)
    t_up8 = timed(lambda: et.expert_gemm_fp8(xq, xsc, w1q, w1sc, plan, out=h8))
    hs8 = torch.empty(S, F, dtype=torch.bfloat16, device=dev)
    t_up8_swiglu = timed(lambda: et.expert_gemm_fp8(xq, xsc, w1q, w1sc, plan, epilogue="swiglu", out=hs8))
    torch.cuda.synchronize()
    nr = min(S, 65536)
    rel8 = ((h8[:nr].float() - h[:nr].float()).norm() / h[:nr].float().norm()).item()
    del xq, xsc, w1q, w1sc, h8, hs8
    t_down = timed(lambda: et.expert_gemm(a2, w2, plan, gather=False, out=y))
    # the down projection on fp8 operands (slot-major: one scale per slot row)
    a2sc = a2.float().abs().amax(1).clamp_min(1e-30) / 448.0
    a2q = (a2.float() / a2sc[:, None]).to(torch.float8_e4m3fn)
    w2f = w2.float()
    w2sc = w2f.abs().amax(2).clamp_min(1e-30) / 448.0
    w2q = (w2f / w2sc[:, :, None]).to(torch.float8_e4m3fn)
    del w2f
    y8 = torch.empty_like(y)
    t_down8 = timed(lambda: et.expert_gemm_fp8(a2q, a2sc, w2q, w2sc, plan, gather=False, out=y8))
    torch.cuda.synchronize()
    rel8_down = ((y8[:nr].float() - y[:nr].float()).norm() / y[:nr].float().norm()).item()
    del a2q, a2sc, w2q, w2sc, y8
    t_disp = timed(lambda: et.dispatch(X, plan, out=xp))
    w1t, w2t = w1.transpose(1, 2), w2.transpose(1, 2)
    t_up_lib = timed(lambda: torch._grouped_mm(xp, w1t, offs=offs))
    t_down_lib = timed(lambda: torch._grouped_mm(a2, w2t, offs=offs))
    fl_up, fl_down = 2.0 * S * d * 2 * F, 2.0 * S * F * d
    # backward: the down projection's input gradient fused with the combine
    # backward (dY gathered, rows times the slot gate), the gate/up
    # projection's input gradient (both through the transposed weights of the
    # experts with slots), and both weight gradients (f32)
    dy = torch.randn(T, d, device=dev, generator=g).to(torch.bfloat16)
    dgu = torch.randn(S, 2 * F, device=dev, generator=g).to(torch.bfloat16)
    w2t = torch.empty(E, F, d, dtype=torch.bfloat16, device=dev)
    w1t = torch.empty(E, d, 2 * F, dtype=torch.bfloat16, device=dev)
    dh = torch.empty(S, F, dtype=torch.bfloat16, device=dev)
    dxp = torch.empty(S, d, dtype=torch.bfloat16, device=dev)
    t_tr2 = timed(lambda: et.expert_weight_transpose(w2, plan, out=w2t))
    t_down_bwd = timed(lambda: et.expert_gemm_input_grad(dy, w2, plan, gather=True, row_scale=plan.slot_gate,
                                                          wt=w2t, out=dh))
    t_up_bwd = timed(lambda: et.expert_gemm_input_grad(dgu, w1, plan, wt=w1t, out=dxp))
    # the activation for training, on the kept gate/up output h (HBM-bound:
    # 6F bytes per slot forward, 10F backward)
    hs = torch.empty(S, F, dtype=torch.bfloat16, device=dev)
    dgu2 = torch.empty(S, 2 * F, dtype=torch.bfloat16, device=dev)
    t_sw = timed(lambda: et.swiglu(h, plan, out=hs))
    t_sw_bwd = timed(lambda: et.swiglu_backward(h, dh, plan, out=dgu2))
    del hs, dgu2
    sw_gbs = 6.0 * F * S / (t_sw * 1e-3) / 1e9
    sw_bwd_gbs = 10.0 * F * S / (t_sw_bwd * 1e-3) / 1e9
    dw1 = torch.empty(E, 2 * F, d, dtype=torch.float32, device=dev)
    t_wg_up = timed(lambda: et.expert_gemm_weight_grad(dgu, xp, plan, out=dw1))
    del dw1
    dyp = torch.randn(S, d, device=dev, generator=g).to(torch.bfloat16)
    dw2 = torch.empty(E, d, F, dtype=torch.float32, device=dev)
    t_wg_down = timed(lambda: et.expert_gemm_weight_grad(dyp, a2, plan, out=dw2))
    del dw2
    try:      # torch's grouped GEMM in its weight-gradient form (sum over each group's rows)
        t_wg_up_lib = timed(lambda: torch._grouped_mm(dgu.t(), xp, offs=offs))
    except RuntimeError:
        t_wg_up_lib = None
    fl_wg_up = 2.0 * S * 2 * F * d
    del w1, w2, h, a2, y, xp, dy, dgu, w2t, w1t, dh, dxp, dyp
    return {"kernel": "expert_gemm_kernel", "expert_ffn": F,
            "gate_up": {"K": d, "N": 2 * F, "mode": "gather (dispatch fused)", "ms": round(t_up, 3),
                        "TFLOP/s": round(fl_up / (t_up * 1e-3) / 1e12, 1),
                        "frac": round(fl_up / (t_up * 1e-3) / MFMA_BF16_PEAK, 4),
                        "torch_grouped_mm_ms": round(t_up_lib, 3), "dispatch_ms": round(t_disp, 3),
                        "torch_dispatch_plus_grouped_mm_ms": round(t_disp + t_up_lib, 3),
                        "swiglu_epilogue_ms": round(t_up_swiglu, 3)},
            "gate_up_fp8": {"K": d, "N": 2 * F, "mode": "gather (dispatch fused)", "operands": "e4m3, row scales",
                            "ms": round(t_up8, 3), "TFLOP/s": round(fl_up / (t_up8 * 1e-3) / 1e12, 1),
                            "frac": round(fl_up / (t_up8 * 1e-3) / MFMA_FP8_PEAK, 4),
                            "swiglu_epilogue_ms": round(t_up8_swiglu, 3),
                            "relative_error_vs_bf16": round(rel8, 4)},
            "down": {"K": F, "N": d, "mode": "slot-major", "ms": round(t_down, 3),
                     "TFLOP/s": round(fl_down / (t_down * 1e-3) / 1e12, 1),
                     "frac": round(fl_down / (t_down * 1e-3) / MFMA_BF16_PEAK, 4),
                     "torch_grouped_mm_ms": round(t_down_lib, 3)},
            "down_fp8": {"K": F, "N": d, "mode": "slot-major", "operands": "e4m3, row scales",
                         "ms": round(t_down8, 3), "TFLOP/s": round(fl_down / (t_down8 * 1e-3) / 1e12, 1),
                         "frac": round(fl_down / (t_down8 * 1e-3) / MFMA_FP8_PEAK, 4),
                         "relative_error_vs_bf16": round(rel8_down, 4)},
            "backward": {"weight_transpose_down_ms": round(t_tr2, 3),
                         "down_input_grad_fused_combine_bwd_ms": round(t_down_bwd, 3),
                         "gate_up_input_grad_ms": round(t_up_bwd, 3),
                         "gate_up_weight_grad_ms": round(t_wg_up, 3),
                         "gate_up_weight_grad_TFLOP/s": round(fl_wg_up / (t_wg_up * 1e-3) / 1e12, 1),
                         "down_weight_grad_ms": round(t_wg_down, 3),
                         "torch_grouped_mm_gate_up_weight_grad_ms": (round(t_wg_up_lib, 3) if t_wg_up_lib
                                                                     else None)},
            "swiglu": {"forward_ms": round(t_sw, 3), "forward_GB/s": round(sw_gbs, 1),
                       "forward_frac": round(sw_gbs * 1e9 / HBM_PEAK, 4), "backward_ms": round(t_sw_bwd, 3),
                       "backward_GB/s": round(sw_bwd_gbs, 1),
                       "backward_frac": round(sw_bwd_gbs * 1e9 / HBM_PEAK, 4)}}


def load_shape(counts, token_offsets) -> dict:
    """Per-token expert counts (k) and per-expert loads of a routing, from its
    counts [E] and token_offsets [T+1] (host arrays)."""
    import numpy as np
    k = np.diff(np.asarray(token_offsets, np.int64))
    c = np.sort(np.asarray(counts, np.int64))[::-1]
    hist = np.bincount(k)
    nz = c[c > 0]
    return {"k_hist": {str(i): int(n) for i, n in enumerate(hist) if n},
            "k_min": int(k.min()), "k_max": int(k.max()), "k_mean": round(float(k.mean()), 4),
            "k_std": round(float(k.std()), 4),
            "expert_load": {"max": int(c[0]), "median": int(np.median(c)), "min": int(c[-1]),
                            "empty_experts": int((c == 0).sum()),
                            "max_over_min_nonempty": round(float(nz[0] / nz[-1]), 2) if nz.size else None,
                            "top8_share": round(float(c[:8].sum() / max(1, c.sum())), 4)}}


def cpu_baseline(workload: str, step, reps: int = 3) -> dict:
    """The CPU restatement (oracle/, C with OpenMP) timed on this host's cores
    on the whole workload, on the very inputs of the GPU step (copied from the
    device): route, dispatch, combine, combine backward with dlogits, dispatch
    backward -- the five operations of one GPU step -- into preallocated
    outputs.  One untimed warm-up pass (it also faults the output pages in),
    then the median of `reps` timed passes.  Threads: OMP_NUM_THREADS if set
    (the GPU box sets it to the CPU share of one GPU), else every core of this
    process's affinity mask.  The CPU outputs are then compared with the GPU
    step's: routing, Xp, Y, dYp, dX and dlogits bit for bit, dgate within one
    binary32 ulp plus the binary64 summation floor."""
    import numpy as np
    import oracle
    nproc = len(os.sched_getaffinity(0))
    want = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or nproc
    threads = oracle.set_threads(want)
    T, d, E, S = step.T, step.d, step.E, step.S
    u16 = lambda t: t.view(torch_mod().int16).cpu().numpy().view(np.uint16)  # noqa: E731
    host = (lambda t: u16(t)) if step.act_bits == 16 else (lambda t: t.cpu().numpy())
    lg, thr = step.logits.cpu().numpy(), step.thr.cpu().numpy()
    x, yp, dy, dxp = host(step.X), host(step.YP), host(step.DY), host(step.DXP)
    adt = x.dtype
    xp, y, dyp = np.empty((S, d), adt), np.empty((T, d), adt), np.empty((S, d), adt)
    dgate, dl, dx = np.empty(S, np.float32), np.empty((T, E), np.float32), np.empty((T, d), adt)

    def one_pass():
        r = oracle.route(lg, thr)
        oracle.dispatch_fwd(x, r, out=xp)
        oracle.combine_fwd(yp, r, T, out=y)
        oracle.combine_bwd(dy, yp, r, E, want_dlogits=True, out=(dyp, dgate, dl))
        oracle.dispatch_bwd(dxp, r, T, out=dx)
        return r

    t0 = time.perf_counter()
    r = one_pass()
    warm = time.perf_counter() - t0
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        r = one_pass()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))

    # full-size parity of the GPU step against these CPU outputs
    step.sync_outputs()
    bits_eq = lambda a, b: bool(np.array_equal(np.ascontiguousarray(a).view(np.uint8),  # noqa: E731
                                               np.ascontiguousarray(b).view(np.uint8)))
    gdg = step.DGATE.cpu().numpy().astype(np.float64)
    dyf = dy.astype(np.float64) if adt == np.float32 else oracle.bf16_to_f32(dy).astype(np.float64)
    ypf = yp.astype(np.float64) if adt == np.float32 else oracle.bf16_to_f32(yp).astype(np.float64)
    mass = np.empty(S)
    for a in range(0, S, 65536):              # sum_c |dY Yp| per slot, in blocks
        b_ = min(S, a + 65536)
        mass[a:b_] = np.abs(dyf[r.sorted_token[a:b_]] * ypf[a:b_]).sum(1)
    del dyf, ypf
    cdg = dgate.astype(np.float64)
    err = np.abs(gdg - cdg)
    parity = {
        "routing_bit_exact": all(bits_eq(step.host_plan[f], getattr(r, f)) for f in
                                 ("counts", "expert_offsets", "token_offsets", "sorted_token", "slot_gate",
                                  "token_slot")),
        "dispatch_bit_exact": bits_eq(host(step.XP), xp),
        "combine_bit_exact": bits_eq(host(step.Y), y),
        "combine_bwd_dyp_bit_exact": bits_eq(host(step.DYP), dyp),
        "dlogits_bit_exact": bits_eq(step.DL.cpu().numpy(), dl),
        "dispatch_bwd_bit_exact": bits_eq(host(step.DX), dx),
        "dgate_within_bar": bool(np.all(err <= 2.0 ** -23 * np.abs(cdg) + 2 * d * 2.0 ** -53 * mass)),
        "dgate_bit_equal_frac": round(float((gdg == cdg).mean()), 6),
        "dgate_max_rel": float((err / np.maximum(np.abs(cdg), 1e-300)).max()),
    }
    return {"value": round(S / med, 1), "unit": "slots/s", "cores": threads, "nproc": nproc,
            "kind": "port", "reps": reps, "rep_s": [round(t, 3) for t in times], "median_s": round(med, 4),
            "warmup_s": round(warm, 3),
            "sample": f"the whole {workload} step ({T} tokens, {S} slots, d={d}), on the GPU step's inputs: "
                      f"route, dispatch, combine, combine backward with dlogits, dispatch backward by the C "
                      f"oracle (OpenMP, {threads} threads of {nproc} in this process's CPU set), one warm-up "
                      f"pass then the median of {reps}",
            "full_size_parity_vs_gpu": parity}


def torch_mod():
    import torch
    return torch


class Step:
    """One workload's resident buffers and its five stages, called through the
    C ABI on one stream with the routed slot count as the slot capacity (so no
    stage synchronises with the host)."""

    def __init__(self, et, lib, dev, workload: str, seed: int):
        import torch
        W = importlib.import_module("peer-review-agents_amd.workloads")
        self.lib, self.dev, self.workload = lib, dev, workload
        cfg = W.CONFIGS[workload]
        self.cfg = cfg
        T, d, E = cfg["T"], cfg["d"], cfg["E"]
        self.T, self.d, self.E = T, d, E
        act = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
        self.act, self.b = act, (2 if act == torch.bfloat16 else 4)
        self.act_bits = 16 if act == torch.bfloat16 else 32
        self.dt_code = 1 if act == torch.bfloat16 else 0
        lg_h, thr_h = W.router_inputs(workload, seed=seed)
        self.logits = torch.from_numpy(lg_h).to(dev)
        self.thr = torch.from_numpy(thr_h).to(dev)
        plan = et.route(self.logits, self.thr)        # sizes the slot buffers (one sync, untimed)
        S = self.S = plan.num_slots
        self.shape = load_shape(plan.counts.cpu().numpy(), plan.token_offsets.cpu().numpy())
        del plan
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.X = torch.randn(T, d, device=dev, generator=g).to(act)
        self.YP = torch.randn(S, d, device=dev, generator=g).to(act)
        self.DY = (torch.randn(T, d, device=dev, generator=g) * 0.02).to(act)
        self.DXP = torch.randn(S, d, device=dev, generator=g).to(act)
        i32 = dict(dtype=torch.int32, device=dev)
        self.counts, self.eoff, self.toff = torch.empty(E, **i32), torch.empty(E + 1, **i32), torch.empty(T + 1, **i32)
        self.st, self.ts = torch.empty(S, **i32), torch.empty(S, **i32)
        self.sg = torch.empty(S, dtype=torch.float32, device=dev)
        self.wsb = et.route_workspace_bytes(T, E)
        self.ws = torch.empty(self.wsb, dtype=torch.uint8, device=dev)
        self.XP = torch.empty(S, d, dtype=act, device=dev)
        self.Y = torch.empty(T, d, dtype=act, device=dev)
        self.DYP = torch.empty(S, d, dtype=act, device=dev)
        self.DGATE = torch.empty(S, dtype=torch.float32, device=dev)
        self.DL = torch.empty(T, E, dtype=torch.float32, device=dev)
        self.DX = torch.empty(T, d, dtype=act, device=dev)
        self.bwsb = et.combine_backward_workspace_bytes(T, S, d, act)
        self.BWS = torch.empty(max(self.bwsb, 8), dtype=torch.uint8, device=dev)
        self.stream = torch.cuda.current_stream(dev)
        self.host_plan = None

    def stage(self, i, stream=None):
        vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        sp = ctypes.c_void_p((stream or self.stream).cuda_stream)
        L, T, E, d, S, dt = self.lib, self.T, self.E, self.d, self.S, self.dt_code
        if i == 0:
            rc = L.et_route(vp(self.logits), vp(self.thr), T, E, vp(self.counts), vp(self.eoff), vp(self.toff),
                            vp(self.st), vp(self.sg), vp(self.ts), S, vp(self.ws), self.wsb, sp)
        elif i == 1:
            rc = L.et_dispatch_fwd(vp(self.X), T, d, dt, vp(self.toff), vp(self.ts), S, vp(self.XP), sp)
        elif i == 2:
            rc = L.et_combine_fwd(vp(self.YP), vp(self.sg), vp(self.toff), vp(self.ts), T, d, dt, S, vp(self.Y), sp)
        elif i == 3:
            rc = L.et_combine_bwd(vp(self.DY), vp(self.YP), vp(self.sg), vp(self.st), vp(self.toff), vp(self.ts),
                                  vp(self.eoff), T, E, d, dt, S, vp(self.DYP), vp(self.DGATE), vp(self.DL),
                                  vp(self.BWS), self.bwsb, sp)
        else:
            rc = L.et_dispatch_bwd(vp(self.DXP), vp(self.toff), vp(self.ts), T, d, dt, S, vp(self.DX), sp)
        if rc != 0:
            raise RuntimeError(f"{self.workload} stage {STAGES[i]} failed: {L.et_last_error().decode()}")

    def timed(self, steps: int, warmup: int, stages) -> tuple:
        """Per-stage HIP-event milliseconds (averaged over `steps`) and the
        wall-clock milliseconds per step."""
        import torch
        if 0 not in stages:
            self.stage(0)                             # the routing the other stages read
        for _ in range(warmup):
            for i in stages:
                self.stage(i)
        torch.cuda.synchronize()
        if int(self.eoff[self.E]) != self.S:
            raise RuntimeError("routing changed between runs")
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(steps):
            ev[k][0].record(self.stream)
            for j, i in enumerate(stages):
                self.stage(i)
                ev[k][j + 1].record(self.stream)
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
        stage_ms = {STAGES[i]: sum(ev[k][j].elapsed_time(ev[k][j + 1]) for k in range(steps)) / steps
                    for j, i in enumerate(stages)}
        return stage_ms, wall_ms

    def graph_ms(self, stages, steps: int) -> float:
        """Milliseconds per step with the stages captured once in a HIP graph
        and replayed `steps` times: what a caller that captures the path sees
        where launches, not bytes, bound the step.  Every stage runs with an
        explicit slot capacity, so the capture holds no host synchronisation."""
        import torch
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cs = torch.cuda.current_stream(self.dev)
            for i in stages:
                self.stage(i, cs)
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        if int(self.eoff[self.E]) != self.S:
            raise RuntimeError("routing changed under graph replay")
        del graph
        return ms

    def sync_outputs(self):
        """Host copies of the routing outputs of the last step."""
        import torch
        torch.cuda.synchronize()
        self.host_plan = {"counts": self.counts.cpu().numpy(), "expert_offsets": self.eoff.cpu().numpy(),
                          "token_offsets": self.toff.cpu().numpy(), "sorted_token": self.st.cpu().numpy(),
                          "slot_gate": self.sg.cpu().numpy(), "token_slot": self.ts.cpu().numpy()}

    def summary(self, stages, stage_ms, wall_ms) -> dict:
        ab = algorithmic_bytes(self.T, self.E, self.S, self.d, self.b)
        nbytes = sum(ab[STAGES[i]] for i in stages)
        return {"workload": f"{self.workload}: T={self.T} d={self.d} E={self.E} {self.cfg['dtype']}, "
                            f"thresholds {self.cfg['thr']}",
                "stages": [STAGES[i] for i in stages], "slots": self.S, "mean_k": round(self.S / self.T, 4),
                "ms_per_step": round(wall_ms, 4), "slots_per_s": round(self.S / (wall_ms * 1e-3), 1),
                "algorithmic_bytes": nbytes, "hbm_frac": round(nbytes / (wall_ms * 1e-3) / HBM_PEAK, 4),
                "stage_ms": {k: round(v, 4) for k, v in stage_ms.items()}, "load_shape": self.shape}

    def release(self):
        for name in ("X", "YP", "DY", "DXP", "XP", "Y", "DYP", "DGATE", "DL", "DX", "BWS", "ws", "logits"):
            setattr(self, name, None)


def expert_gemm_brief(et, dev, stream, plan, X, reps: int = 3) -> dict:
    """The expert FFN's two projections on a workload's routing (gate/up with
    the dispatch fused, down slot-major), each against torch's grouped GEMM
    (hipBLASLt) plus, for gate/up, the dispatch torch needs.  Random-init
    weights of the FFN shape of the headline leg."""
    import torch
    T, d = X.shape
    E, S, F = plan.num_experts, plan.rows, EXPERT_FFN
    g = torch.Generator(device=dev)
    g.manual_seed(4245)
    w1 = (torch.randn(E, 2 * F, d, device=dev, generator=g) * d ** -0.5).to(torch.bfloat16)
    w2 = (torch.randn(E, d, F, device=dev, generator=g) * F ** -0.5).to(torch.bfloat16)
    h = torch.empty(S, 2 * F, dtype=torch.bfloat16, device=dev)
    a2 = torch.randn(S, F, device=dev, generator=g).to(torch.bfloat16)
    y = torch.empty(S, d, dtype=torch.bfloat16, device=dev)
    xp = et.dispatch(X, plan)
    offs = plan.expert_offsets[1:].contiguous()

    def timed(fn):
        fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    t_up = timed(lambda: et.expert_gemm(X, w1, plan, out=h))
    t_down = timed(lambda: et.expert_gemm(a2, w2, plan, gather=False, out=y))
    t_disp = timed(lambda: et.dispatch(X, plan, out=xp))
    w1t, w2t = w1.transpose(1, 2), w2.transpose(1, 2)
    t_up_lib = timed(lambda: torch._grouped_mm(xp, w1t, offs=offs))
    t_down_lib = timed(lambda: torch._grouped_mm(a2, w2t, offs=offs))
    fl_up, fl_down = 2.0 * S * d * 2 * F, 2.0 * S * F * d
    del w1, w2, h, a2, y, xp
    return {"expert_ffn": F,
            "gate_up_ms": round(t_up, 3), "gate_up_frac": round(fl_up / (t_up * 1e-3) / MFMA_BF16_PEAK, 4),
            "torch_grouped_mm_gate_up_ms": round(t_up_lib, 3), "dispatch_ms": round(t_disp, 3),
            "down_ms": round(t_down, 3), "down_frac": round(fl_down / (t_down * 1e-3) / MFMA_BF16_PEAK, 4),
            "torch_grouped_mm_down_ms": round(t_down_lib, 3)}


def extra_workload(et, lib, dev, workload: str, seed: int, stages, steps: int = 10, warmup: int = 3,
                   gemm: bool = False) -> dict:
    """A full-size step of another configuration, timed like the headline
    step (HIP events per stage, wall clock per step), its buffers freed after.
    With `gemm`, the expert FFN projections on its routing too."""
    import torch
    st = Step(et, lib, dev, workload, seed)
    stage_ms, wall_ms = st.timed(steps, warmup, stages)
    out = st.summary(stages, stage_ms, wall_ms)
    out["steps"] = steps
    g_ms = st.graph_ms(stages, steps)
    out["graph_replay"] = {"ms_per_step": round(g_ms, 4), "slots_per_s": round(st.S / (g_ms * 1e-3), 1),
                           "hbm_frac": round(out["algorithmic_bytes"] / (g_ms * 1e-3) / HBM_PEAK, 4)}
    if gemm and st.act == torch.bfloat16:
        plan = et.RoutingPlan(st.counts, st.eoff, st.toff, st.st, st.sg, st.ts, st.T, st.E, st.S, st.S)
        out["expert_gemm"] = expert_gemm_brief(et, dev, st.stream, plan, st.X)
    st.release()
    del st
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="C3", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-reps", type=int, default=3,
                    help="timed passes of the CPU baseline after its warm-up (0 skips it)")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the side measurements (other configs, router, expert GEMM)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the full-size steps of the other configurations (C1, C2, C4)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the path on one GPU's "
              "local share of experts and has no multi-GPU (expert-parallel) mode; "
              "run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    et = importlib.import_module("peer-review-agents_amd")
    W = importlib.import_module("peer-review-agents_amd.workloads")
    lib = et.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    print(f"bench: workload {args.workload}, {args.steps} steps after {args.warmup} warm-up", file=sys.stderr,
          flush=True)
    step = Step(et, lib, dev, args.workload, args.seed)
    T, d, E, S, cfg = step.T, step.d, step.E, step.S, step.cfg
    stream = step.stream
    all_stages = list(range(len(STAGES)))

    copy_ref = copy_ceiling(dev, stream)

    # ---- timed region -----------------------------------------------------------
    stage_ms, ms_per_step = step.timed(args.steps, args.warmup, all_stages)

    abytes = algorithmic_bytes(T, E, S, d, step.b)
    step_bytes = sum(abytes.values())
    kernels = {}
    for name in STAGES:
        gbs = abytes[name] / (stage_ms[name] * 1e-3) / 1e9
        kernels[name] = {"ms": round(stage_ms[name], 4), "GB/s": round(gbs, 1),
                         "frac": round(gbs * 1e9 / HBM_PEAK, 4), "bytes": abytes[name]}
    # The dominant stage, et_combine_bwd, is three launches on one stream
    # (combine_bwd_order, combine_bwd_vec, combine_bwd_finish; the order pass
    # only where the slots are walked in token windows); its event time covers
    # all of them.
    dom = "combine_bwd"
    ach = abytes[dom] / (stage_ms[dom] * 1e-3) / 1e9
    roofline = {"kernel": "combine_bwd (combine_bwd_order + combine_bwd_vec + combine_bwd_finish)", "bound": "hbm",
                "achieved": round(ach, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(ach * 1e9 / HBM_PEAK, 4), "traffic": read_traffic(args.workload),
                "algorithmic_bytes": abytes[dom], "ms": round(stage_ms[dom], 4)}

    # The same step captured once in a HIP graph and replayed.
    graph_ms = step.graph_ms(all_stages, args.steps)
    graph_replay = {"ms_per_step": round(graph_ms, 4), "slots_per_s": round(S / (graph_ms * 1e-3), 1),
                    "hbm_frac": round(step_bytes / (graph_ms * 1e-3) / HBM_PEAK, 4)}
    slots_per_s = S / (ms_per_step * 1e-3)
    for name in STAGES:
        k = kernels[name]
        print(f"  {name:13s} {k['ms']:8.4f} ms  {k['GB/s']:8.1f} GB/s  {100 * k['frac']:5.1f}% of peak",
              file=sys.stderr)
    print(f"  copy ref      {copy_ref['ms']:8.4f} ms  {copy_ref['GB/s']:8.1f} GB/s  "
          f"{100 * copy_ref['frac']:5.1f}% of peak ({copy_ref['kernel']}, {copy_ref['bytes']} B)",
          file=sys.stderr)
    print(f"  step {ms_per_step:.4f} ms, {slots_per_s / 1e6:.2f} M slots/s, "
          f"{100 * step_bytes / (ms_per_step * 1e-3) / HBM_PEAK:.1f}% of HBM peak; replayed as a HIP graph "
          f"{graph_ms:.4f} ms ({100 * graph_replay['hbm_frac']:.1f}%)", file=sys.stderr, flush=True)

    # ---- side measurements (after the timed region) -------------------------------
    dyn = rp = rb = eg = None
    extras = {}
    extras_error = None
    if not args.no_extras:
        # the optional legs: an exception in one is reported in the JSON line
        # (extras_error) and does not cost the headline measurement
        try:
            dyn = threshold_dynamics(et, W, dev, stream, "C5", args.seed)
            print(f"  C5 threshold dynamics: {dyn['steps']} steps, route {dyn['route_ms']:.4f} ms + EMA update "
                  f"{dyn['ema_update_ms']:.4f} ms per step, mean k {dyn['mean_k_first_step']} -> "
                  f"{dyn['mean_k_last_step']}; all steps replayed as one HIP graph "
                  f"{dyn['graph_replay_ms_per_step']:.4f} ms per step; et_route_update (routing and update in one call) "
                  f"{dyn['route_update_ms']:.4f} ms per step, {dyn['route_update_graph_replay_ms_per_step']:.4f} "
                  f"ms replayed", file=sys.stderr, flush=True)
            if step.act == torch.bfloat16 and E <= 256:
                rp = router_producer(et, dev, stream, step.X, E)
                print(f"  router producer: logits {rp['us']:.1f} us ({rp['GB/s']:.0f} GB/s, {100 * rp['frac']:.1f}% of "
                      f"peak; torch bf16 linear {rp['torch_linear_bf16_us']:.1f} us), fused route "
                      f"{rp['fused_route_us']:.1f} us vs logits + route {rp['logits_then_route_us']:.1f} us",
                      file=sys.stderr, flush=True)
            plan_obj = et.RoutingPlan(step.counts, step.eoff, step.toff, step.st, step.sg, step.ts, T, E, S, S)
            rb = router_backward(et, dev, stream, plan_obj, step.X, step.DXP, step.DGATE, step.DL)
            print(f"  router backward: dispatch_bwd {rb['dispatch_bwd_us']:.1f} us -> with the router input gradient "
                  f"{rb['dispatch_bwd_router_us']:.1f} us" + (f"; dW {rb['router_wgrad_us']:.1f} us "
                  f"({100 * rb['router_wgrad_frac']:.1f}% of peak; torch f32 mm {rb['torch_mm_f32_wgrad_us']:.1f} us)"
                  if "router_wgrad_us" in rb else ""), file=sys.stderr, flush=True)
            if step.act == torch.bfloat16 and d % 8 == 0 and S > 0:
                eg = expert_gemm_leg(et, dev, stream, plan_obj, step.X)
                gu, dn = eg["gate_up"], eg["down"]
                print(f"  expert GEMM: gate/up {gu['ms']:.3f} ms ({gu['TFLOP/s']:.0f} TFLOP/s, dispatch fused; with the "
                      f"SwiGLU epilogue {gu['swiglu_epilogue_ms']:.3f} ms; torch grouped {gu['torch_grouped_mm_ms']:.3f} "
                      f"ms + dispatch {gu['dispatch_ms']:.3f} ms), down {dn['ms']:.3f} ms ({dn['TFLOP/s']:.0f} TFLOP/s; "
                      f"torch grouped {dn['torch_grouped_mm_ms']:.3f} ms)", file=sys.stderr)
                g8 = eg["gate_up_fp8"]
                print(f"  expert GEMM fp8: gate/up {g8['ms']:.3f} ms ({g8['TFLOP/s']:.0f} TFLOP/s, {100 * g8['frac']:.1f}% "
                      f"of the fp8 peak; with the SwiGLU epilogue {g8['swiglu_epilogue_ms']:.3f} ms; relative error "
                      f"against bf16 {g8['relative_error_vs_bf16']:.4f}), down {eg['down_fp8']['ms']:.3f} ms "
                      f"({eg['down_fp8']['TFLOP/s']:.0f} TFLOP/s)", file=sys.stderr)
                bw = eg["backward"]
                print(f"  expert GEMM backward: down dA fused with the combine backward "
                      f"{bw['down_input_grad_fused_combine_bwd_ms']:.3f} ms (transpose {bw['weight_transpose_down_ms']:.3f}),"
                      f" gate/up dA {bw['gate_up_input_grad_ms']:.3f} ms, dW gate/up {bw['gate_up_weight_grad_ms']:.3f} ms "
                      f"(torch grouped {bw['torch_grouped_mm_gate_up_weight_grad_ms']}), dW down "
                      f"{bw['down_weight_grad_ms']:.3f} ms", file=sys.stderr)
                sw = eg["swiglu"]
                print(f"  SwiGLU for training: forward {sw['forward_ms']:.3f} ms ({100 * sw['forward_frac']:.1f}% of peak), "
                      f"backward {sw['backward_ms']:.3f} ms ({100 * sw['backward_frac']:.1f}% of peak)", file=sys.stderr,
                      flush=True)
            # the other row configurations at full size: C1 (the CPU reference
            # configuration, f32, all five stages), C2 (variable k, all five
            # stages) and C4 (one GPU's EP=8 expert share, backward only)
            for name, stages in (("C1", all_stages), ("C2", all_stages), ("C4", [3, 4])):
                if name == args.workload or args.no_other_configs:
                    continue
                extras[name] = extra_workload(et, lib, dev, name, args.seed, stages, gemm=True)
                x = extras[name]
                print(f"  {name} full size ({'+'.join(x['stages'])}): {x['ms_per_step']:.4f} ms per step, "
                      f"{x['slots_per_s'] / 1e6:.2f} M slots/s, {100 * x['hbm_frac']:.1f}% of HBM peak, mean k "
                      f"{x['mean_k']}; replayed as a HIP graph {x['graph_replay']['ms_per_step']:.4f} ms "
                      f"({100 * x['graph_replay']['hbm_frac']:.1f}%)", file=sys.stderr, flush=True)
                if "expert_gemm" in x:
                    b = x["expert_gemm"]
                    print(f"    expert GEMM: gate/up {b['gate_up_ms']:.3f} ms (torch grouped {b['torch_grouped_mm_gate_up_ms']:.3f}"
                          f" + dispatch {b['dispatch_ms']:.3f}), down {b['down_ms']:.3f} ms (torch grouped "
                          f"{b['torch_grouped_mm_down_ms']:.3f})", file=sys.stderr, flush=True)
        except Exception as exc:  # noqa: BLE001
            import traceback
            traceback.print_exc()
            extras_error = f"{type(exc).__name__}: {exc}"

    cpu = None
    if args.cpu_reps > 0:
        cpu = cpu_baseline(args.workload, step, reps=args.cpu_reps)
        print(f"  CPU baseline: {cpu['value'] / 1e6:.3f} M slots/s ({cpu['median_s']:.3f} s per pass, "
              f"{cpu['cores']} threads of {cpu['nproc']}); full-size parity vs GPU: "
              f"{cpu['full_size_parity_vs_gpu']}", file=sys.stderr, flush=True)

    out = {
        "metric": METRIC,
        "value": round(slots_per_s, 1),
        "unit": "slots/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: T={T} d={d} E={E} {cfg['dtype']}, "
                               f"thresholds {cfg['thr']}", "T": T, "d": d, "E": E, "slots": S,
                   "mean_k": round(S / T, 4), "seed": args.seed, "parallelism": "single GPU"},
        "hbm_frac": round(step_bytes / (ms_per_step * 1e-3) / HBM_PEAK, 4),
        "step_bytes": step_bytes,
        "roofline": roofline,
        "load_shape": step.shape,
        "graph_replay": graph_replay,
        "cpu_baseline": cpu,
        "copy_ceiling": copy_ref,
        "other_configs": extras or None,
        "extras_error": extras_error,
        "threshold_dynamics": dyn,
        "router_producer": rp,
        "router_backward": rb,
        "expert_gemm": eg,
        "kernels": kernels,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
