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
    """Measured HBM bytes of one et_combine_bwd call (its two kernels), from the
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
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    r_ms = u_ms = 0.0
    torch.cuda.synchronize()
    slots = []
    for i in range(steps):
        ev[0].record(stream)
        plan = et.route(logits[i], thr, slot_capacity=cap, workspace=rws)
        ev[1].record(stream)
        et.threshold_update_(thr, logits[i], cfg["k_target"], cfg["momentum"], stat=stat, workspace=tws)
        ev[2].record(stream)
        slots.append(plan.expert_offsets[E:E + 1])
        torch.cuda.synchronize()
        r_ms += ev[0].elapsed_time(ev[1])
        u_ms += ev[1].elapsed_time(ev[2])
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
    return {"steps": steps, "T": T, "E": E, "route_ms": round(r_ms / steps, 4),
            "ema_update_ms": round(u_ms / steps, 4), "mean_k_first_step": round(k[0], 4),
            "mean_k_last_step": round(k[-1], 4), "k_target": cfg["k_target"],
            "graph_replay_ms_per_step": round(g_ms, 4)}


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


def cpu_baseline(workload: str, seed: int, tokens: int) -> dict:
    """The CPU restatement (oracle/, single thread) on the first `tokens`
    tokens of the same workload, running the same five operations as one GPU
    step.  Routing uses the workload's real logits.  The row operands are a block
    of 1024 seeded random rows, tiled to the needed row counts; the row kernels
    have no data-dependent control flow, so tiling changes no timing."""
    import numpy as np
    import oracle
    W = importlib.import_module("peer-review-agents_amd.workloads")
    cfg = W.CONFIGS[workload]
    lg, thr = W.router_inputs(workload, seed=seed)
    lg = np.ascontiguousarray(lg[:tokens])
    d, E = cfg["d"], cfg["E"]
    r = oracle.route(lg, thr)
    S = r.num_slots
    conv = oracle.f32_to_bf16 if cfg["dtype"] == "bf16" else (lambda a: a)
    blk = conv(W.randn_rows(1024, d, 1))
    dyblk = conv(W.randn_rows(1024, d, 3, 0.02))
    x, yp, dxp = np.resize(blk, (tokens, d)), np.resize(blk, (S, d)), np.resize(blk, (S, d))
    dy = np.resize(dyblk, (tokens, d))
    t0 = time.perf_counter()
    r = oracle.route(lg, thr)
    oracle.dispatch_fwd(x, r)
    oracle.combine_fwd(yp, r, tokens)
    oracle.combine_bwd(dy, yp, r, E, want_dlogits=True)
    oracle.dispatch_bwd(dxp, r, tokens)
    dt = time.perf_counter() - t0
    return {"value": round(S / dt, 1), "unit": "slots/s", "cores": 1, "kind": "port",
            "sample": f"first {tokens} of {cfg['T']} tokens of {workload} ({S} slots), one fwd+bwd pass "
                      f"(route, dispatch, combine, combine backward with dlogits, dispatch backward) by "
                      f"the C oracle on one host thread: {dt:.2f} s"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="C3", choices=["C1", "C2", "C3", "C4", "C5"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-tokens", type=int, default=32768,
                    help="tokens in the CPU baseline's sample (0 skips it)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the path on one GPU's "
              "local share of experts and has no multi-GPU (expert-parallel) mode; "
              "run with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    et = importlib.import_module("peer-review-agents_amd")
    W = importlib.import_module("peer-review-agents_amd.workloads")
    lib = et.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = W.CONFIGS[args.workload]
    T, d, E = cfg["T"], cfg["d"], cfg["E"]
    act = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
    b = 2 if act == torch.bfloat16 else 4
    dt_code = 1 if act == torch.bfloat16 else 0

    # ---- resident inputs ------------------------------------------------------
    lg_h, thr_h = W.router_inputs(args.workload, seed=args.seed)
    logits = torch.from_numpy(lg_h).to(dev)
    thr = torch.from_numpy(thr_h).to(dev)
    plan = et.route(logits, thr)                 # sizes the slot buffers (one sync, untimed)
    S = plan.num_slots
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    X = torch.randn(T, d, device=dev, generator=g).to(act)
    YP = torch.randn(S, d, device=dev, generator=g).to(act)
    DY = (torch.randn(T, d, device=dev, generator=g) * 0.02).to(act)
    DXP = torch.randn(S, d, device=dev, generator=g).to(act)
    i32 = dict(dtype=torch.int32, device=dev)
    counts, eoff, toff = torch.empty(E, **i32), torch.empty(E + 1, **i32), torch.empty(T + 1, **i32)
    st, ts = torch.empty(S, **i32), torch.empty(S, **i32)
    sg = torch.empty(S, dtype=torch.float32, device=dev)
    wsb = et.route_workspace_bytes(T, E)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    XP = torch.empty(S, d, dtype=act, device=dev)
    Y = torch.empty(T, d, dtype=act, device=dev)
    DYP = torch.empty(S, d, dtype=act, device=dev)
    DGATE = torch.empty(S, dtype=torch.float32, device=dev)
    DL = torch.empty(T, E, dtype=torch.float32, device=dev)
    DX = torch.empty(T, d, dtype=act, device=dev)
    bwsb = et.combine_backward_workspace_bytes(T, S, d, act)
    BWS = torch.empty(max(bwsb, 1), dtype=torch.uint8, device=dev)
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = [vp(t) for t in (logits, thr, counts, eoff, toff, st, sg, ts, ws, X, XP, YP, Y, DY, DYP, DGATE, DL,
                         DXP, DX, BWS)]
    (p_lg, p_thr, p_cnt, p_eo, p_to, p_st, p_sg, p_ts, p_ws, p_x, p_xp, p_yp, p_y, p_dy, p_dyp, p_dg, p_dl,
     p_dxp, p_dx, p_bws) = P

    def stage(i, sp=sp):
        if i == 0:
            rc = lib.et_route(p_lg, p_thr, T, E, p_cnt, p_eo, p_to, p_st, p_sg, p_ts, S, p_ws, wsb, sp)
        elif i == 1:
            rc = lib.et_dispatch_fwd(p_x, T, d, dt_code, p_to, p_ts, S, p_xp, sp)
        elif i == 2:
            rc = lib.et_combine_fwd(p_yp, p_sg, p_to, p_ts, T, d, dt_code, S, p_y, sp)
        elif i == 3:
            rc = lib.et_combine_bwd(p_dy, p_yp, p_sg, p_st, p_to, p_ts, p_eo, T, E, d, dt_code, S, p_dyp, p_dg,
                                    p_dl, p_bws, bwsb, sp)
        else:
            rc = lib.et_dispatch_bwd(p_dxp, p_to, p_ts, T, d, dt_code, S, p_dx, sp)
        if rc != 0:
            raise RuntimeError(f"stage {STAGES[i]} failed: {lib.et_last_error().decode()}")

    copy_ref = copy_ceiling(dev, stream)
    for _ in range(args.warmup):
        for i in range(len(STAGES)):
            stage(i)
    torch.cuda.synchronize()
    assert int(eoff[E]) == S, "routing changed between runs"

    # ---- timed region -----------------------------------------------------------
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(STAGES) + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        ev[k][0].record(stream)
        for i in range(len(STAGES)):
            stage(i)
            ev[k][i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    stage_ms = {name: 0.0 for name in STAGES}
    for k in range(args.steps):
        for i, name in enumerate(STAGES):
            stage_ms[name] += ev[k][i].elapsed_time(ev[k][i + 1]) / args.steps
    ms_per_step = wall * 1e3 / args.steps
    abytes = algorithmic_bytes(T, E, S, d, b)
    step_bytes = sum(abytes.values())
    kernels = {}
    for name in STAGES:
        gbs = abytes[name] / (stage_ms[name] * 1e-3) / 1e9
        kernels[name] = {"ms": round(stage_ms[name], 4), "GB/s": round(gbs, 1),
                         "frac": round(gbs * 1e9 / HBM_PEAK, 4), "bytes": abytes[name]}
    # The dominant stage, et_combine_bwd, is two launches on one stream
    # (combine_bwd_vec, then combine_bwd_finish); its event time covers both.
    dom = "combine_bwd"
    ach = abytes[dom] / (stage_ms[dom] * 1e-3) / 1e9
    roofline = {"kernel": "combine_bwd (combine_bwd_vec + combine_bwd_finish)", "bound": "hbm",
                "achieved": round(ach, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(ach * 1e9 / HBM_PEAK, 4), "traffic": read_traffic(args.workload),
                "algorithmic_bytes": abytes[dom], "ms": round(stage_ms[dom], 4)}

    # The same step captured once in a HIP graph and replayed: what a caller
    # that captures the path sees where launches, not bytes, bound the step
    # (C1, C5).  Every stage runs with an explicit slot capacity, so the
    # capture holds no host synchronisation.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cs = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        for i in range(len(STAGES)):
            stage(i, cs)
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    assert int(eoff[E]) == S, "routing changed under graph replay"
    del graph
    graph_replay = {"ms_per_step": round(graph_ms, 4), "slots_per_s": round(S / (graph_ms * 1e-3), 1),
                    "hbm_frac": round(step_bytes / (graph_ms * 1e-3) / HBM_PEAK, 4)}

    dyn = None
    if cfg["thr"] == "ema":
        dyn = threshold_dynamics(et, W, dev, stream, args.workload, args.seed)
        print(f"  threshold dynamics: {dyn['steps']} steps, route {dyn['route_ms']:.4f} ms + EMA update "
              f"{dyn['ema_update_ms']:.4f} ms per step, mean k {dyn['mean_k_first_step']} -> "
              f"{dyn['mean_k_last_step']}; all steps replayed as one HIP graph "
              f"{dyn['graph_replay_ms_per_step']:.4f} ms per step", file=sys.stderr)

    rp = None
    if act == torch.bfloat16 and E <= 256:
        rp = router_producer(et, dev, stream, X, E)
        print(f"  router producer: logits {rp['us']:.1f} us ({rp['GB/s']:.0f} GB/s, {100 * rp['frac']:.1f}% of "
              f"peak; torch bf16 linear {rp['torch_linear_bf16_us']:.1f} us), fused route {rp['fused_route_us']:.1f}"
              f" us vs logits + route {rp['logits_then_route_us']:.1f} us", file=sys.stderr)

    plan_obj = et.RoutingPlan(counts, eoff, toff, st, sg, ts, T, E, S, S)
    rb = router_backward(et, dev, stream, plan_obj, X, DXP, DGATE, DL)
    print(f"  router backward: dispatch_bwd {rb['dispatch_bwd_us']:.1f} us -> with the router input gradient "
          f"{rb['dispatch_bwd_router_us']:.1f} us" + (f"; dW {rb['router_wgrad_us']:.1f} us "
          f"({100 * rb['router_wgrad_frac']:.1f}% of peak; torch f32 mm {rb['torch_mm_f32_wgrad_us']:.1f} us)"
          if "router_wgrad_us" in rb else ""), file=sys.stderr)

    eg = None
    if act == torch.bfloat16 and d % 8 == 0 and S > 0:
        eg = expert_gemm_leg(et, dev, stream, plan_obj, X)
        gu, dn = eg["gate_up"], eg["down"]
        print(f"  expert GEMM: gate/up {gu['ms']:.3f} ms ({gu['TFLOP/s']:.0f} TFLOP/s, dispatch fused; with the SwiGLU "
              f"epilogue {gu['swiglu_epilogue_ms']:.3f} ms; torch grouped {gu['torch_grouped_mm_ms']:.3f} ms + dispatch "
              f"{gu['dispatch_ms']:.3f} ms), down {dn['ms']:.3f} ms ({dn['TFLOP/s']:.0f} TFLOP/s; torch grouped "
              f"{dn['torch_grouped_mm_ms']:.3f} ms)", file=sys.stderr)
        g8 = eg["gate_up_fp8"]
        print(f"  expert GEMM fp8: gate/up {g8['ms']:.3f} ms ({g8['TFLOP/s']:.0f} TFLOP/s, {100 * g8['frac']:.1f}% of the "
              f"fp8 peak; with the SwiGLU epilogue {g8['swiglu_epilogue_ms']:.3f} ms; relative error against bf16 "
              f"{g8['relative_error_vs_bf16']:.4f}), down {eg['down_fp8']['ms']:.3f} ms "
              f"({eg['down_fp8']['TFLOP/s']:.0f} TFLOP/s)", file=sys.stderr)
        bw = eg["backward"]
        print(f"  expert GEMM backward: down dA fused with the combine backward {bw['down_input_grad_fused_combine_bwd_ms']:.3f}"
              f" ms (transpose {bw['weight_transpose_down_ms']:.3f}), gate/up dA {bw['gate_up_input_grad_ms']:.3f} ms, "
              f"dW gate/up {bw['gate_up_weight_grad_ms']:.3f} ms (torch grouped {bw['torch_grouped_mm_gate_up_weight_grad_ms']}"
              f"), dW down {bw['down_weight_grad_ms']:.3f} ms", file=sys.stderr)
        sw = eg["swiglu"]
        print(f"  SwiGLU for training: forward {sw['forward_ms']:.3f} ms ({100 * sw['forward_frac']:.1f}% of peak), "
              f"backward {sw['backward_ms']:.3f} ms ({100 * sw['backward_frac']:.1f}% of peak)", file=sys.stderr)

    cpu = None
    if args.cpu_tokens > 0:
        cpu = cpu_baseline(args.workload, args.seed, min(args.cpu_tokens, T))

    slots_per_s = S / (ms_per_step * 1e-3)
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
        "graph_replay": graph_replay,
        "cpu_baseline": cpu,
        "copy_ceiling": copy_ref,
        "threshold_dynamics": dyn,
        "router_producer": rp,
        "router_backward": rb,
        "expert_gemm": eg,
        "kernels": kernels,
    }
    for name in STAGES:
        k = kernels[name]
        print(f"  {name:13s} {k['ms']:8.4f} ms  {k['GB/s']:8.1f} GB/s  {100 * k['frac']:5.1f}% of peak",
              file=sys.stderr)
    print(f"  copy ref      {copy_ref['ms']:8.4f} ms  {copy_ref['GB/s']:8.1f} GB/s  "
          f"{100 * copy_ref['frac']:5.1f}% of peak ({copy_ref['kernel']}, {copy_ref['bytes']} B)",
          file=sys.stderr)
    print(f"  step {ms_per_step:.4f} ms, {slots_per_s / 1e6:.2f} M slots/s, "
          f"{100 * out['hbm_frac']:.1f}% of HBM peak; replayed as a HIP graph {graph_ms:.4f} ms "
          f"({100 * graph_replay['hbm_frac']:.1f}%)", file=sys.stderr)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
