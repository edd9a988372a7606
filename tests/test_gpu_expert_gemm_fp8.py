"""The expert grouped GEMM on fp8 e4m3 operands (et_expert_gemm_fp8) on the GPU.

c[s] = ((A[row(s)] @ W[e(s)]^T) * a_scale[row(s)]) * w_scale[e(s)] over the
routing CSR, binary32 accumulation, bf16 out.  Parity is pinned by what the
arithmetic fixes, as for the bf16 GEMM:
  * integer operands (every integer of magnitude <= 16 is exact in e4m3) with
    power-of-two scales: every product and partial sum below 2^24 is exact in
    binary32 in any order, so each output must be the exact float64 value
    rounded once to bf16 (torch's cast) -- a dropped k-step, a wrong expert,
    token, row or scale, a transposed operand or a missed edge tile changes
    some entry;
  * the SwiGLU epilogue on such exact products equals the CPU oracle's
    binary32 (g * sigmoid(g)) * u rounded to bf16, bit for bit;
  * the gather mode equals the slot-major mode on the gathered rows bit for
    bit, and random operands stay within the binary32 summation bound of the
    float64 product of the dequantized operands plus one bf16 rounding;
  * rows past the routed slots are left untouched.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn


def _plan(et, dev, T, E, k, seed, skew=0.0, slot_capacity=None):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    logits = torch.randn(T, E, generator=g, device=dev)
    if skew:
        logits[:, 0] += skew
    s = torch.sigmoid(logits.double())
    thr = torch.quantile(s[:min(T, 8192)], max(0.0, 1.0 - k / E), dim=0).float().contiguous()
    return et.route(logits, thr, slot_capacity=slot_capacity)


def _int_f8(shape, g, dev, lim=4):
    return torch.randint(-lim, lim + 1, shape, generator=g, device=dev).to(torch.float32).to(F8)


def _pow2(shape, g, dev):
    return torch.exp2(torch.randint(-3, 3, shape, generator=g, device=dev).to(torch.float32))


def _reference(x, sa, w, sw, plan, rows, gather):
    """float64 [rows, N]: ((A @ W_e^T) * sa[row]) * sw[e, n] over the slots below rows."""
    eo = plan.expert_offsets.cpu().tolist()
    st = plan.sorted_token[:rows].long()
    E, N, K = w.shape
    ref = torch.zeros(rows, N, dtype=torch.float64, device=x.device)
    mass = torch.zeros(rows, N, dtype=torch.float64, device=x.device)
    for e in range(E):
        lo, hi = min(eo[e], rows), min(eo[e + 1], rows)
        if hi <= lo:
            continue
        idx = st[lo:hi] if gather else torch.arange(lo, hi, device=x.device)
        a = x[idx].double()
        wd = w[e].double()
        sr = sa[idx].double()[:, None] * sw[e].double()[None, :]
        ref[lo:hi] = (a @ wd.T) * sr
        mass[lo:hi] = (a.abs() @ wd.abs().T) * sr.abs()
    return ref, mass


SHAPES = [  # (T, K, N, E, k, skew): K off the 128-k chunk, N off the 256-wide tile, empty experts, skew
    (1, 16, 8, 1, 1, 0.0), (300, 48, 200, 5, 2, 0.0), (1000, 256, 264, 8, 3, 0.0),
    (777, 528, 520, 33, 4, 0.0), (4096, 1024, 768, 16, 2, 0.0), (5000, 144, 512, 64, 4, 12.0),
]


@pytest.mark.parametrize("T,K,N,E,k,skew", SHAPES)
@pytest.mark.parametrize("gather", [True, False])
def test_expert_gemm_fp8_exact_on_integer_inputs(et, dev, T, K, N, E, k, skew, gather):
    print(f"expert_gemm_fp8 T={T} K={K} N={N} E={E} gather={gather}", flush=True)
    plan = _plan(et, dev, T, E, k, seed=T + K, skew=skew)
    S = plan.rows
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    w = _int_f8((E, N, K), g, dev)
    sw = _pow2((E, N), g, dev)
    if gather:
        x = _int_f8((T, K), g, dev)
        sa = _pow2((T,), g, dev)
        c = et.expert_gemm_fp8(x, sa, w, sw, plan, gather=True)
    else:
        xs = _int_f8((T, K), g, dev)
        x = xs[plan.sorted_token.long()].contiguous()          # slot-major rows
        sa = _pow2((S,), g, dev)
        c = et.expert_gemm_fp8(x, sa, w, sw, plan, gather=False)
    ref, _ = _reference(x.float(), sa, w.float(), sw, plan, S, gather)
    assert torch.equal(c.view(torch.int16), ref.to(torch.float32).to(torch.bfloat16).view(torch.int16))


def test_expert_gemm_fp8_swiglu_exact_on_integer_inputs(et, orc, dev):
    T, K, F, E = 2000, 256, 200, 16
    plan = _plan(et, dev, T, E, 3, seed=4)
    S = plan.rows
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    x = _int_f8((T, K), g, dev, lim=2)
    w = _int_f8((E, 2 * F, K), g, dev, lim=2)
    sa = _pow2((T,), g, dev) * 0.25
    sw = _pow2((E, 2 * F), g, dev) * 0.25
    h = et.expert_gemm_fp8(x, sa, w, sw, plan, epilogue="swiglu")
    ref, _ = _reference(x.float(), sa, w.float(), sw, plan, S, True)   # exact: small integers x powers of two
    gate = ref[:, :F].to(torch.float32).cpu().numpy()
    up = ref[:, F:].to(torch.float32).cpu().numpy()
    want = orc.f32_to_bf16(orc.swiglu(gate, up)).view(np.int16)
    assert np.array_equal(h.view(torch.int16).cpu().numpy(), want)


def test_expert_gemm_fp8_gather_equals_slot_major_and_random_bound(et, dev):
    T, K, N, E = 3000, 384, 512, 32
    plan = _plan(et, dev, T, E, 4, seed=11)
    S = plan.rows
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    x = (torch.randn(T, K, generator=g, device=dev) * 2).to(F8)
    w = (torch.randn(E, N, K, generator=g, device=dev) * 0.5).to(F8)
    sa = torch.rand(T, generator=g, device=dev) + 0.5
    sw = torch.rand(E, N, generator=g, device=dev) * 0.1 + 0.01
    c1 = et.expert_gemm_fp8(x, sa, w, sw, plan, gather=True)
    st = plan.sorted_token.long()
    c2 = et.expert_gemm_fp8(x[st].contiguous(), sa[st].contiguous(), w, sw, plan, gather=False)
    assert torch.equal(c1.view(torch.int16), c2.view(torch.int16))
    assert torch.equal(et.expert_gemm_fp8(x, sa, w, sw, plan).view(torch.int16), c1.view(torch.int16))
    ref, mass = _reference(x.float(), sa, w.float(), sw, plan, S, True)
    err = (c1.double() - ref).abs()
    bound = K * 2.0 ** -24 * mass * 4 + ref.abs() * 2.0 ** -8 + 1e-30
    assert bool((err <= bound).all())


def test_expert_gemm_fp8_leaves_rows_past_the_slots(et, dev):
    T, K, N, E = 500, 128, 256, 8
    S = _plan(et, dev, T, E, 2, seed=3).num_slots
    plan = _plan(et, dev, T, E, 2, seed=3, slot_capacity=S + 40)
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    x = _int_f8((T, K), g, dev)
    w = _int_f8((E, N, K), g, dev)
    sa, sw = _pow2((T,), g, dev), _pow2((E, N), g, dev)
    out = torch.full((S + 40, N), 3.0, dtype=torch.bfloat16, device=dev)
    et.expert_gemm_fp8(x, sa, w, sw, plan, out=out)
    assert bool((out[S:] == 3.0).all())
    ref, _ = _reference(x.float(), sa, w.float(), sw, plan, S, True)
    assert torch.equal(out[:S].view(torch.int16), ref.to(torch.float32).to(torch.bfloat16).view(torch.int16))


def test_expert_gemm_fp8_scales_at_any_4_byte_offset(et, dev):
    """Scales are loaded one dword per lane: views that start 4 bytes into
    their storage give the same bits as aligned copies."""
    T, K, N, E = 700, 192, 272, 6
    plan = _plan(et, dev, T, E, 2, seed=13)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    x = _int_f8((T, K), g, dev)
    w = _int_f8((E, N, K), g, dev)
    sa, sw = _pow2((T,), g, dev), _pow2((E, N), g, dev)
    sa1 = torch.empty(T + 1, device=dev)[1:]
    sa1.copy_(sa)
    sw1 = torch.empty(E * N + 1, device=dev)[1:].view(E, N)
    sw1.copy_(sw)
    assert sa1.data_ptr() % 16 and sw1.data_ptr() % 16
    for ep in ("none", "swiglu"):
        c0 = et.expert_gemm_fp8(x, sa, w, sw, plan, epilogue=ep)
        c1 = et.expert_gemm_fp8(x, sa1, w, sw1, plan, epilogue=ep)
        assert torch.equal(c0.view(torch.int16), c1.view(torch.int16))
