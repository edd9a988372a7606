"""SwiGLU of the expert FFN and its backward (et_swiglu_fwd / et_swiglu_bwd) on
the GPU, over the routed slots of a real routing plan.

Parity is bit-exact against the CPU oracle's slot-row forms
(oracle_swiglu_fwd_rows / oracle_swiglu_bwd_rows, whose binary32 expressions
are pinned against float64 derivatives and finite differences): both evaluate
the same separately rounded operations with the same sigmoid and round once to
bf16.  A NaN output (0 * inf of extreme inputs) only has to be NaN on both
sides: the sign and payload of a generated NaN are the machine's.  Also:
rows past the routed slots are left untouched, an undersized capacity computes
exactly the rows below it, and on exact integer products the training forward
equals the expert GEMM's fused SwiGLU epilogue bit for bit.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _plan(et, dev, T, E, k, seed, slot_capacity=None):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    logits = torch.randn(T, E, generator=g, device=dev)
    thr = torch.quantile(torch.sigmoid(logits.double()), max(0.0, 1.0 - k / E), dim=0).float().contiguous()
    return et.route(logits, thr, slot_capacity=slot_capacity)


def _u16(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _same(got_bits, want_bits):
    """bf16 bit patterns equal, except that NaN only has to match NaN."""
    gf = (got_bits.astype(np.uint32) << 16).view(np.float32)
    wf = (want_bits.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(wf)
    return np.array_equal(np.isnan(gf), nan) and np.array_equal(got_bits[~nan], want_bits[~nan])


def _random_bf16(shape, seed, dev, wide=False):
    g = torch.Generator().manual_seed(seed)
    if wide:
        # finite bf16 bit patterns of every magnitude (exponent fields 0..254)
        bits = torch.randint(0, 1 << 16, shape, generator=g, dtype=torch.int32)
        bits = torch.where((bits & 0x7F80) == 0x7F80, bits & 0xBFFF, bits)
        return bits.to(torch.int16).view(torch.bfloat16).to(dev)
    return (torch.randn(shape, generator=g) * 4).to(torch.bfloat16).to(dev)


@pytest.mark.parametrize("T,E,k,F,wide", [(256, 4, 2, 8, False), (1000, 16, 3, 136, False),
                                          (3000, 64, 4, 512, False), (777, 8, 2, 1536, True)])
def test_swiglu_forward_and_backward_bit_exact(et, orc, dev, T, E, k, F, wide):
    print(f"swiglu T={T} E={E} F={F} wide={wide}", flush=True)
    plan = _plan(et, dev, T, E, k, seed=T)
    S = plan.num_slots
    cap = S + 40                                           # rows past the routed slots stay untouched
    plan = _plan(et, dev, T, E, k, seed=T, slot_capacity=cap)
    gu = _random_bf16((cap, 2 * F), 1, dev, wide)
    dh = _random_bf16((cap, F), 2, dev, wide)
    h = torch.full((cap, F), 7.0, dtype=torch.bfloat16, device=dev)
    dgu = torch.full((cap, 2 * F), -3.0, dtype=torch.bfloat16, device=dev)
    et.swiglu(gu, plan, out=h)
    et.swiglu_backward(gu, dh, plan, out=dgu)
    torch.cuda.synchronize()
    gub, dhb = _u16(gu), _u16(dh)
    assert _same(_u16(h)[:S], orc.swiglu_rows(gub[:S]))
    assert _same(_u16(dgu)[:S], orc.swiglu_backward_rows(gub[:S], dhb[:S]))
    assert bool((h[S:] == 7.0).all()) and bool((dgu[S:] == -3.0).all())
    # repeated calls give identical bits
    assert torch.equal(et.swiglu(gu, plan).view(torch.int16)[:S], h.view(torch.int16)[:S])


def test_swiglu_undersized_capacity(et, orc, dev):
    T, E, F = 2000, 8, 64
    S = _plan(et, dev, T, E, 3, seed=5).num_slots
    cap = S // 3
    plan = _plan(et, dev, T, E, 3, seed=5, slot_capacity=cap)
    gu = _random_bf16((cap, 2 * F), 3, dev)
    dh = _random_bf16((cap, F), 4, dev)
    h = et.swiglu(gu, plan)
    dgu = et.swiglu_backward(gu, dh, plan)
    torch.cuda.synchronize()
    assert _same(_u16(h), orc.swiglu_rows(_u16(gu)))
    assert _same(_u16(dgu), orc.swiglu_backward_rows(_u16(gu), _u16(dh)))


def test_swiglu_forward_equals_gemm_epilogue_on_exact_products(et, dev):
    """Integer operands with |gate|, |up| <= 64: the plain GEMM's gu is exact in
    bf16, so the training forward on it and the epilogue on the accumulators
    see the same binary32 values and must agree bit for bit."""
    T, E, K, F = 1500, 8, 64, 96
    plan = _plan(et, dev, T, E, 2, seed=9)
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randint(-1, 2, (T, K), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randint(-1, 2, (E, 2 * F, K), generator=g, device=dev).to(torch.bfloat16)
    gu = et.expert_gemm(x, w, plan)
    fused = et.expert_gemm(x, w, plan, epilogue="swiglu")
    S = plan.num_slots
    assert torch.equal(et.swiglu(gu, plan).view(torch.int16)[:S], fused.view(torch.int16)[:S])


def test_swiglu_rejects_bad_shapes(et, dev):
    plan = _plan(et, dev, 100, 4, 2, seed=1)
    R = plan.rows
    with pytest.raises(ValueError):
        et.swiglu(torch.zeros(R, 24, dtype=torch.bfloat16, device=dev), plan)       # F = 12
    with pytest.raises(ValueError):
        et.swiglu(torch.zeros(R + 1, 32, dtype=torch.bfloat16, device=dev), plan)
    with pytest.raises(TypeError):
        et.swiglu(torch.zeros(R, 32, dtype=torch.float32, device=dev), plan)
    with pytest.raises(ValueError):
        et.swiglu_backward(torch.zeros(R, 32, dtype=torch.bfloat16, device=dev),
                           torch.zeros(R, 8, dtype=torch.bfloat16, device=dev), plan)
