"""Router producer (logits = X W^T on the matrix cores) on the GPU.

Parity is pinned by what the arithmetic fixes:
  * integer-valued bf16 inputs whose partial sums stay below 2^24 are summed
    exactly in binary32 in any order, so the kernel must return the exact
    integer product -- a dropped k-step, a swapped operand, a wrong row or
    column, or a missed edge tile changes some entry by at least 1;
  * random inputs stay within the rigorous binary32 summation bound
    d * 2^-24 * sum_k |x_k w_k| of the float64 product, and their mean error is
    at the sqrt(d) level of a correctly rounded accumulation;
  * repeated calls are bit-identical, and routing those logits gives exactly
    the CPU oracle's routing of the same logits.
The float64 products are computed by torch on the device as the checker.
"""
import importlib

import numpy as np
import pytest
import torch

from test_gpu_parity import assert_route_equal, host

W = importlib.import_module("peer-review-agents_amd.workloads")

pytestmark = pytest.mark.gpu

SHAPES = [  # (T, d, E): ragged token tiles, expert counts off the 32-column tile, d off the 64-wide chunk
    (1, 8, 1), (5, 24, 8), (130, 520, 40), (257, 1032, 100), (1000, 4096, 128),
    (300, 256, 200), (129, 64, 256), (64, 7168, 32), (33, 2048, 64), (128, 1024, 96),
    # large batches take the two-token-tile launch shapes (ragged last tile)
    (33001, 136, 40), (66001, 72, 100), (70003, 64, 256), (65536, 520, 128),
    # the 2 x 2 launch with long rows (4-chunk X ring; 65 chunks, the last one ragged)
    (33000, 4104, 128),
]


def _int_bf16(shape, gen, dev, lim=4):
    return torch.randint(-lim, lim + 1, shape, generator=gen, device=dev).to(torch.bfloat16)


@pytest.mark.parametrize("T,d,E", SHAPES)
def test_router_logits_exact_on_integer_inputs(et, dev, T, d, E):
    print(f"router_logits integer T={T} d={d} E={E}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(T * 7919 + d * 31 + E)
    x = _int_bf16((T, d), g, dev)
    w = _int_bf16((E, d), g, dev)
    L = et.router_logits(x, w)
    want = x.double() @ w.double().T
    assert L.dtype == torch.float32 and tuple(L.shape) == (T, E)
    assert torch.equal(L.double(), want)


def test_router_logits_random_within_bound(et, dev):
    T, d, E = 4096, 4096, 128
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    x = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(E, d, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    L = et.router_logits(x, w)
    L2 = et.router_logits(x, w)
    assert torch.equal(L.view(torch.int32), L2.view(torch.int32))
    xd, wd = x.double(), w.double()
    ref = xd @ wd.T
    mass = xd.abs() @ wd.abs().T
    err = (L.double() - ref).abs()
    assert bool((err <= d * 2.0 ** -24 * mass).all())
    # a correctly rounded accumulation errs at the sqrt(d) * 2^-24 level on average
    assert float((err / mass).mean()) < 4 * d ** 0.5 * 2.0 ** -24


@pytest.mark.parametrize("T,E", [(2048, 16), (2048, 200), (66000, 128), (66000, 256)])
def test_router_logits_k_order(et, dev, T, E):
    """The k walk of token t starts at k0 = (floor(t / 256) mod 4) * 64 *
    floor(d / 256) and wraps.  With d = 512, x = 2^24 at k = 0 and 1 at k = 128
    and k = 256, and w = 1: from k0 = 128 (t / 256 = 1 mod 4) the two ones meet
    first and the sum is 2^24 + 2; from k0 = 0, 256 or 384 each one is added to
    2^24 and rounds away (ties to even).  Both launch shapes and both k-chunk
    widths (E <= 128 and E > 128) give the same bits."""
    print(f"router_logits k order T={T} E={E}", flush=True)
    d = 512
    x = torch.zeros(T, d, device=dev, dtype=torch.bfloat16)
    x[:, 0] = 2.0 ** 24
    x[:, 128] = 1.0
    x[:, 256] = 1.0
    w = torch.ones(E, d, device=dev, dtype=torch.bfloat16)
    L = et.router_logits(x, w)
    t = torch.arange(T, device=dev)
    want = torch.where((t // 256) % 4 == 1, 2.0 ** 24 + 2, 2.0 ** 24).double()
    assert torch.equal(L.double(), want[:, None].expand(T, E))


@pytest.mark.parametrize("T,E", [(2048, 16), (2048, 200), (66000, 128), (66000, 256)])
def test_router_logits_rounds_every_16_k(et, dev, T, E):
    """Each logit is rounded after every k-step of 16, also where one MFMA
    covers 32 k (up to 128 experts).  x = 2^24 at k = 0, 1 at k = 1 and 1 at
    k = 16, w = 1: rounding after k 0..15 gives 2^24 (the tie 2^24 + 1 goes to
    even), and adding the second 1 rounds away again, so every logit is 2^24
    from any start of the k walk; one rounding over k 0..31 would give 2^24 + 2."""
    print(f"router_logits 16-k rounding T={T} E={E}", flush=True)
    d = 512
    x = torch.zeros(T, d, device=dev, dtype=torch.bfloat16)
    x[:, 0] = 2.0 ** 24
    x[:, 1] = 1.0
    x[:, 16] = 1.0
    w = torch.ones(E, d, device=dev, dtype=torch.bfloat16)
    L = et.router_logits(x, w)
    assert bool((L == 2.0 ** 24).all())


def test_router_logits_full_size_c3_and_routing(et, orc, dev):
    cfg = W.CONFIGS["C3"]
    T, d, E = cfg["T"], cfg["d"], cfg["E"]
    print(f"router_logits C3 T={T} d={d} E={E}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    x = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(E, d, generator=g, device=dev) * d ** -0.5).to(torch.bfloat16)
    L = et.router_logits(x, w)
    for i in range(0, T, 8192):                     # float64 check in slices of 8192 tokens
        xd = x[i:i + 8192].double()
        ref = xd @ w.double().T
        mass = xd.abs() @ w.double().abs().T
        assert bool(((L[i:i + 8192].double() - ref).abs() <= d * 2.0 ** -24 * mass).all())
    del xd, ref, mass
    lg = host(L)
    thr = W.thresholds("C3", lg)
    plan = et.route(L, torch.from_numpy(thr).to(dev))
    assert_route_equal(plan, orc.route(lg, thr))


def test_router_logits_writes_into_out_and_handles_empty(et, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    x = _int_bf16((70, 128), g, dev)
    w = _int_bf16((16, 128), g, dev)
    out = torch.full((70, 16), float("nan"), device=dev)
    r = et.router_logits(x, w, out=out)
    assert r.data_ptr() == out.data_ptr()
    assert torch.equal(out.double(), x.double() @ w.double().T)
    empty = et.router_logits(x[:0], w)
    assert tuple(empty.shape) == (0, 16)


def test_router_logits_host_validation(et, dev):
    bf = torch.bfloat16
    x = torch.zeros(8, 64, device=dev, dtype=bf)
    with pytest.raises(TypeError):
        et.router_logits(x.float(), torch.zeros(4, 64, device=dev, dtype=bf))
    with pytest.raises(ValueError):
        et.router_logits(x, torch.zeros(4, 32, device=dev, dtype=bf))
    with pytest.raises(ValueError):
        et.router_logits(x, torch.zeros(257, 64, device=dev, dtype=bf))
    with pytest.raises(ValueError):
        et.router_logits(torch.zeros(8, 12, device=dev, dtype=bf), torch.zeros(4, 12, device=dev, dtype=bf))
    base = torch.zeros(8 * 64 + 4, device=dev, dtype=bf)
    with pytest.raises(ValueError):                 # 8-byte offset: not 16-byte aligned
        et.router_logits(base[4:].view(8, 64), torch.zeros(4, 64, device=dev, dtype=bf))
    with pytest.raises(ValueError):
        et.router_logits(x, torch.zeros(4, 64, device=dev, dtype=bf), out=torch.zeros(8, 5, device=dev))


# --------------------------------------------------------------------------- #
# fused producer + routing: bit-identical to router_logits followed by route
# --------------------------------------------------------------------------- #

def _assert_plans_identical(a, b):
    for f in ("counts", "expert_offsets", "token_offsets", "sorted_token", "token_slot"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f
    assert torch.equal(a.slot_gate.view(torch.int32), b.slot_gate.view(torch.int32))


def _router_case(dev, T, d, E, seed, q):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(E, d, generator=g, device=dev) * d ** -0.5).to(torch.bfloat16)
    return x, w


ROUTE_SHAPES = [  # (T, d, E, per-expert threshold quantile)
    (1, 8, 1, 0.5), (5, 24, 8, 0.75), (130, 520, 40, 0.9), (1000, 256, 128, 0.95), (300, 256, 200, 0.97),
    (129, 64, 256, 0.99), (33001, 136, 40, 0.8), (66001, 72, 100, 0.93), (70003, 64, 256, 0.97),
    (16384, 2048, 64, 0.875), (4096, 512, 8, 0.75), (40000, 4096, 64, 0.875),
]


@pytest.mark.parametrize("T,d,E,q", ROUTE_SHAPES)
def test_router_route_matches_composition(et, dev, T, d, E, q):
    print(f"router_route T={T} d={d} E={E} q={q}", flush=True)
    x, w = _router_case(dev, T, d, E, T + 17 * E, q)
    L = et.router_logits(x, w)
    thr = torch.quantile(torch.sigmoid(L.double()), q, dim=0).float().contiguous()
    thr[0] = 2.0                                   # expert 0 unreachable by threshold: only argmax fallbacks
    want = et.route(L, thr)
    got, L2 = et.router_route(x, w, thr, return_logits=True)
    assert got.num_slots == want.num_slots
    _assert_plans_identical(got, want)
    assert torch.equal(L2.view(torch.int32), L.view(torch.int32))
    assert et.router_route(x, w, thr).num_slots == want.num_slots      # the scores-free variant


def test_router_route_argmax_fallback_and_nonfinite(et, dev):
    T, d, E = 2000, 128, 96
    x, w = _router_case(dev, T, d, E, 5, 0.9)
    x[3, 0] = float("inf")                         # +-inf logits
    x[4, :16] = float("inf")
    x[5, 0] = float("inf")
    x[5, 1] = float("-inf")                        # inf - inf: NaN logits
    x[6] = float("nan")
    L = et.router_logits(x, w)
    assert bool(torch.isnan(L).any()) and bool(torch.isinf(L).any())
    for thr_val in (0.5, 0.999, 1.5):              # 1.5: every token falls back to its argmax expert
        thr = torch.full((E,), thr_val, device=dev)
        _assert_plans_identical(et.router_route(x, w, thr), et.route(L, thr))


def test_router_route_logits_at_the_threshold(et, orc, dev):
    """The fused epilogue decides most pairs in the logit domain (per-expert
    bounds around the logit of the threshold) and takes the exact score only
    between the bounds.  Here every logit sits within a few float steps of its
    expert's threshold logit l0 (thr = sigmoid(l0) as the oracle computes it,
    or one step above or below), so the exact path decides most pairs; other
    experts carry threshold values the bounds handle specially (<= 0, -0, 1,
    > 1, NaN, subnormal, the float below 1).  Logits are built exactly as
    a + b 2^-8 + c 2^-16 from three bf16 terms against a W holding 1, 2^-8 and
    2^-16.  Fused routing must equal router_logits -> route bit for bit."""
    E, T = 64, 4096
    d = 3 * E + 8
    rng = np.random.default_rng(12)
    l0 = (rng.standard_normal(E) * 3).astype(np.float32)
    thr = orc.sigmoid(l0).copy()
    thr[1::3] = np.nextafter(thr[1::3], np.float32(np.inf))
    thr[2::3] = np.nextafter(thr[2::3], np.float32(-np.inf))
    special = [0.0, -0.0, -1.0, 1.0, 1.5, np.nan, 1e-45, np.nextafter(np.float32(1), np.float32(0)), 0.5, 3e-39]
    thr[-len(special):] = np.float32(special)
    # per token, each expert's logit = l0 moved by a few float steps
    steps = rng.integers(-40, 41, size=(T, E))
    target = l0[None, :].repeat(T, 0)
    for k in range(1, 41):                         # nextafter, k steps either way
        up = steps >= k
        dn = steps <= -k
        target[up] = np.nextafter(target[up], np.float32(np.inf))
        target[dn] = np.nextafter(target[dn], np.float32(-np.inf))
    a = orc.bf16_to_f32(orc.f32_to_bf16(target))
    r1 = (target - a) * np.float32(256)
    b = orc.bf16_to_f32(orc.f32_to_bf16(r1))
    c = orc.bf16_to_f32(orc.f32_to_bf16((r1 - b) * np.float32(256)))
    x = np.zeros((T, d), np.float32)
    w = np.zeros((E, d), np.float32)
    e = np.arange(E)
    x[:, 3 * e], x[:, 3 * e + 1], x[:, 3 * e + 2] = a, b, c
    w[e, 3 * e], w[e, 3 * e + 1], w[e, 3 * e + 2] = 1.0, 2.0 ** -8, 2.0 ** -16
    xb = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    wb = torch.from_numpy(w).to(dev).to(torch.bfloat16)
    thr_d = torch.from_numpy(thr).to(dev)
    L = et.router_logits(xb, wb)
    near = (L - torch.from_numpy(l0).to(dev)).abs() <= 64 * torch.from_numpy(np.spacing(np.abs(l0))).to(dev)
    assert float(near[:, :-len(special)].float().mean()) > 0.99    # the logits really sit at the thresholds
    want = et.route(L, thr_d)
    _assert_plans_identical(et.router_route(xb, wb, thr_d), want)
    assert_route_equal(want, orc.route(host(L), thr))


def test_router_route_explicit_and_undersized_capacity(et, dev):
    T, d, E = 3000, 256, 64
    x, w = _router_case(dev, T, d, E, 9, 0.9)
    L = et.router_logits(x, w)
    thr = torch.quantile(torch.sigmoid(L.double()), 0.9, dim=0).float().contiguous()
    S = et.route(L, thr).num_slots
    for cap in (S, S // 2, 0):
        a = et.router_route(x, w, thr, slot_capacity=cap)
        b = et.route(L, thr, slot_capacity=cap)
        assert a.num_slots is None and a.capacity == cap
        _assert_plans_identical(a, b)


def test_router_route_full_size_c3(et, orc, dev):
    cfg = W.CONFIGS["C3"]
    T, d, E = cfg["T"], cfg["d"], cfg["E"]
    print(f"router_route C3 T={T} d={d} E={E}", flush=True)
    x, w = _router_case(dev, T, d, E, 31, 0.0)
    L = et.router_logits(x, w)
    lg = host(L)
    thr_h = W.thresholds("C3", lg)
    thr = torch.from_numpy(thr_h).to(dev)
    got = et.router_route(x, w, thr)
    _assert_plans_identical(got, et.route(L, thr))
    assert_route_equal(got, orc.route(lg, thr_h))
