"""Seeded random shapes through the whole path on the GPU, against the CPU
oracle: routing (bit-exact), dispatch, combine and dispatch backward (bit-exact),
combine backward (dYp bit-exact, dgate within one binary32 ulp of the oracle
plus the binary64 summation floor, dlogits bit-exact from dgate), the dispatch backward with the router input gradient (bit-exact), and,
where the shape allows it (bf16, E <= 256, d a multiple of 8), the router
logits GEMM (exact on integer inputs) and the fused producer + routing
(bit-identical to router_logits + route).

Each case draws T, E, d, the activation dtype and a routing mode (per-expert
quantile thresholds, all-fallback, all-selected, NaN/inf/tie specials); sizes
are kept small enough for the oracle to finish in well under a second.  Those
shapes all walk combine backward's slots in plain slot order (dY <= 16 MiB), so
a second set draws shapes above that size with more than 1.25 slots per token,
which take the token-window walk.  A third set draws wider routing shapes (T up
to 20000, E up to 1024) and threshold regimes, logits at the thresholds
included, for routing and the EMA update alone."""
import numpy as np
import pytest
import torch

from test_gpu_parity import (assert_dgate, assert_dlogits, bits, check_rows, dev_f32, host, make_rows,
                             synthetic_router, to_dev)

pytestmark = pytest.mark.gpu

E_CHOICES = [1, 2, 3, 5, 8, 13, 31, 32, 33, 64, 65, 100, 127, 128, 129, 200, 256, 300, 513]
D_CHOICES = [1, 3, 7, 8, 12, 16, 24, 64, 100, 128, 264, 520, 1024, 1032, 2056]
MODES = ["quantile", "quantile", "fallback", "all", "special"]


def draw(seed):
    rng = np.random.default_rng([2024, seed])
    E = int(rng.choice(E_CHOICES))
    d = int(rng.choice(D_CHOICES))
    mode = str(rng.choice(MODES))
    dtype = str(rng.choice(["f32", "bf16"]))
    T = int(rng.integers(1, 400))
    k = E if mode == "all" else 4
    T = max(1, min(T, int(3e6 // max(1, k * d))))      # S * d stays near 3M elements or below
    return T, d, E, dtype, mode


@pytest.mark.parametrize("seed", range(48))
def test_random_shape_whole_path(et, orc, dev, seed):
    T, d, E, dtype, mode = draw(seed)
    print(f"random case {seed}: T={T} d={d} E={E} {dtype} {mode}", flush=True)
    lg, thr = synthetic_router(T, E, mode, seed)
    check_rows(et, orc, dev, lg, thr, d, dtype, seed=seed)

    # dispatch backward with the router input gradient
    r = orc.route(lg, thr)
    plan = et.route(dev_f32(lg, dev), dev_f32(thr, dev))
    _, _, _, dxp = make_rows(orc, r, T, d, dtype, seed + 1)
    rng = np.random.default_rng([seed, 77])
    w = rng.standard_normal((E, d)).astype(np.float32)
    if dtype == "bf16":
        w = orc.f32_to_bf16(w)
    dgate = rng.standard_normal(r.num_slots).astype(np.float32)
    dx = et.dispatch_backward(to_dev(dxp, dev), plan, router_weight=to_dev(w, dev), dgate=dev_f32(dgate, dev))
    want = orc.dispatch_bwd_router(dxp, r, T, dgate, w)
    got = host(dx)
    np.testing.assert_array_equal(got.view(np.uint16) if got.dtype == np.uint16 else got.view(np.uint32),
                                  want.view(np.uint16) if want.dtype == np.uint16 else want.view(np.uint32))

    # router producer, where its shape constraints hold
    if dtype == "bf16" and E <= 256 and d % 8 == 0:
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        xi = torch.randint(-4, 5, (T, d), generator=g, device=dev).to(torch.bfloat16)
        wi = torch.randint(-4, 5, (E, d), generator=g, device=dev).to(torch.bfloat16)
        L = et.router_logits(xi, wi)
        assert torch.equal(L.double(), xi.double() @ wi.double().T)
        xs = torch.randn(T, d, generator=g, device=dev).to(torch.bfloat16)
        ws = (torch.randn(E, d, generator=g, device=dev) * d ** -0.5).to(torch.bfloat16)
        Ls = et.router_logits(xs, ws)
        thr_d = dev_f32(thr, dev)
        a = et.route(Ls, thr_d)
        b = et.router_route(xs, ws, thr_d)
        for f in ("counts", "expert_offsets", "token_offsets", "sorted_token", "token_slot"):
            assert torch.equal(getattr(a, f), getattr(b, f)), f
        assert torch.equal(a.slot_gate.view(torch.int32), b.slot_gate.view(torch.int32))


def draw_windowed(seed):
    """A shape whose combine backward walks token windows: dY above 16 MiB
    and more than 1.25 slots per token (so the quantile or all-selected
    routing), with S * d kept near 40M elements or below."""
    rng = np.random.default_rng([2025, seed])
    dtype = str(rng.choice(["f32", "bf16"]))
    b = 4 if dtype == "f32" else 2
    mode = str(rng.choice(["quantile", "quantile", "all"]))
    d = int(rng.choice([1032, 2048, 3000, 4096, 8192, 12288]))
    t_min = (16 << 20) // (d * b) + 1
    # quantile routing selects about E / 4 experts per token: keep S * d <= 60M
    e_max = 60e6 / (0.25 * d * t_min)
    E = (int(rng.choice([e for e in [6, 8, 13, 31, 33, 64, 65, 100, 129] if e <= e_max] or [6]))
         if mode == "quantile" else int(rng.choice([2, 3, 4])))
    k = E * 0.25 if mode == "quantile" else E
    t_max = max(t_min, int(40e6 // max(1.0, k * d)))
    T = int(rng.integers(t_min, max(t_min + 1, min(t_max, 3 * t_min))))
    return T, d, E, dtype, mode


@pytest.mark.parametrize("seed", range(12))
def test_random_shape_windowed_combine_backward(et, orc, dev, seed):
    """Combine backward on random shapes that take the token-window walk
    (windows of 3 MiB of dY rows, so 2 to ~30 windows, the last one ragged):
    dYp bit-exact, dgate within the binary32 bar, dlogits bit-exact from
    dgate, against the oracle; also with spare slot capacity."""
    T, d, E, dtype, mode = draw_windowed(seed)
    print(f"windowed case {seed}: T={T} d={d} E={E} {dtype} {mode}", flush=True)
    lg, thr = synthetic_router(T, E, mode, seed)
    r = orc.route(lg, thr)
    S = r.num_slots
    assert S * 4 > T * 5 and T * d * (4 if dtype == "f32" else 2) > 16 << 20    # the windowed rule holds
    plan = et.route(dev_f32(lg, dev), dev_f32(thr, dev))
    _, yp, dy, _ = make_rows(orc, r, T, d, dtype, seed)
    DY, YP = to_dev(dy, dev), to_dev(yp, dev)
    dyp_g, dgate_g, dl_g = et.combine_backward(DY, YP, plan, need_dlogits=True)
    dyp_o, dgate_o, _ = orc.combine_bwd(dy, yp, r, E, want_dlogits=True)
    np.testing.assert_array_equal(bits(host(dyp_g)), bits(dyp_o))
    cvt = orc.bf16_to_f32 if dtype == "bf16" else (lambda a: a)
    mass = np.einsum("sd,sd->s", np.abs(cvt(dy)[r.sorted_token].astype(np.float64)),
                     np.abs(cvt(yp).astype(np.float64)))
    dgate_h = host(dgate_g)
    assert_dgate(dgate_h, dgate_o, mass, d)
    assert_dlogits(host(dl_g), dgate_h, r, E)
    spare = et.route(dev_f32(lg, dev), dev_f32(thr, dev), slot_capacity=S + 129)
    YP2 = torch.cat([YP, torch.zeros(129, d, dtype=YP.dtype, device=dev)])
    dyp_b, dgate_b, dl_b = et.combine_backward(DY, YP2, spare, need_dlogits=True)
    iv = (lambda t: t.view(torch.int16)) if dtype == "bf16" else (lambda t: t.view(torch.int32))
    assert torch.equal(iv(dyp_b[:S]), iv(dyp_g))
    assert torch.equal(dgate_b[:S].view(torch.int32), dgate_g.view(torch.int32))
    assert torch.equal(dl_b.view(torch.int32), dl_g.view(torch.int32))


# --------------------------------------------------------------------------- #
# routing and the EMA update alone, over wider shapes
# --------------------------------------------------------------------------- #

R_E_CHOICES = [1, 4, 7, 8, 31, 64, 65, 128, 200, 256, 400, 512, 777, 1024]


def route_case(seed):
    """T up to 20000 tokens, E up to 1024, and a threshold regime: per-expert
    quantiles, a high common threshold (many argmax fallbacks), zero (every
    pair), or logits placed within a few float steps of each threshold's
    logit (so the bounds decide nothing and the exact scores do), with NaN
    and +-inf mixed in."""
    rng = np.random.default_rng([4096, seed])
    E = int(rng.choice(R_E_CHOICES))
    T = int(rng.integers(1, max(2, min(20000, 4_000_000 // E))))
    mode = str(rng.choice(["quantile", "high", "zero", "edge"]))
    lg = (rng.standard_normal((T, E)) * rng.choice([0.5, 1.5, 4.0])).astype(np.float32)
    if mode == "quantile":
        thr = np.quantile(1 / (1 + np.exp(-lg.astype(np.float64))), rng.uniform(0.5, 0.99), axis=0).astype(np.float32)
    elif mode == "high":
        thr = np.full(E, 0.999, np.float32)
    elif mode == "zero":
        thr = np.zeros(E, np.float32)
    else:
        l0 = (rng.standard_normal(E) * 2).astype(np.float32)
        thr = (1 / (1 + np.exp(-l0.astype(np.float64)))).astype(np.float32)
        steps = rng.integers(-6, 7, size=(T, E))
        lg = np.repeat(l0[None, :], T, 0)
        for s_ in range(1, 7):
            up, dn = steps >= s_, steps <= -s_
            lg[up] = np.nextafter(lg[up], np.float32(np.inf))
            lg[dn] = np.nextafter(lg[dn], np.float32(-np.inf))
    lg = np.ascontiguousarray(lg, np.float32)
    lg[rng.random((T, E)) < 0.003] = np.nan
    lg[rng.random((T, E)) < 0.002] = np.inf
    lg[rng.random((T, E)) < 0.002] = -np.inf
    return T, E, mode, lg, thr


@pytest.mark.parametrize("seed", range(40))
def test_random_routing_and_threshold_update(et, orc, dev, seed):
    """Routing bit-exact with the oracle on each drawn case, then the EMA
    update (statistic and thresholds) bit-exact for a drawn k_target, alone
    and in route_update."""
    from test_gpu_parity import assert_route_equal

    T, E, mode, lg, thr = route_case(seed)
    print(f"route/update case {seed}: T={T} E={E} {mode}", flush=True)
    L = dev_f32(lg, dev)
    assert_route_equal(et.route(L, dev_f32(thr, dev)), orc.route(lg, thr))
    k = int(np.random.default_rng([seed, 9]).integers(1, E + 1))
    thr0 = np.random.default_rng([seed, 10]).random(E).astype(np.float32)
    thr_o, stat_o = orc.threshold_update(lg, thr0, k, 0.99)
    t = dev_f32(thr0, dev)
    stat = et.threshold_update_(t, L, k, 0.99)
    np.testing.assert_array_equal(bits(host(stat)), bits(stat_o))
    np.testing.assert_array_equal(bits(host(t)), bits(thr_o))
    # route_update: routes with thr, then updates it (E <= 256 takes the
    # digit histograms from the routing pass)
    thr_o2, stat_o2 = orc.threshold_update(lg, thr, k, 0.99)
    t2 = dev_f32(thr, dev)
    stat2 = torch.empty(E, device=dev)
    plan = et.route_update(L, t2, k, 0.99, stat=stat2)
    assert_route_equal(plan, orc.route(lg, thr))
    np.testing.assert_array_equal(bits(host(stat2)), bits(stat_o2))
    np.testing.assert_array_equal(bits(host(t2)), bits(thr_o2))
