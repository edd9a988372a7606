"""Seeded random shapes through the whole path on the GPU, against the CPU
oracle: routing (bit-exact), dispatch, combine and dispatch backward (bit-exact),
combine backward (dYp bit-exact, dgate within one binary32 ulp of the oracle
plus the binary64 summation floor, dlogits bit-exact from dgate), the dispatch backward with the router input gradient (bit-exact), and,
where the shape allows it (bf16, E <= 256, d a multiple of 8), the router
logits GEMM (exact on integer inputs) and the fused producer + routing
(bit-identical to router_logits + route).

Each case draws T, E, d, the activation dtype and a routing mode (per-expert
quantile thresholds, all-fallback, all-selected, NaN/inf/tie specials); sizes
are kept small enough for the oracle to finish in well under a second."""
import numpy as np
import pytest
import torch

from test_gpu_parity import check_rows, dev_f32, host, make_rows, synthetic_router, to_dev

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
