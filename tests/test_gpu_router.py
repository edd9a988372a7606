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
