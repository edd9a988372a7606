"""CPU oracle for the Expert-Threshold MoE dispatch path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (bench.py also times it as
the CPU baseline).  The product library never imports, links or falls back to it.

The functions wrap ``etmoe_oracle.c`` (built into ``liboracle_etmoe.so`` by the
Makefile beside it) over numpy arrays.  The reference tree has no
implementation of this path (it is an agent-launcher CLI; see the header of
``etmoe_oracle.c``), so parity against the reference is unpinned for every
function here; each is pinned against independent mathematics in
``tests/test_oracle.py`` instead.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_etmoe.so")

DT_F32 = 0
DT_BF16 = 1

_i64 = ctypes.c_int64
_p = ctypes.c_void_p


def build(force: bool = False) -> str:
    """Compile the C restatement with the committed Makefile."""
    src = os.path.join(_HERE, "etmoe_oracle.c")
    stale = not os.path.exists(_LIB_PATH) or (
        os.path.exists(src) and os.path.getmtime(src) > os.path.getmtime(_LIB_PATH))
    if force or stale:
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []),
                       check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_bf16_to_f32.restype = ctypes.c_float
        L.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_exp_nonpos.restype = ctypes.c_float
        L.oracle_exp_nonpos.argtypes = [ctypes.c_float]
        L.oracle_sigmoid.restype = ctypes.c_float
        L.oracle_sigmoid.argtypes = [ctypes.c_float]
        L.oracle_swiglu.restype = ctypes.c_float
        L.oracle_swiglu.argtypes = [ctypes.c_float, ctypes.c_float]
        L.oracle_swiglu_grad_f32.restype = None
        L.oracle_swiglu_grad_f32.argtypes = [_p, _p, _p, _i64, _p, _p]
        L.oracle_swiglu_f32.restype = None
        L.oracle_swiglu_f32.argtypes = [_p, _p, _i64, _p]
        L.oracle_swiglu_fwd_rows.restype = None
        L.oracle_swiglu_fwd_rows.argtypes = [_p, _i64, _i64, _p]
        L.oracle_swiglu_bwd_rows.restype = None
        L.oracle_swiglu_bwd_rows.argtypes = [_p, _p, _i64, _i64, _p]
        L.oracle_sigmoid_order_scan.restype = None
        L.oracle_sigmoid_order_scan.argtypes = [ctypes.c_uint64, ctypes.c_uint64, _p]
        L.oracle_select.restype = _i64
        L.oracle_select.argtypes = [_p, _p, _i64, _i64, _p, _p]
        L.oracle_route.restype = _i64
        L.oracle_route.argtypes = [_p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64]
        L.oracle_dispatch_fwd.restype = None
        L.oracle_dispatch_fwd.argtypes = [_p, _i64, _i64, ctypes.c_int, _p, _p, _p]
        L.oracle_combine_fwd.restype = None
        L.oracle_combine_fwd.argtypes = [_p, _p, _p, _p, _i64, _i64, ctypes.c_int, _p]
        L.oracle_dispatch_bwd.restype = None
        L.oracle_dispatch_bwd.argtypes = [_p, _p, _p, _i64, _i64, ctypes.c_int, _p]
        L.oracle_dispatch_bwd_router.restype = None
        L.oracle_dispatch_bwd_router.argtypes = [_p, _p, _p, _p, _i64, _p, _p, _p, _i64, _i64, ctypes.c_int, _p]
        L.oracle_combine_bwd.restype = None
        L.oracle_combine_bwd.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64,
                                         ctypes.c_int, _p, _p, _p]
        L.oracle_set_threads.restype = ctypes.c_int
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        L.oracle_threshold_update.restype = _i64
        L.oracle_threshold_update.argtypes = [_p, _p, _i64, _i64, _i64, ctypes.c_float, _p]
        _lib = L
    return _lib


def set_threads(n: int) -> int:
    """Threads of the oracle's parallel loops (OpenMP); returns the count in
    use.  Results are the same bits for any count."""
    return int(lib().oracle_set_threads(int(n)))


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _act_dt(a: np.ndarray) -> int:
    """Activations are float32 arrays, or bfloat16 stored as uint16 words."""
    if a.dtype == np.float32:
        return DT_F32
    if a.dtype == np.uint16:
        return DT_BF16
    raise TypeError(f"activation dtype must be float32 or uint16 (bf16 bits), got {a.dtype}")


# --------------------------------------------------------------------------- #
# scalar helpers
# --------------------------------------------------------------------------- #

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round-to-nearest-even."""
    x = _c(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x0040).astype(np.uint16)
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def sigmoid_order_scan(k0: int, k1: int) -> tuple:
    """(largest deficit below the running max in order steps, smallest score
    bits, largest score bits, negative scores) of the specified sigmoid over
    the floats with order index in [k0, k1) (oracle_sigmoid_order_scan)."""
    out = np.zeros(4, np.uint32)
    lib().oracle_sigmoid_order_scan(k0, k1, out.ctypes.data)
    return tuple(int(v) for v in out)


def sigmoid(logits: np.ndarray) -> np.ndarray:
    """Element-wise specified sigmoid (slow scalar loop through ctypes; tests only)."""
    L = lib()
    flat = _c(logits, np.float32).ravel()
    out = np.empty_like(flat)
    for i, v in enumerate(flat):
        out[i] = L.oracle_sigmoid(float(v))
    return out.reshape(np.shape(logits))


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """Element-wise (g * sigmoid(g)) * u in binary32 (oracle_swiglu; tests only)."""
    gf = _c(g, np.float32).ravel()
    uf = _c(u, np.float32).ravel()
    out = np.empty_like(gf)
    lib().oracle_swiglu_f32(_ptr(gf), _ptr(uf), gf.size, _ptr(out))
    return out.reshape(np.shape(g))


def swiglu_grad(g: np.ndarray, u: np.ndarray, dh: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(dg, du) of h = (g * sigmoid(g)) * u for upstream dh, binary32
    (oracle_swiglu_grad; tests only)."""
    gf, uf, df = (_c(x, np.float32).ravel() for x in (g, u, dh))
    dg, du = np.empty_like(gf), np.empty_like(gf)
    lib().oracle_swiglu_grad_f32(_ptr(gf), _ptr(uf), _ptr(df), gf.size, _ptr(dg), _ptr(du))
    return dg.reshape(np.shape(g)), du.reshape(np.shape(g))


def swiglu_rows(gu_bits: np.ndarray) -> np.ndarray:
    """bf16 bits [n, F] of h from bf16 bits gu [n, 2F] (oracle_swiglu_fwd_rows)."""
    gu = _c(gu_bits, np.uint16)
    n, F2 = gu.shape
    h = np.empty((n, F2 // 2), dtype=np.uint16)
    lib().oracle_swiglu_fwd_rows(_ptr(gu), n, F2 // 2, _ptr(h))
    return h


def swiglu_backward_rows(gu_bits: np.ndarray, dh_bits: np.ndarray) -> np.ndarray:
    """bf16 bits [n, 2F] of (dg | du) from bf16 bits gu [n, 2F] and dh [n, F]
    (oracle_swiglu_bwd_rows)."""
    gu = _c(gu_bits, np.uint16)
    dh = _c(dh_bits, np.uint16)
    n, F2 = gu.shape
    assert dh.shape == (n, F2 // 2)
    out = np.empty_like(gu)
    lib().oracle_swiglu_bwd_rows(_ptr(gu), _ptr(dh), n, F2 // 2, _ptr(out))
    return out


def exp_nonpos(x: np.ndarray) -> np.ndarray:
    L = lib()
    flat = _c(x, np.float32).ravel()
    out = np.empty_like(flat)
    for i, v in enumerate(flat):
        out[i] = L.oracle_exp_nonpos(float(v))
    return out.reshape(np.shape(x))


# --------------------------------------------------------------------------- #
# routing
# --------------------------------------------------------------------------- #

def select(logits: np.ndarray, thr: np.ndarray):
    """Selection matrix (uint8 [T,E]) and scores (float32 [T,E]) of the spec."""
    logits = _c(logits, np.float32)
    thr = _c(thr, np.float32)
    T, E = logits.shape
    sel = np.zeros((T, E), np.uint8)
    score = np.zeros((T, E), np.float32)
    S = lib().oracle_select(_ptr(logits), _ptr(thr), T, E, _ptr(sel), _ptr(score))
    return sel, score, int(S)


@dataclass
class Routing:
    counts: np.ndarray          # int32 [E]
    expert_offsets: np.ndarray  # int32 [E+1]
    token_offsets: np.ndarray   # int32 [T+1]
    sorted_token: np.ndarray    # int32 [S]
    slot_gate: np.ndarray       # float32 [S]
    token_slot: np.ndarray      # int32 [S]

    @property
    def num_slots(self) -> int:
        return int(self.expert_offsets[-1])


def route(logits: np.ndarray, thr: np.ndarray) -> Routing:
    logits = _c(logits, np.float32)
    thr = _c(thr, np.float32)
    T, E = logits.shape
    assert thr.shape == (E,)
    cap = max(T * E, 1)
    counts = np.zeros(E, np.int32)
    eo = np.zeros(E + 1, np.int32)
    to = np.zeros(T + 1, np.int32)
    st = np.zeros(cap, np.int32)
    sg = np.zeros(cap, np.float32)
    ts = np.zeros(cap, np.int32)
    S = lib().oracle_route(_ptr(logits), _ptr(thr), T, E, _ptr(counts), _ptr(eo), _ptr(to),
                           _ptr(st), _ptr(sg), _ptr(ts), cap)
    if S < 0:
        raise MemoryError("oracle_route: allocation failed")
    return Routing(counts, eo, to, st[:S].copy(), sg[:S].copy(), ts[:S].copy())


# --------------------------------------------------------------------------- #
# dispatch / combine
# --------------------------------------------------------------------------- #

def _out(out, shape, dtype):
    """A caller-supplied output array (checked), or a new zeroed one."""
    if out is None:
        return np.zeros(shape, dtype)
    if out.shape != tuple(shape) or out.dtype != dtype or not out.flags.c_contiguous:
        raise ValueError(f"out must be a contiguous {dtype} array of shape {tuple(shape)}")
    return out


def dispatch_fwd(x: np.ndarray, r: Routing, out: np.ndarray | None = None) -> np.ndarray:
    dt = _act_dt(x)
    x = np.ascontiguousarray(x)
    T, d = x.shape
    xp = _out(out, (r.num_slots, d), x.dtype)
    lib().oracle_dispatch_fwd(_ptr(x), T, d, dt, _ptr(r.token_offsets), _ptr(r.token_slot), _ptr(xp))
    return xp


def combine_fwd(yp: np.ndarray, r: Routing, T: int, out: np.ndarray | None = None) -> np.ndarray:
    dt = _act_dt(yp)
    yp = np.ascontiguousarray(yp)
    d = yp.shape[1]
    y = _out(out, (T, d), yp.dtype)
    lib().oracle_combine_fwd(_ptr(yp), _ptr(r.slot_gate), _ptr(r.token_offsets),
                             _ptr(r.token_slot), T, d, dt, _ptr(y))
    return y


def dispatch_bwd(dxp: np.ndarray, r: Routing, T: int, out: np.ndarray | None = None) -> np.ndarray:
    dt = _act_dt(dxp)
    dxp = np.ascontiguousarray(dxp)
    d = dxp.shape[1]
    dx = _out(out, (T, d), dxp.dtype)
    lib().oracle_dispatch_bwd(_ptr(dxp), _ptr(r.token_offsets), _ptr(r.token_slot), T, d, dt, _ptr(dx))
    return dx


def dispatch_bwd_router(dxp: np.ndarray, r: Routing, T: int, dgate: np.ndarray, w: np.ndarray) -> np.ndarray:
    """dX = dispatch backward + dlogits . W through the routed pairs, with the
    per-slot dl = dgate * (g * (1 - g)) (see oracle_dispatch_bwd_router)."""
    dt = _act_dt(dxp)
    assert _act_dt(w) == dt
    dxp = np.ascontiguousarray(dxp)
    w = np.ascontiguousarray(w)
    dgate = np.ascontiguousarray(dgate, np.float32)
    d = dxp.shape[1]
    E = w.shape[0]
    dx = np.zeros((T, d), dxp.dtype)
    lib().oracle_dispatch_bwd_router(_ptr(dxp), _ptr(r.token_offsets), _ptr(r.token_slot),
                                     _ptr(r.expert_offsets), E, _ptr(r.slot_gate), _ptr(dgate), _ptr(w),
                                     T, d, dt, _ptr(dx))
    return dx


def combine_bwd(dy: np.ndarray, yp: np.ndarray, r: Routing, E: int, want_dlogits: bool = False,
                out: tuple | None = None):
    """(dYp, dgate, dlogits or None); `out` optionally supplies the arrays."""
    dt = _act_dt(dy)
    assert _act_dt(yp) == dt
    dy = np.ascontiguousarray(dy)
    yp = np.ascontiguousarray(yp)
    T, d = dy.shape
    o = out if out is not None else (None, None, None)
    dyp = _out(o[0], (r.num_slots, d), dy.dtype)
    dgate = _out(o[1], (r.num_slots,), np.float32)
    dlogits = _out(o[2], (T, E), np.float32) if want_dlogits else None
    lib().oracle_combine_bwd(_ptr(dy), _ptr(yp), _ptr(r.slot_gate), _ptr(r.sorted_token),
                             _ptr(r.expert_offsets), T, E, d, dt, _ptr(dyp), _ptr(dgate),
                             _ptr(dlogits))
    return dyp, dgate, dlogits


# --------------------------------------------------------------------------- #
# EMA threshold update
# --------------------------------------------------------------------------- #

def capacity(T: int, E: int, k_target: int) -> int:
    c = (T * k_target + E - 1) // E
    return min(max(c, 1), T)


def threshold_update(logits: np.ndarray, thr: np.ndarray, k_target: int, momentum: float = 0.99):
    """Returns (new_thr, stat); the input thr array is not modified."""
    logits = _c(logits, np.float32)
    T, E = logits.shape
    thr = np.array(thr, dtype=np.float32, copy=True)
    stat = np.full(E, np.nan, np.float32)
    c = lib().oracle_threshold_update(_ptr(logits), _ptr(thr), T, E, k_target,
                                      float(np.float32(momentum)), _ptr(stat))
    if c < 0:
        raise MemoryError("oracle_threshold_update: allocation failed")
    return thr, stat
