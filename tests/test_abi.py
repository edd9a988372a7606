"""C-ABI checks that need no GPU: the library loads, exports every entry point
declared in include/etmoe.h, and rejects bad arguments before enqueueing any
device work (these calls return before touching the HIP runtime)."""
import ctypes
import os

import pytest

from conftest import ROOT

ET_ERR_INVALID_ARGUMENT = -1
ET_ERR_WORKSPACE_TOO_SMALL = -2


def test_library_exports_every_header_symbol(et):
    syms = et.header_symbols()
    assert len(syms) == 26
    lib = et.lib()
    for name in syms:
        assert hasattr(lib, name), name
    raw = ctypes.CDLL(et.LIB_PATH)                # plain dlopen/dlsym view as well
    for name in syms:
        assert getattr(raw, name) is not None


def test_abi_version_and_header_agree(et):
    hdr = open(os.path.join(ROOT, "include", "etmoe.h")).read()
    assert "#define ET_ABI_VERSION 11" in hdr
    assert et.lib().et_abi_version() == 11


def test_workspace_sizes(et):
    lib = et.lib()
    assert lib.et_route_workspace_bytes(65536, 128) >= 2 * 256 * 128 * 4
    assert lib.et_route_workspace_bytes(0, 8) > 0
    assert lib.et_route_workspace_bytes(10, 0) == 0
    # the pair lists hold room for every (token, expert) pair, 8 bytes each;
    # past 1 GiB of them et_route takes the two-read kernels, whose workspace
    # is O(E) per block
    assert lib.et_route_workspace_bytes(65536, 128) >= 65536 * 128 * 8
    assert lib.et_route_workspace_bytes(540000, 256) < (64 << 20)
    assert lib.et_route_workspace_bytes(2 ** 21, 1023) < (64 << 20)
    assert lib.et_threshold_workspace_bytes(131072, 64) >= 64 * 256 * 4 + 131072 * 64 * 4
    assert lib.et_threshold_workspace_bytes(10, 0) == 0


def _err(et):
    return et.lib().et_last_error().decode()


def test_route_rejects_bad_arguments_without_launching(et):
    lib = et.lib()
    ws = ctypes.c_void_p(0x1000)
    dummy = ctypes.c_void_p(0x2000)
    rc = lib.et_route(dummy, dummy, 16, 0, dummy, dummy, dummy, dummy, dummy, dummy, 16, ws, 1 << 20, None)
    assert rc == ET_ERR_INVALID_ARGUMENT and "num_experts" in _err(et)
    rc = lib.et_route(dummy, dummy, 16, 2000, dummy, dummy, dummy, dummy, dummy, dummy, 16, ws, 1 << 20, None)
    assert rc == ET_ERR_INVALID_ARGUMENT
    rc = lib.et_route(dummy, dummy, 1 << 26, 64, dummy, dummy, dummy, dummy, dummy, dummy, 16, ws, 1 << 30, None)
    assert rc == ET_ERR_INVALID_ARGUMENT and "2^31" in _err(et)
    rc = lib.et_route(None, dummy, 16, 4, dummy, dummy, dummy, dummy, dummy, dummy, 16, ws, 1 << 20, None)
    assert rc == ET_ERR_INVALID_ARGUMENT and "logits" in _err(et)
    rc = lib.et_route(dummy, dummy, 16, 4, dummy, dummy, dummy, None, dummy, dummy, 16, ws, 1 << 20, None)
    assert rc == ET_ERR_INVALID_ARGUMENT
    rc = lib.et_route(dummy, dummy, 4096, 8, dummy, dummy, dummy, dummy, dummy, dummy, 16, ws, 16, None)
    assert rc == ET_ERR_WORKSPACE_TOO_SMALL and "workspace" in _err(et)


def test_route_noalloc_rejects_bad_arguments_and_oversize_without_launching(et):
    """The no-allocation routing checks its arguments, then whether the
    workspace et_route would need fits the static scratch (8 MiB: every T up
    to E = 408), all before any HIP call."""
    lib = et.lib()
    d = ctypes.c_void_p(0x2000)
    rc = lib.et_route_noalloc(d, d, 16, 0, d, d, d, d, d, d, 16, None)
    assert rc == ET_ERR_INVALID_ARGUMENT and "et_route_noalloc" in _err(et) and "num_experts" in _err(et)
    rc = lib.et_route_noalloc(None, d, 16, 4, d, d, d, d, d, d, 16, None)
    assert rc == ET_ERR_INVALID_ARGUMENT and "logits" in _err(et)
    rc = lib.et_route_noalloc(d, d, 16, 4, d, d, d, None, d, d, 16, None)
    assert rc == ET_ERR_INVALID_ARGUMENT
    # The two-read routing it runs keeps O(E) counts per block (at most ~512
    # blocks): every T fits up to E = 408.  E = 409 and E = 1024 are rejected
    # with the sizes named (E = 408 runs, tests/test_zz_no_alloc.py).
    for E in (1024, 409):
        rc = lib.et_route_noalloc(d, d, 65536, E, d, d, d, d, d, d, 16, None)
        assert rc == ET_ERR_WORKSPACE_TOO_SMALL and "scratch" in _err(et) and str(8 << 20) in _err(et)


def test_row_entry_points_reject_bad_arguments(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    assert lib.et_dispatch_fwd(p, 8, 16, 7, p, p, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "dtype" in _err(et)
    assert lib.et_dispatch_fwd(p, -1, 16, 0, p, p, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_dispatch_fwd(p, 8, 16, 0, None, p, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_combine_fwd(p, None, p, p, 8, 16, 1, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_dispatch_bwd(p, p, p, 8, -3, 1, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_combine_bwd(p, p, p, p, p, p, None, 8, 4, 16, 0, 8, p, p, p, p, 1 << 20, None) == ET_ERR_INVALID_ARGUMENT
    assert "expert_offsets" in _err(et)
    assert lib.et_combine_bwd(p, p, p, None, p, p, p, 8, 4, 16, 0, 8, p, p, p, p, 1 << 20, None) == ET_ERR_INVALID_ARGUMENT
    assert "sorted_token" in _err(et)
    assert lib.et_combine_bwd(p, p, p, p, p, p, p, 8, 0, 16, 0, 8, p, p, p, p, 1 << 20, None) == ET_ERR_INVALID_ARGUMENT
    # zero-size work is a successful no-op that launches nothing
    assert lib.et_dispatch_fwd(p, 0, 16, 0, p, p, 8, p, None) == 0
    assert lib.et_combine_fwd(p, p, p, p, 0, 16, 0, 8, p, None) == 0


def test_threshold_update_rejects_bad_arguments(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    assert lib.et_threshold_update(p, p, 16, 8, 0, 0.99, None, p, 1 << 20, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_threshold_update(p, p, 16, 8, 9, 0.99, None, p, 1 << 20, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_threshold_update(p, p, 16, 8, 2, 1.5, None, p, 1 << 20, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_threshold_update(p, p, 16, 8, 2, float("nan"), None, p, 1 << 20, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_threshold_update(p, p, 16, 8, 2, 0.9, None, p, 8, None) == ET_ERR_WORKSPACE_TOO_SMALL
    # an empty batch is a no-op
    assert lib.et_threshold_update(p, p, 0, 8, 2, 0.9, None, p, 1 << 20, None) == 0


def test_route_update_rejects_bad_arguments(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    rws = lib.et_route_workspace_bytes(16, 8)
    tws = lib.et_threshold_workspace_bytes(16, 8)

    def call(T=16, E=8, cap=8, rwsb=rws, k=2, m=0.9, twsb=tws):
        return lib.et_route_update(p, p, T, E, p, p, p, p, p, p, cap, p, rwsb, k, m, None, p, twsb, None)

    assert call(k=0) == ET_ERR_INVALID_ARGUMENT               # the update's checks
    assert call(k=9) == ET_ERR_INVALID_ARGUMENT
    assert call(m=1.5) == ET_ERR_INVALID_ARGUMENT
    assert call(E=0) == ET_ERR_INVALID_ARGUMENT               # the routing's checks
    assert call(cap=-1) == ET_ERR_INVALID_ARGUMENT
    assert call(rwsb=8) == ET_ERR_WORKSPACE_TOO_SMALL
    assert call(twsb=8) == ET_ERR_WORKSPACE_TOO_SMALL
    assert "et_route_update" in _err(et)
    # the two workspaces are written at once: overlapping byte ranges are
    # refused before anything is enqueued (the same buffer, or slices of one)
    assert call() == ET_ERR_INVALID_ARGUMENT and "overlap" in _err(et)
    q = ctypes.c_void_p(0x1000 + rws - 256)
    rc = lib.et_route_update(p, p, 16, 8, p, p, p, p, p, p, 8, p, rws, 2, 0.9, None, q, tws, None)
    assert rc == ET_ERR_INVALID_ARGUMENT and "overlap" in _err(et)


def test_error_string_is_per_call(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    lib.et_dispatch_fwd(p, 8, 16, 9, p, p, 8, p, None)
    first = _err(et)
    lib.et_threshold_update(p, p, 16, 8, 0, 0.99, None, p, 1 << 20, None)
    assert _err(et) != first and "k_target" in _err(et)


def test_combine_bwd_workspace(et):
    lib = et.lib()
    # one binary64 partial per slot and 2 KiB of the row (one wave's two 1 KiB pieces; C3:
    # d = 4096 bf16 -> 4 partials; d = 512 f32 -> 1), then the slot walk order (one int32
    # per slot) from a 256-byte boundary
    r = lambda x: (x + 255) // 256 * 256
    assert lib.et_combine_bwd_workspace_bytes(65536, 528736, 4096, 1) == r(528736 * 4 * 8) + 528736 * 4
    assert lib.et_combine_bwd_workspace_bytes(4096, 8191, 512, 0) == r(8191 * 1 * 8) + 8191 * 4
    assert lib.et_combine_bwd_workspace_bytes(1, 8191, 512, 0) == r(8191 * 1 * 8) + 8191 * 4
    assert lib.et_combine_bwd_workspace_bytes(1, 100, 4104, 1) == r(100 * 5 * 8) + 100 * 4   # 9 pieces, 5 waves
    assert lib.et_combine_bwd_workspace_bytes(10, 100, 7, 1) == 0        # element path: none
    assert lib.et_combine_bwd_workspace_bytes(10, 100, 8, 5) == 0        # bad dtype
    p = ctypes.c_void_p(0x1000)                   # 16-byte aligned: the vector path is chosen
    rc = lib.et_combine_bwd(p, p, p, p, p, p, p, 8, 4, 64, 1, 8, p, p, p, None, 0, None)
    assert rc == ET_ERR_WORKSPACE_TOO_SMALL and "workspace" in _err(et)
    rc = lib.et_combine_bwd(p, p, p, p, p, p, p, 8, 4, 64, 1, 8, p, p, p, p, 63, None)
    assert rc == ET_ERR_WORKSPACE_TOO_SMALL
    need = lib.et_combine_bwd_workspace_bytes(8, 8, 64, 1)
    odd = ctypes.c_void_p(0x1004)                 # the binary64 partials need 8-byte alignment
    rc = lib.et_combine_bwd(p, p, p, p, p, p, p, 8, 4, 64, 1, 8, p, p, p, odd, need, None)
    assert rc == ET_ERR_INVALID_ARGUMENT and "aligned" in _err(et)


def test_router_logits_rejects_bad_arguments(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    assert lib.et_router_logits(p, p, 16, 64, 0, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "num_experts" in _err(et)
    assert lib.et_router_logits(p, p, 16, 64, 257, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_router_logits(p, p, 16, 12, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "multiple of 8" in _err(et)
    assert lib.et_router_logits(p, p, -1, 64, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_router_logits(p, None, 16, 64, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_router_logits(ctypes.c_void_p(0x1008), p, 16, 64, 8, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "aligned" in _err(et)
    assert lib.et_router_logits(p, p, 1 << 25, 64, 128, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_router_logits(p, p, 0, 64, 8, p, None) == 0      # no tokens: nothing to do


def test_expert_gemm_rejects_bad_arguments(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    # (a, a_rows, sorted_token, w, expert_offsets, E, K, N, slot_capacity, epilogue, row_scale, c, stream)
    assert lib.et_expert_gemm(p, 16, p, p, p, 0, 64, 64, 16, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "num_experts" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 1025, 64, 64, 16, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 60, 64, 16, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "K must" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 64, 12, 16, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "N must" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 64, 64, 16, 3, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "epilogue" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 64, 24, 16, 2, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "SwiGLU" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 64, 64, 16, 1, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "row_scale" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 1 << 16, 1 << 14, 16, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "2 GiB" in _err(et)
    assert lib.et_expert_gemm(p, 1 << 20, p, p, p, 4, 4096, 64, 16, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "gather" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 64, 64, -1, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_expert_gemm(p, 16, p, p, None, 4, 64, 64, 16, 0, None, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "null" in _err(et)
    assert lib.et_expert_gemm(ctypes.c_void_p(0x1008), 16, p, p, p, 4, 64, 64, 16, 0, None, p, None) \
        == ET_ERR_INVALID_ARGUMENT
    assert "aligned" in _err(et)
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 64, 64, 16, 0, None, ctypes.c_void_p(0x1008), None) \
        == ET_ERR_INVALID_ARGUMENT
    # no slot rows: nothing to do, nothing launched
    assert lib.et_expert_gemm(p, 16, p, p, p, 4, 64, 64, 0, 0, None, p, None) == 0


def test_swiglu_rejects_bad_arguments(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    # et_swiglu_fwd(gu, F, expert_offsets, E, slot_capacity, h, stream)
    assert lib.et_swiglu_fwd(p, 12, p, 4, 16, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "multiple of 8" in _err(et)
    assert lib.et_swiglu_fwd(p, 16, p, 0, 16, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "num_experts" in _err(et)
    assert lib.et_swiglu_fwd(p, 16, p, 4, -1, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_swiglu_fwd(p, 16, None, 4, 16, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "null" in _err(et)
    assert lib.et_swiglu_fwd(ctypes.c_void_p(0x1008), 16, p, 4, 16, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "aligned" in _err(et)
    # et_swiglu_bwd(gu, dh, F, expert_offsets, E, slot_capacity, dgu, stream)
    assert lib.et_swiglu_bwd(p, None, 16, p, 4, 16, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "null" in _err(et)
    assert lib.et_swiglu_bwd(p, ctypes.c_void_p(0x1004), 16, p, 4, 16, p, None) == ET_ERR_INVALID_ARGUMENT
    assert lib.et_swiglu_bwd(p, p, 0, p, 4, 16, p, None) == ET_ERR_INVALID_ARGUMENT
    # no slot rows: nothing to do, nothing launched
    assert lib.et_swiglu_fwd(p, 16, p, 4, 0, p, None) == 0
    assert lib.et_swiglu_bwd(p, p, 16, p, 4, 0, p, None) == 0


def test_expert_gemm_fp8_rejects_bad_arguments(et):
    lib = et.lib()
    p = ctypes.c_void_p(0x1000)
    # (a, a_rows, a_scale, sorted_token, w, w_scale, expert_offsets, E, K, N, slot_capacity, epilogue, c, stream)
    assert lib.et_expert_gemm_fp8(p, 16, p, p, p, p, p, 4, 72, 64, 16, 0, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "multiple of 16" in _err(et)
    assert lib.et_expert_gemm_fp8(p, 16, p, p, p, p, p, 4, 64, 64, 16, 1, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "plain and SwiGLU" in _err(et)
    assert lib.et_expert_gemm_fp8(p, 16, None, p, p, p, p, 4, 64, 64, 16, 0, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "a_scale" in _err(et)
    assert lib.et_expert_gemm_fp8(p, 16, p, p, p, ctypes.c_void_p(0x1002), p, 4, 64, 64, 16, 0, p, None) \
        == ET_ERR_INVALID_ARGUMENT
    assert "w_scale" in _err(et)
    assert lib.et_expert_gemm_fp8(p, 16, p, p, p, p, p, 4, 64, 24, 16, 2, p, None) == ET_ERR_INVALID_ARGUMENT
    assert "SwiGLU" in _err(et)
    assert lib.et_expert_gemm_fp8(p, 16, p, p, p, p, p, 4, 64, 64, 0, 0, p, None) == 0   # nothing to do
