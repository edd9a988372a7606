// et_rows.hip -- the row-moving kernels of the path on gfx950: dispatch
// (permute), combine (gate-weighted un-permute), combine backward (dYp, dgate,
// dlogits) and dispatch backward (dX, optionally with the router's input
// gradient dlogits . W added in the same pass).
//
// All four are token-major: a token's slot list token_slot[token_offsets[t] ..
// token_offsets[t+1]) is read by the waves that own the token, and whole rows
// move.  Token-major order is what makes the traffic minimal: X and dY rows are
// read exactly once (then written or consumed k_t times from registers), Y and
// dX rows are written exactly once, and sums over a token's slots are formed in
// registers in ascending expert order without atomics.
//
// Vector path: rows whose byte size is a multiple of 16 move as 16-byte chunks,
// 64 lanes x 16 B = 1 KiB per wave instruction (fully coalesced).  Every row
// kernel splits a row into 1 KiB pieces with one wave each; combine backward
// writes one partial dot product per (slot, piece), and a slot-parallel finish
// kernel sums them in piece order into dgate and dlogits.  Rows of other sizes
// take the element path.
#include <algorithm>

#include "et_common.hpp"

namespace et {

constexpr int kRowWaves = 4;
constexpr int kRowThreads = kRowWaves * kWave;

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4u ld16(const char* p) { return *reinterpret_cast<const v4u*>(p); }
__device__ __forceinline__ void st16(char* p, v4u v) { *reinterpret_cast<v4u*>(p) = v; }

template <int DT> struct Pack;

template <> struct Pack<ET_DTYPE_F32> {
    static constexpr int N = 4;
    __device__ static __forceinline__ void unpack(v4u w, float* f)
    {
        f[0] = u2f(w.x); f[1] = u2f(w.y); f[2] = u2f(w.z); f[3] = u2f(w.w);
    }
    __device__ static __forceinline__ v4u pack(const float* f)
    {
        v4u w;
        w.x = f2u(f[0]); w.y = f2u(f[1]); w.z = f2u(f[2]); w.w = f2u(f[3]);
        return w;
    }
};

template <> struct Pack<ET_DTYPE_BF16> {
    static constexpr int N = 8;
    __device__ static __forceinline__ void unpack(v4u w, float* f)
    {
        f[0] = bf16lo(w.x); f[1] = bf16hi(w.x); f[2] = bf16lo(w.y); f[3] = bf16hi(w.y);
        f[4] = bf16lo(w.z); f[5] = bf16hi(w.z); f[6] = bf16lo(w.w); f[7] = bf16hi(w.w);
    }
    __device__ static __forceinline__ v4u pack(const float* f)
    {
        v4u w;
        w.x = pack_bf16x2(f[0], f[1]); w.y = pack_bf16x2(f[2], f[3]);
        w.z = pack_bf16x2(f[4], f[5]); w.w = pack_bf16x2(f[6], f[7]);
        return w;
    }
};

template <int DT> __device__ __forceinline__ float load_elem(const char* base, int64_t i);
template <> __device__ __forceinline__ float load_elem<ET_DTYPE_F32>(const char* base, int64_t i)
{
    return reinterpret_cast<const float*>(base)[i];
}
template <> __device__ __forceinline__ float load_elem<ET_DTYPE_BF16>(const char* base, int64_t i)
{
    return u2f(uint32_t(reinterpret_cast<const uint16_t*>(base)[i]) << 16);
}
template <int DT> __device__ __forceinline__ void store_elem(char* base, int64_t i, float v);
template <> __device__ __forceinline__ void store_elem<ET_DTYPE_F32>(char* base, int64_t i, float v)
{
    reinterpret_cast<float*>(base)[i] = v;
}
template <> __device__ __forceinline__ void store_elem<ET_DTYPE_BF16>(char* base, int64_t i, float v)
{
    reinterpret_cast<uint16_t*>(base)[i] = (uint16_t)f32_to_bf16_bits(v);
}

// Wave-uniform token id and the clamped range of its slot-list entries.
struct TokenSpan {
    int t;
    int j0, j1;
};

__device__ __forceinline__ bool token_span(int T, const int32_t* __restrict__ tok_off, int64_t cap,
                                           TokenSpan& sp)
{
    sp.t = (int)blockIdx.x * kRowWaves + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    if (sp.t >= T) return false;
    const int64_t a = tok_off[sp.t];
    const int64_t b = tok_off[sp.t + 1];
    sp.j0 = (int)min(max(a, (int64_t)0), cap);
    sp.j1 = (int)max(min(b, cap), (int64_t)sp.j0);
    return true;
}

// The u-th entry of the 64-entry block of the slot list starting at jb: each
// lane loads one entry, then entries are broadcast with readlane.
__device__ __forceinline__ int load_slot_block(const int32_t* __restrict__ tok_slot, int jb, int j1)
{
    const int j = jb + lane_id();
    return j < j1 ? tok_slot[j] : -1;
}

// ---------------------------------------------------------------------------
// Row pieces.  The vector dispatch and combine kernels split every row into
// pieces of whole 16-byte chunks and give each (token, piece) pair its own
// wave: consecutive waves take consecutive pieces of one token, then move to
// the next token.  On gfx950 many short-lived waves that each move 1 KiB per
// instruction stream closer to HBM peak than one wave looping over a whole row
// (measured at d = 4096 bf16 for all three kernels: 1 KiB pieces in 128-thread
// blocks beat 2-8 KiB pieces and 256-1024-thread blocks).
// ---------------------------------------------------------------------------

struct PieceSpan {
    int t;       // token
    int64_t cb;  // first chunk of the wave's piece
    int j0, j1;  // the token's slot-list entries, clamped to the capacity
};

// Wave -> (token, piece), for WPB waves per block and launches that cover
// tokens [t_base, t_end).  False for the waves past t_end.
template <int WPB>
__device__ __forceinline__ bool piece_span(int t_base, int t_end, uint32_t npieces, int64_t piece_chunks,
                                           const int32_t* __restrict__ tok_off, int64_t cap, PieceSpan& sp)
{
    const uint32_t gw = blockIdx.x * (uint32_t)WPB +
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const uint32_t tl = gw / npieces;
    const int64_t t = (int64_t)t_base + tl;
    if (t >= t_end) return false;
    sp.t = (int)t;
    sp.cb = (int64_t)(gw - tl * npieces) * piece_chunks;
    const int64_t a = tok_off[t];
    const int64_t b = tok_off[t + 1];
    sp.j0 = (int)min(max(a, (int64_t)0), cap);      // a list entry below 0 is never read
    sp.j1 = (int)max(min(b, cap), (int64_t)sp.j0);
    return true;
}

__device__ __forceinline__ v4u ld16_nt(const char* p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
}
__device__ __forceinline__ void st16_nt(char* p, v4u v)
{
    __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(p));
}

// A non-temporal store at device scope (nt sc1): written through the XCD's L2
// instead of being held there, so it leaves that L2 to the data a kernel
// re-reads.  The compiler's non-temporal store has no scope bits, hence the
// inline assembly.  The compiler's memory waits count only the operations it
// issued itself; vector memory operations retire in issue order on gfx950, so
// every wait it places for a load still covers that load.
__device__ __forceinline__ void st16_nt_dev(char* p, v4u v)
{
    asm volatile("global_store_dwordx4 %0, %1, off nt sc1" ::"v"(p), "v"(v) : "memory");
}

// ---------------------------------------------------------------------------
// dispatch forward: Xp[s] = X[t] for each slot s of t.  One wave per 1 KiB
// piece of a token's row: each lane loads its 16-byte chunk once and stores it
// to every slot of the token.
// ---------------------------------------------------------------------------

constexpr int kScatterWaves = 2;

__global__ __launch_bounds__(kScatterWaves * kWave) void dispatch_fwd_vec(
    const char* __restrict__ x, int t_base, int t_end, int64_t nch, uint32_t npieces,
    const int32_t* __restrict__ tok_off, const int32_t* __restrict__ tok_slot, int64_t cap,
    char* __restrict__ xp)
{
    PieceSpan sp;
    if (!piece_span<kScatterWaves>(t_base, t_end, npieces, kWave, tok_off, cap, sp)) return;
    const int64_t idx = sp.cb + lane_id();
    const bool on = idx < nch;
    const int64_t rb = nch * 16;
    v4u v = {0u, 0u, 0u, 0u};
    if (on) v = ld16(x + (int64_t)sp.t * rb + idx * 16);
    for (int jb = sp.j0; jb < sp.j1; jb += kWave) {
        const int my = load_slot_block(tok_slot, jb, sp.j1);
        const int n = min(kWave, sp.j1 - jb);
        for (int u = 0; u < n; ++u) {
            const int s = __builtin_amdgcn_readlane(my, u);
            if (s < 0 || (int64_t)s >= cap) continue;
            if (on) st16(xp + (int64_t)s * rb + idx * 16, v);
        }
    }
}

template <int DT>
__global__ __launch_bounds__(kRowThreads) void dispatch_fwd_elem(
    const char* __restrict__ x, int T, int64_t d, const int32_t* __restrict__ tok_off,
    const int32_t* __restrict__ tok_slot, int64_t cap, char* __restrict__ xp)
{
    TokenSpan sp;
    if (!token_span(T, tok_off, cap, sp)) return;
    const int lane = lane_id();
    for (int j = sp.j0; j < sp.j1; ++j) {
        const int s = tok_slot[j];
        if (s < 0 || (int64_t)s >= cap) continue;
        for (int64_t c = lane; c < d; c += kWave)
            store_elem<DT>(xp, (int64_t)s * d + c, load_elem<DT>(x, (int64_t)sp.t * d + c));
    }
}

// ---------------------------------------------------------------------------
// combine forward: Y[t] = sum_s gate[s] * Yp[s] (fma chain in ascending expert
// order).  Without GATE this is the dispatch backward dX[t] = sum dXp[s].  One
// wave per 1 KiB piece of a token's row: each lane accumulates its 16-byte
// chunk over the token's slots.  The gathered rows are read once and never
// again, so loads and the final store are non-temporal.
// ---------------------------------------------------------------------------

constexpr int kGatherWaves = 2;
constexpr int kGatherBatch = 8;     // slots whose loads a gather wave issues together

// ROUTER (dispatch backward only): every slot also adds dl * W[e] with the
// slot's router-logit gradient dl and expert e, read per token-list entry
// from rl_dl / rl_e, and the router weight rows W (same dtype and row length
// as yp; L2-resident).
template <int DT, bool GATE, bool ROUTER = false>
__global__ __launch_bounds__(kGatherWaves * kWave) void combine_fwd_vec(
    const char* __restrict__ yp, const float* __restrict__ gate, int t_base, int t_end, int64_t nch,
    uint32_t npieces, const int32_t* __restrict__ tok_off, const int32_t* __restrict__ tok_slot,
    int64_t cap, char* __restrict__ y, const int32_t* __restrict__ rl_e = nullptr,
    const float* __restrict__ rl_dl = nullptr, const char* __restrict__ wr = nullptr)
{
    using P = Pack<DT>;
    constexpr int N = P::N;
    PieceSpan sp;
    if (!piece_span<kGatherWaves>(t_base, t_end, npieces, kWave, tok_off, cap, sp)) return;
    const int64_t idx = sp.cb + lane_id();
    const bool on = idx < nch;
    const int64_t rb = nch * 16;
    float acc[N];
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = 0.0f;
    if constexpr (!ROUTER) {
        // Batches of kGatherBatch slots: every load of a batch (rows and
        // gates) is issued before the first is used, then the batch is
        // accumulated in list order, skipping invalid slots as one at a time.
        for (int jb = sp.j0; jb < sp.j1; jb += kWave) {
            const int my = load_slot_block(tok_slot, jb, sp.j1);
            const int n = min(kWave, sp.j1 - jb);
            for (int u0 = 0; u0 < n; u0 += kGatherBatch) {
                v4u w[kGatherBatch];
                float g[kGatherBatch];
                bool ok[kGatherBatch];
#pragma unroll
                for (int i = 0; i < kGatherBatch; ++i) {
                    const int s = __builtin_amdgcn_readlane(my, min(u0 + i, n - 1));
                    ok[i] = u0 + i < n && s >= 0 && (int64_t)s < cap;
                    const int sc = ok[i] ? s : 0;
                    w[i] = v4u{0u, 0u, 0u, 0u};
                    if (ok[i] && on) w[i] = ld16_nt(yp + (int64_t)sc * rb + idx * 16);
                    g[i] = GATE && ok[i] ? gate[sc] : 1.0f;
                }
#pragma unroll
                for (int i = 0; i < kGatherBatch; ++i) {
                    if (ok[i] && on) {
                        float f[N];
                        P::unpack(w[i], f);
#pragma unroll
                        for (int c = 0; c < N; ++c) acc[c] = __builtin_fmaf(g[i], f[c], acc[c]);
                    }
                }
            }
        }
        if (on) st16_nt(y + (int64_t)sp.t * rb + idx * 16, P::pack(acc));
        return;
    }
    for (int jb = sp.j0; jb < sp.j1; jb += kWave) {
        const int my = load_slot_block(tok_slot, jb, sp.j1);
        const int n = min(kWave, sp.j1 - jb);
        int mye = 0;
        float myd = 0.0f;
        if constexpr (ROUTER) {
            const int j = jb + lane_id();
            mye = j < sp.j1 ? rl_e[j] : 0;
            myd = j < sp.j1 ? rl_dl[j] : 0.0f;
        }
        // Walk the valid slots; the load of the next slot's chunk is issued
        // at the end of the current slot's iteration.  (Issuing it before the
        // current slot's arithmetic, a two-deep pipeline, measured slower.)
        int u = 0;
        int s = -1;
        v4u w = {0u, 0u, 0u, 0u}, wv = {0u, 0u, 0u, 0u};
        for (; u < n; ++u) {
            s = __builtin_amdgcn_readlane(my, u);
            if (s >= 0 && (int64_t)s < cap) break;
        }
        if (u < n && on) {
            w = ld16_nt(yp + (int64_t)s * rb + idx * 16);
            if constexpr (ROUTER) wv = ld16(wr + (int64_t)__builtin_amdgcn_readlane(mye, u) * rb + idx * 16);
        }
        while (u < n) {
            const int cur = s;
            const int ucur = u;
            const v4u wc = w, wvc = wv;
            for (++u; u < n; ++u) {
                s = __builtin_amdgcn_readlane(my, u);
                if (s >= 0 && (int64_t)s < cap) break;
            }
            const float g = GATE ? gate[cur] : 1.0f;
            if (on) {
                float f[N];
                P::unpack(wc, f);
#pragma unroll
                for (int i = 0; i < N; ++i) acc[i] = __builtin_fmaf(g, f[i], acc[i]);
                if constexpr (ROUTER) {
                    const float dl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(myd), ucur));
                    P::unpack(wvc, f);
#pragma unroll
                    for (int i = 0; i < N; ++i) acc[i] = __builtin_fmaf(dl, f[i], acc[i]);
                }
            }
            if (u < n && on) {
                w = ld16_nt(yp + (int64_t)s * rb + idx * 16);
                if constexpr (ROUTER)
                    wv = ld16(wr + (int64_t)__builtin_amdgcn_readlane(mye, u) * rb + idx * 16);
            }
        }
    }
    if (on) st16_nt(y + (int64_t)sp.t * rb + idx * 16, P::pack(acc));
}

template <int DT>
__global__ __launch_bounds__(kRowThreads) void combine_fwd_elem(
    const char* __restrict__ yp, const float* __restrict__ gate, int T, int64_t d,
    const int32_t* __restrict__ tok_off, const int32_t* __restrict__ tok_slot, int64_t cap,
    char* __restrict__ y, const int32_t* __restrict__ rl_e = nullptr, const float* __restrict__ rl_dl = nullptr,
    const char* __restrict__ wr = nullptr)
{
    TokenSpan sp;
    if (!token_span(T, tok_off, cap, sp)) return;
    const int lane = lane_id();
    for (int64_t c = lane; c < d; c += kWave) {
        float acc = 0.0f;
        for (int j = sp.j0; j < sp.j1; ++j) {
            const int s = tok_slot[j];
            if (s < 0 || (int64_t)s >= cap) continue;
            const float g = gate ? gate[s] : 1.0f;
            acc = __builtin_fmaf(g, load_elem<DT>(yp, (int64_t)s * d + c), acc);
            if (wr) acc = __builtin_fmaf(rl_dl[j], load_elem<DT>(wr, (int64_t)rl_e[j] * d + c), acc);
        }
        store_elem<DT>(y, (int64_t)sp.t * d + c, acc);
    }
}

// ---------------------------------------------------------------------------
// combine backward: dYp[s] = gate[s] * dY[t]; dgate[s] = <dY[t], Yp[s]>;
// dlogits[t, e(s)] = dgate[s] * g (1 - g), zero for unselected experts.
// ---------------------------------------------------------------------------

constexpr int kMaxLanesE = ET_MAX_EXPERTS / kWave;  // expert registers per lane

// Expert of slot s: the largest e with eoff[e] <= s (binary search in LDS).
__device__ __forceinline__ int expert_of_slot(const int* eoff_lds, int E, int s)
{
    int lo = 0, hi = E;  // eoff[lo] <= s < eoff[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (eoff_lds[mid] <= s) lo = mid; else hi = mid;
    }
    return lo;
}

// Records slot s's results: dgate, and the dlogits value in the lane/register
// that owns expert e(s) of this token's dlogits row.
__device__ __forceinline__ void finish_slot(int s, float dot, float g, float* __restrict__ dgate,
                                            const int* eoff_lds, int E, bool want_dl, float* dlv)
{
    if (lane_id() == 0) dgate[s] = dot;
    if (want_dl) {
        const int e = expert_of_slot(eoff_lds, E, s);
        const float v = dot * (g * (1.0f - g));
        const int reg = e >> 6;
        const bool mine = (e & (kWave - 1)) == lane_id();
#pragma unroll
        for (int i = 0; i < kMaxLanesE; ++i)
            if (i == reg && mine) dlv[i] = v;
    }
}

__device__ __forceinline__ void write_dlogits_row(float* __restrict__ dlogits, int t, int E, const float* dlv)
{
    float* row = dlogits + (int64_t)t * E;
#pragma unroll
    for (int i = 0; i < kMaxLanesE; ++i) {
        const int e = i * kWave + lane_id();
        if (e < E) row[e] = dlv[i];
    }
}

__device__ __forceinline__ void load_eoff_lds(int* eoff_lds, const int32_t* __restrict__ eoff, int E,
                                              bool want_dl)
{
    if (want_dl)
        for (int e = threadIdx.x; e <= E; e += kRowThreads) eoff_lds[e] = eoff[e];
    __syncthreads();
}

// Vector path, pass 1.  For every routed slot s and every pair q of 1 KiB
// pieces of the row, one wave writes those pieces of dYp[s] = gate[s] *
// dY[token(s)] and their partial dot <dY[t], Yp[s]> to part[s * nparts + q].
// The partial is formed in binary64: every product of two binary32 (or bf16)
// values is exact in binary64, each lane sums its 16 (bf16) or 8 (binary32)
// products in two chains (even and odd elements, then added), and one DPP
// wave reduction sums the lanes, so the partial carries about a dozen
// binary64 roundings.  Yp is read once and dYp written once, both
// non-temporal; the dYp stores also at device scope (nt sc1), which writes
// them through the XCD's L2 and makes the pass about 1% faster at T = 65536,
// d = 4096 (the L2 then holds less of a window's dY, which is fetched again
// from beyond it more often, and still the pass is faster).
//
// Walk order.  Walking tokens (each token's ~k slots at once) has the waves in
// flight touch a slot run in every expert block, each run visited again and
// again over time, and walking slots in slot order re-reads each dY row k
// times from HBM.  Instead the tokens are cut into windows of TW consecutive
// tokens (TW dY rows, 3 MiB, re-read from the cache); inside a window each
// expert's slots are one contiguous run (slots are ordered by token within an
// expert), and the runs are walked one after another, so consecutive waves
// take consecutive slots of one run.  At d = 4096 bf16, E = 128, k = 8 this is
// 8-9% faster than the token walk (Zipf-skewed and uniform expert loads); with
// about one slot per token, or a dY that the caches hold, the plain slot order
// (s = J, no order pass) is faster still and is used instead.  The
// window-ordered index of slot s is
//     J(s) = base[w] + pre[w][e] + (s - off[w][e]),  w = token(s) / TW, e = expert(s)
// with off[w][e] = the first slot of expert e whose token is >= w * TW,
// pre[w][e] = the window's slots in experts < e and base[w] =
// token_offsets[w * TW] (the slots of the tokens before the window).  One
// small kernel builds order[J(s)] = s; the main kernel walks J with one wave
// per (J, pair of pieces).  Each XCD (block b runs on XCD b % 8) takes a
// contiguous eighth of the J range, so one XCD's L2 holds the dY rows of the
// window it walks: windows are sized at 3 MiB of dY for the 4 MB L2 of an
// XCD (4 MiB and more thrash it; measured 3-15% slower).
//
// When the routed slots exceed an undersized capacity (expert_offsets[E] >
// cap) the order pass writes nothing and the main kernel walks the token
// lists instead: J in [0, cap), s = token_slot[J], skipping s >= cap -- the
// (slot, piece) pairs a token-major walk of the capacity-clamped lists visits.
// Either way each (slot, piece) partial is formed the same way, so the
// results do not depend on the order.
constexpr int kBwdWaves = 1;
constexpr int kWinPieces = 2;                    // 1 KiB row pieces per wave
constexpr int64_t kWinBytes = int64_t(3) << 20;  // dY bytes of one token window (target)
constexpr int kXcds = 8;

static int64_t win_tokens(int64_t rb)
{
    return std::min<int64_t>(8192, std::max<int64_t>(64, kWinBytes / std::max<int64_t>(rb, 1)));
}

// Slot order (no windows) where windows do not pay for their order pass:
// about one slot per token (capacity <= 1.25 T, so dY rows are not re-read),
// or a dY small enough to stay in the caches.
constexpr int64_t kSlotOrderBytes = int64_t(16) << 20;

static bool bwd_slot_order(int64_t T, int64_t cap, int64_t rb)
{
    return cap * 4 <= T * 5 || T * rb <= kSlotOrderBytes;
}

// order[J(s)] = s for the slots of one token window per block.  The
// window's token-list entries are [j0, j1) = [token_offsets[w TW],
// token_offsets[(w + 1) TW]), which is also its range of J.  The block counts
// the window's slots per expert and finds each expert's first slot (LDS
// atomics: add and min, so the result does not depend on their order), scans
// the counts, then places every slot.  Each thread loads kOrderBatch entries
// before using any, so a window of up to kOrderThreads * kOrderBatch entries
// pays one memory latency per pass.  Blocks past the nwin windows zero-fill
// dlogits instead.
constexpr int kOrderThreads = 1024;
constexpr int kOrderBatch = 8;
constexpr int kOrderZeroBlocks = 256;                // blocks of the order launch that zero-fill dlogits

// Slots of token-list entries jb + k * kOrderThreads + threadIdx.x (k <
// kOrderBatch) below j1, with their experts; -1 where out of range.
__device__ __forceinline__ void order_batch(const int32_t* __restrict__ tok_slot, int64_t jb, int64_t j1, int64_t S,
                                            const int32_t* eo, int E, int (&sv)[kOrderBatch], int (&ev)[kOrderBatch])
{
#pragma unroll
    for (int k = 0; k < kOrderBatch; ++k) {
        const int64_t j = jb + (int64_t)k * kOrderThreads + threadIdx.x;
        sv[k] = j < j1 ? tok_slot[j] : -1;
    }
#pragma unroll
    for (int k = 0; k < kOrderBatch; ++k) {
        if (sv[k] < 0 || (int64_t)sv[k] >= S) sv[k] = -1;
        ev[k] = sv[k] >= 0 ? expert_of_slot(eo, E, sv[k]) : 0;
    }
}

__global__ __launch_bounds__(kOrderThreads) void combine_bwd_order(
    const int32_t* __restrict__ tok_off, const int32_t* __restrict__ tok_slot, const int32_t* __restrict__ eoff,
    int E, int T, int TW, int64_t cap, int32_t* __restrict__ order, float* __restrict__ dlogits, int nwin)
{
    if ((int)blockIdx.x >= nwin) {
        // The blocks past the windows zero-fill dlogits (16 bytes per thread a
        // step), which pass 2 then writes at the routed entries: this launch
        // occupies few CUs with its windows, so the fill costs no time here,
        // where at the start of pass 1 it would take bandwidth from the rows.
        const int64_t n4 = (int64_t)T * E / 4;
        float4* d4 = reinterpret_cast<float4*>(dlogits);
        const int64_t stride = (int64_t)(gridDim.x - nwin) * kOrderThreads;
        for (int64_t i = (int64_t)(blockIdx.x - nwin) * kOrderThreads + threadIdx.x; i < n4; i += stride)
            d4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (blockIdx.x == (unsigned)nwin && threadIdx.x == 0)
            for (int64_t j = n4 * 4; j < (int64_t)T * E; ++j) dlogits[j] = 0.0f;
        return;
    }
    extern __shared__ int32_t sh[];                 // eo [E + 1], cnt [E], first [E]
    int32_t* eo = sh;
    int32_t* cnt = sh + E + 1;
    int32_t* first = cnt + E;
    const int64_t t0 = (int64_t)blockIdx.x * TW;
    const int64_t t1 = min(t0 + TW, (int64_t)T);
    for (int e = threadIdx.x; e <= E; e += kOrderThreads) {
        eo[e] = eoff[e];
        if (e < E) {
            cnt[e] = 0;
            first[e] = INT32_MAX;
        }
    }
    __syncthreads();
    const int64_t S = eo[E];
    if (S > cap) return;                            // undersized: pass 1 walks the token lists
    const int64_t j0 = min(max((int64_t)tok_off[t0], (int64_t)0), S);
    const int64_t j1 = max(min((int64_t)tok_off[t1], S), j0);
    constexpr int64_t kStep = (int64_t)kOrderThreads * kOrderBatch;
    for (int64_t jb = j0; jb < j1; jb += kStep) {
        int sv[kOrderBatch], ev[kOrderBatch];
        order_batch(tok_slot, jb, j1, S, eo, E, sv, ev);
#pragma unroll
        for (int k = 0; k < kOrderBatch; ++k)
            if (sv[k] >= 0) {
                atomicAdd(&cnt[ev[k]], 1);
                atomicMin(&first[ev[k]], sv[k]);
            }
    }
    __syncthreads();
    if (threadIdx.x < kWave) {                      // exclusive scan of cnt, in place
        int run = 0;
        for (int e0 = 0; e0 < E; e0 += kWave) {
            const int e = e0 + (int)threadIdx.x;
            const int c = e < E ? cnt[e] : 0;
            const int incl = wave_incl_scan(c);
            if (e < E) cnt[e] = run + incl - c;
            run += __builtin_amdgcn_readlane(incl, kWave - 1);
        }
    }
    __syncthreads();
    for (int64_t jb = j0; jb < j1; jb += kStep) {
        int sv[kOrderBatch], ev[kOrderBatch];
        order_batch(tok_slot, jb, j1, S, eo, E, sv, ev);
#pragma unroll
        for (int k = 0; k < kOrderBatch; ++k)
            if (sv[k] >= 0) {
                const int64_t J = j0 + cnt[ev[k]] + ((int64_t)sv[k] - first[ev[k]]);
                if (J >= j0 && J < j1) order[J] = sv[k];
            }
    }
}

// acc + a * b with the product exact: two binary32 (or bf16) values multiply
// exactly in binary64 (24 + 24 significant bits, and no binary32 product
// under- or overflows there), so the fma rounds once, at the addition.
__device__ __forceinline__ double fma_exact(float a, float b, double acc)
{
    return __builtin_fma((double)a, (double)b, acc);
}

// The main pass: one wave per (J, pair of pieces); both pieces' loads are
// issued before either is used.  With zero_dl (no order launch did it) the
// first waves in dispatch order also zero-fill dlogits (1 KiB each), which
// pass 2 then writes at the routed entries.
template <int DT>
__global__ __launch_bounds__(kBwdWaves * kWave) void combine_bwd_vec(
    const char* __restrict__ dy, const char* __restrict__ yp, const float* __restrict__ gate,
    const int32_t* __restrict__ sorted_token, const int32_t* __restrict__ order,
    const int32_t* __restrict__ tok_slot, const int32_t* __restrict__ eoff, int E, int T, int64_t nch,
    uint32_t npieces, int64_t cap, char* __restrict__ dyp, double* __restrict__ part, float* __restrict__ dlogits,
    bool zero_dl)
{
    using P = Pack<DT>;
    constexpr int N = P::N;
    const int64_t S = eoff[E];
    const bool fits = S <= cap;
    const int32_t* __restrict__ walk = fits ? order : tok_slot;     // null: slot order (s = J)
    const int64_t nj = fits ? S : cap;
    const int lane = lane_id();
    const int64_t rb = nch * 16;
    const uint32_t nq = (npieces + kWinPieces - 1) / kWinPieces;
    const int64_t items = nj * nq;
    // XCD-contiguous order: the items' blocks are split into kXcds
    // contiguous ranges of `per` blocks; the blocks b with b % kXcds == x walk
    // range x (the grid is a multiple of kXcds blocks)
    const int64_t per = ((items + kBwdWaves - 1) / kBwdWaves + kXcds - 1) / kXcds;
    const int64_t rows = gridDim.x / kXcds;
    const int64_t x0 = (int64_t)(blockIdx.x % kXcds) * per;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    if (dlogits && zero_dl) {
        const int64_t n = (int64_t)T * E;
        const int64_t stride = (int64_t)gridDim.x * kBwdWaves * 4 * kWave;
        for (int64_t f = ((int64_t)blockIdx.x * kBwdWaves + wv) * 4 * kWave; f < n; f += stride)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (f + k * kWave + lane < n) dlogits[f + k * kWave + lane] = 0.0f;
    }
    for (int64_t row = blockIdx.x / kXcds; row < per; row += rows) {
        const int64_t it = (x0 + row) * kBwdWaves + wv;
        if (it >= items) break;
        const int64_t J = it / nq;
        const uint32_t q = (uint32_t)(it - J * nq);
        const int s = walk ? walk[J] : (int)J;
        if (s < 0 || (int64_t)s >= cap || (int64_t)s >= S) continue;
        const int t = sorted_token[s];
        if (t < 0 || t >= T) continue;
        const float g = gate[s];
        int64_t idx[kWinPieces];
        bool on[kWinPieces];
        v4u wy[kWinPieces], wd[kWinPieces];
#pragma unroll
        for (int i = 0; i < kWinPieces; ++i) {
            idx[i] = (int64_t)(q * kWinPieces + i) * kWave + lane;
            on[i] = idx[i] < nch;
            wy[i] = v4u{0u, 0u, 0u, 0u};
            wd[i] = v4u{0u, 0u, 0u, 0u};
            if (on[i]) {
                wy[i] = ld16_nt(yp + (int64_t)s * rb + idx[i] * 16);
                wd[i] = ld16(dy + (int64_t)t * rb + idx[i] * 16);
            }
        }
        // the wave's partial dot: even and odd elements of both pieces in two
        // binary64 chains (an element past the row reads 0 from both rows)
        double a0 = 0.0, a1 = 0.0;
#pragma unroll
        for (int i = 0; i < kWinPieces; ++i) {
            float f[N], df[N], o[N];
            P::unpack(wy[i], f);
            P::unpack(wd[i], df);
#pragma unroll
            for (int k = 0; k < N; ++k) o[k] = g * df[k];
            if (on[i]) st16_nt_dev(dyp + (int64_t)s * rb + idx[i] * 16, P::pack(o));
#pragma unroll
            for (int k = 0; k < N; k += 2) {
                a0 = fma_exact(df[k], f[k], a0);
                a1 = fma_exact(df[k + 1], f[k + 1], a1);
            }
        }
        const double dot = wave_sum_dpp_f64(a0 + a1);
        if (lane == 0) part[(int64_t)s * nq + q] = dot;
    }
}

// Vector path, pass 2: one thread per slot s < min(expert_offsets[E], cap):
// dgate[s] = the binary64 sum of the slot's partial dots in order,
// rounded once to binary32, and dlogits[sorted_token[s], e(s)] = dgate[s] *
// (g * (1 - g)) in binary32, with e(s) found by a binary search of
// expert_offsets in LDS.  A slot that pass 1 skipped (its
// token-list entry at or past an undersized capacity) gets dgate 0 and leaves
// its dlogits entry at the zero pass 1 wrote.
constexpr int kFinishThreads = 256;

__global__ __launch_bounds__(kFinishThreads) void combine_bwd_finish(
    const double* __restrict__ part, uint32_t nparts, const float* __restrict__ gate,
    const int32_t* __restrict__ sorted_token, const int32_t* __restrict__ tok_off,
    const int32_t* __restrict__ tok_slot, const int32_t* __restrict__ eoff, int E, int64_t cap,
    float* __restrict__ dgate, float* __restrict__ dlogits)
{
    extern __shared__ int32_t eo[];                                     // [E + 1]
    const bool want_dl = dlogits != nullptr;
    const int64_t s = (int64_t)blockIdx.x * kFinishThreads + threadIdx.x;
    // The slot's loads depend on s only: issue them (clamped below the
    // capacity, every array holds cap slots) before the expert offsets land.
    const int64_t sc = min(s, cap - 1);
    const double* ps = part + sc * nparts;
    double v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = ps[min((uint32_t)i, nparts - 1)];
    const float g = gate[sc];
    const int t = sorted_token[sc];
    const int64_t routed = eoff[E];
    if (want_dl)
        for (int e = threadIdx.x; e <= E; e += kFinishThreads) eo[e] = eoff[e];
    __syncthreads();
    const int64_t S = min(routed, cap);
    if (s >= S) return;
    if (routed > cap) {
        // Undersized capacity: pass 1 skipped slot s unless its token-list
        // entry is also below the capacity.  Only the token whose list
        // straddles the capacity needs a search.
        const int64_t a = max(tok_off[t], 0), b = tok_off[t + 1];
        bool kept = b <= cap;
        for (int64_t j = a; !kept && j < cap && j < b; ++j) kept = tok_slot[j] == (int32_t)s;
        if (!kept) {
            dgate[s] = 0.0f;
            return;
        }
    }
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if ((uint32_t)i < nparts) acc += v[i];
    for (uint32_t q0 = 8; q0 < nparts; q0 += 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ps[min(q0 + i, nparts - 1)];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (q0 + i < nparts) acc += v[i];
    }
    const float dot = (float)acc;
    dgate[s] = dot;
    if (want_dl) {
        const int e = expert_of_slot(eo, E, (int)s);
        dlogits[(int64_t)t * E + e] = dot * (g * (1.0f - g));
    }
}

template <int DT>
__global__ __launch_bounds__(kRowThreads) void combine_bwd_elem(
    const char* __restrict__ dy, const char* __restrict__ yp, const float* __restrict__ gate,
    const int32_t* __restrict__ tok_off, const int32_t* __restrict__ tok_slot,
    const int32_t* __restrict__ eoff, int T, int E, int64_t d, int64_t cap,
    char* __restrict__ dyp, float* __restrict__ dgate, float* __restrict__ dlogits)
{
    __shared__ int eoff_lds[ET_MAX_EXPERTS + 1];
    const bool want_dl = dlogits != nullptr;
    load_eoff_lds(eoff_lds, eoff, E, want_dl);
    TokenSpan sp;
    if (!token_span(T, tok_off, cap, sp)) return;
    const int lane = lane_id();
    float dlv[kMaxLanesE];
#pragma unroll
    for (int i = 0; i < kMaxLanesE; ++i) dlv[i] = 0.0f;
    for (int j = sp.j0; j < sp.j1; ++j) {
        const int s = tok_slot[j];
        if (s < 0 || (int64_t)s >= cap) continue;
        const float g = gate[s];
        double part = 0.0;
        for (int64_t c = lane; c < d; c += kWave) {
            const float dv = load_elem<DT>(dy, (int64_t)sp.t * d + c);
            part = __builtin_fma((double)dv, (double)load_elem<DT>(yp, (int64_t)s * d + c), part);
            store_elem<DT>(dyp, (int64_t)s * d + c, g * dv);
        }
        finish_slot(s, (float)wave_sum_dpp_f64(part), g, dgate, eoff_lds, E, want_dl, dlv);
    }
    if (want_dl) write_dlogits_row(dlogits, sp.t, E, dlv);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// Router-gradient terms of dispatch backward, per token-list entry j (token
// order): the slot s = tok_slot[j], its expert e(s), and dl = dgate[s] *
// (g * (1 - g)) with g = gate[s] -- the same binary32 expression as the
// dlogits entry of combine backward.  Entries past min(S, cap), or whose slot
// is dropped by an undersized capacity, get e = 0 and dl = 0.
__global__ __launch_bounds__(kFinishThreads) void router_terms_kernel(
    const int32_t* __restrict__ tok_slot, const int32_t* __restrict__ eoff, int E, const float* __restrict__ gate,
    const float* __restrict__ dgate, int64_t cap, int32_t* __restrict__ rl_e, float* __restrict__ rl_dl)
{
    extern __shared__ int32_t eo[];                                     // [E + 1]
    for (int e = threadIdx.x; e <= E; e += kFinishThreads) eo[e] = eoff[e];
    __syncthreads();
    const int64_t j = (int64_t)blockIdx.x * kFinishThreads + threadIdx.x;
    const int64_t S = min((int64_t)eo[E], cap);
    if (j >= cap) return;
    int e = 0;
    float dl = 0.0f;
    if (j < S) {
        const int s = tok_slot[j];
        if (s >= 0 && (int64_t)s < cap) {
            e = expert_of_slot(eo, E, s);
            const float g = gate[s];
            dl = dgate[s] * (g * (1.0f - g));
        }
    }
    rl_e[j] = e;
    rl_dl[j] = dl;
}

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int elem_bytes(int dtype) { return dtype == ET_DTYPE_BF16 ? 2 : 4; }

static int check_common(const char* fn, int64_t T, int64_t d, int dtype, int64_t cap,
                        const int32_t* tok_off, const int32_t* tok_slot)
{
    if (T < 0 || T >= (int64_t(1) << 31)) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": num_tokens out of range");
    if (d < 0) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": d < 0");
    if (dtype != ET_DTYPE_F32 && dtype != ET_DTYPE_BF16)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": dtype must be ET_DTYPE_F32 or ET_DTYPE_BF16");
    if (cap < 0) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": slot_capacity < 0");
    if (T > 0 && (!tok_off || (cap > 0 && !tok_slot)))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null token_offsets/token_slot");
    return ET_OK;
}

#define ET_SWITCH_DT(dt, ...)                                          \
    if ((dt) == ET_DTYPE_BF16) { constexpr int DT = ET_DTYPE_BF16; __VA_ARGS__; } \
    else { constexpr int DT = ET_DTYPE_F32; __VA_ARGS__; }

// Launches a piece kernel over tokens [0, T) with npieces waves per token and
// wpb waves per block, in as many launches as keep every launch's wave index
// below 2^31 (one launch for any realistic shape).
template <typename F>
static void for_each_piece_launch(int64_t T, int64_t npieces, int wpb, F&& launch)
{
    const int64_t max_tokens = std::max<int64_t>(1, ((int64_t(1) << 31) - wpb) / npieces);
    for (int64_t t0 = 0; t0 < T; t0 += max_tokens) {
        const int64_t t1 = std::min<int64_t>(T, t0 + max_tokens);
        const int64_t waves = (t1 - t0) * npieces;
        launch(dim3((unsigned)((waves + wpb - 1) / wpb)), (int)t0, (int)t1);
    }
}

static dim3 row_grid(int64_t T) { return dim3((unsigned)((T + kRowWaves - 1) / kRowWaves)); }

}  // namespace et

using namespace et;

extern "C" int et_dispatch_fwd(const void* x, int64_t T, int64_t d, int dtype,
                               const int32_t* token_offsets, const int32_t* token_slot,
                               int64_t cap, void* xp, void* stream)
{
    if (int rc = check_common("et_dispatch_fwd", T, d, dtype, cap, token_offsets, token_slot)) return rc;
    if (T == 0 || d == 0 || cap == 0) return ET_OK;
    if (!x || !xp) return fail(ET_ERR_INVALID_ARGUMENT, "et_dispatch_fwd: null x/xp");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t rb = d * elem_bytes(dtype);
    const char* xc = static_cast<const char*>(x);
    char* xpc = static_cast<char*>(xp);
    if (rb % 16 == 0 && aligned16(x) && aligned16(xp)) {
        const int64_t nch = rb / 16;
        const int64_t np = (nch + kWave - 1) / kWave;
        for_each_piece_launch(T, np, kScatterWaves, [&](dim3 grid, int t0, int t1) {
            dispatch_fwd_vec<<<grid, dim3(kScatterWaves * kWave), 0, s>>>(xc, t0, t1, nch, (uint32_t)np, token_offsets,
                                                                         token_slot, cap, xpc);
        });
    } else {
        ET_SWITCH_DT(dtype, dispatch_fwd_elem<DT><<<row_grid(T), dim3(kRowThreads), 0, s>>>(xc, (int)T, d, token_offsets, token_slot, cap, xpc));
    }
    return check_launch("dispatch_fwd");
}

static int combine_like(const char* fn, const void* yp, const float* gate, const int32_t* token_offsets,
                        const int32_t* token_slot, int64_t T, int64_t d, int dtype, int64_t cap, void* y,
                        void* stream)
{
    if (int rc = check_common(fn, T, d, dtype, cap, token_offsets, token_slot)) return rc;
    if (T == 0 || d == 0) return ET_OK;
    if (!y || (cap > 0 && !yp)) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null input/output");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t rb = d * elem_bytes(dtype);
    const char* ypc = static_cast<const char*>(yp);
    char* yc = static_cast<char*>(y);
    if (rb % 16 == 0 && aligned16(yp) && aligned16(y)) {
        const int64_t nch = rb / 16;
        const int64_t np = (nch + kWave - 1) / kWave;
        for_each_piece_launch(T, np, kGatherWaves, [&](dim3 grid, int t0, int t1) {
            ET_SWITCH_DT(dtype,
                if (gate)
                    combine_fwd_vec<DT, true><<<grid, dim3(kGatherWaves * kWave), 0, s>>>(
                        ypc, gate, t0, t1, nch, (uint32_t)np, token_offsets, token_slot, cap, yc);
                else
                    combine_fwd_vec<DT, false><<<grid, dim3(kGatherWaves * kWave), 0, s>>>(
                        ypc, nullptr, t0, t1, nch, (uint32_t)np, token_offsets, token_slot, cap, yc));
        });
    } else {
        ET_SWITCH_DT(dtype, combine_fwd_elem<DT><<<row_grid(T), dim3(kRowThreads), 0, s>>>(ypc, gate, (int)T, d, token_offsets, token_slot, cap, yc));
    }
    return check_launch(fn);
}

extern "C" int et_combine_fwd(const void* yp, const float* slot_gate, const int32_t* token_offsets,
                              const int32_t* token_slot, int64_t T, int64_t d, int dtype, int64_t cap,
                              void* y, void* stream)
{
    if (cap > 0 && T > 0 && !slot_gate) return fail(ET_ERR_INVALID_ARGUMENT, "et_combine_fwd: null slot_gate");
    return combine_like("et_combine_fwd", yp, slot_gate, token_offsets, token_slot, T, d, dtype, cap, y, stream);
}

extern "C" int et_dispatch_bwd(const void* dxp, const int32_t* token_offsets, const int32_t* token_slot,
                               int64_t T, int64_t d, int dtype, int64_t cap, void* dx, void* stream)
{
    return combine_like("et_dispatch_bwd", dxp, nullptr, token_offsets, token_slot, T, d, dtype, cap, dx, stream);
}

static size_t router_terms_bytes(int64_t cap) { return cap > 0 ? 2 * ((size_t(cap) * 4 + 255) & ~size_t(255)) : 0; }

extern "C" size_t et_dispatch_bwd_router_workspace_bytes(int64_t slot_capacity)
{
    return slot_capacity < 0 ? 0 : router_terms_bytes(slot_capacity);
}

extern "C" int et_dispatch_bwd_router(const void* dxp, const int32_t* token_offsets, const int32_t* token_slot,
                                      int64_t T, int64_t d, int dtype, int64_t cap, const float* slot_gate,
                                      const float* dgate, const int32_t* expert_offsets, int64_t E,
                                      const void* w_router, void* dx, void* workspace, size_t workspace_bytes,
                                      void* stream)
{
    const char* fn = "et_dispatch_bwd_router";
    if (int rc = check_common(fn, T, d, dtype, cap, token_offsets, token_slot)) return rc;
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (!expert_offsets) return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null expert_offsets");
    if (T == 0 || d == 0) return ET_OK;
    if (!dx || (cap > 0 && (!dxp || !slot_gate || !dgate || !w_router || !workspace)))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null input/output/workspace");
    const size_t need = router_terms_bytes(cap);
    if (workspace_bytes < need)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, std::string(fn) + ": workspace needs " + std::to_string(need) +
                                                    " bytes, got " + std::to_string(workspace_bytes));
    hipStream_t s = static_cast<hipStream_t>(stream);
    int32_t* rl_e = static_cast<int32_t*>(workspace);
    float* rl_dl = reinterpret_cast<float*>(static_cast<char*>(workspace) + need / 2);
    if (cap > 0) {
        const unsigned nb = (unsigned)((cap + kFinishThreads - 1) / kFinishThreads);
        router_terms_kernel<<<dim3(nb), dim3(kFinishThreads), size_t(E + 1) * 4, s>>>(
            token_slot, expert_offsets, (int)E, slot_gate, dgate, cap, rl_e, rl_dl);
        if (int rc = check_launch("router_terms_kernel")) return rc;
    }
    const int64_t rb = d * elem_bytes(dtype);
    const char* dxpc = static_cast<const char*>(dxp);
    const char* wrc = static_cast<const char*>(w_router);
    char* dxc = static_cast<char*>(dx);
    if (rb % 16 == 0 && aligned16(dxp) && aligned16(dx) && aligned16(w_router)) {
        const int64_t nch = rb / 16;
        const int64_t np = (nch + kWave - 1) / kWave;
        for_each_piece_launch(T, np, kGatherWaves, [&](dim3 grid, int t0, int t1) {
            ET_SWITCH_DT(dtype, combine_fwd_vec<DT, false, true><<<grid, dim3(kGatherWaves * kWave), 0, s>>>(
                                    dxpc, nullptr, t0, t1, nch, (uint32_t)np, token_offsets, token_slot, cap, dxc,
                                    rl_e, rl_dl, wrc));
        });
    } else {
        ET_SWITCH_DT(dtype, combine_fwd_elem<DT><<<row_grid(T), dim3(kRowThreads), 0, s>>>(
                                dxpc, nullptr, (int)T, d, token_offsets, token_slot, cap, dxc, rl_e, rl_dl, wrc));
    }
    return check_launch(fn);
}

static bool bwd_vector_path(int64_t d, int dtype) { return d > 0 && (d * elem_bytes(dtype)) % 16 == 0; }

// Workspace of the vector path: the binary64 partial dots [cap * bwd_parts(np)],
// then the slot order [cap] int32 at the next 256-byte boundary.
static size_t bwd_order_offset(int64_t cap, int64_t nparts)
{
    return ((size_t)(cap * nparts) * sizeof(double) + 255) & ~(size_t)255;
}

// Binary64 partial dots per slot: one per wave, i.e. per kWinPieces pieces.
static int64_t bwd_parts(int64_t np) { return (np + kWinPieces - 1) / kWinPieces; }

extern "C" size_t et_combine_bwd_workspace_bytes(int64_t num_tokens, int64_t slot_capacity, int64_t d, int dtype)
{
    (void)num_tokens;
    if (slot_capacity < 0 || d < 0 || (dtype != ET_DTYPE_F32 && dtype != ET_DTYPE_BF16)) return 0;
    if (!bwd_vector_path(d, dtype)) return 0;
    const int64_t np = (d * elem_bytes(dtype) / 16 + kWave - 1) / kWave;
    return bwd_order_offset(slot_capacity, bwd_parts(np)) + (size_t)slot_capacity * 4;
}

extern "C" int et_combine_bwd(const void* dy, const void* yp, const float* slot_gate,
                              const int32_t* sorted_token, const int32_t* token_offsets,
                              const int32_t* token_slot, const int32_t* expert_offsets, int64_t T, int64_t E,
                              int64_t d, int dtype, int64_t cap, void* dyp, float* dgate, float* dlogits,
                              void* workspace, size_t workspace_bytes, void* stream)
{
    if (int rc = check_common("et_combine_bwd", T, d, dtype, cap, token_offsets, token_slot)) return rc;
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_combine_bwd: num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (!expert_offsets) return fail(ET_ERR_INVALID_ARGUMENT, "et_combine_bwd: null expert_offsets");
    if (cap > 0 && !sorted_token) return fail(ET_ERR_INVALID_ARGUMENT, "et_combine_bwd: null sorted_token");
    if (T == 0) return ET_OK;
    if (cap > 0 && (!slot_gate || !dgate || (d > 0 && (!dy || !yp || !dyp))))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_combine_bwd: null input/output");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t rb = d * elem_bytes(dtype);
    const char* dyc = static_cast<const char*>(dy);
    const char* ypc = static_cast<const char*>(yp);
    char* dypc = static_cast<char*>(dyp);
    if (bwd_vector_path(d, dtype) && aligned16(dy) && aligned16(yp) && aligned16(dyp)) {
        const size_t need = et_combine_bwd_workspace_bytes(T, cap, d, dtype);
        if (need > 0 && (!workspace || workspace_bytes < need))
            return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_combine_bwd: workspace needs " + std::to_string(need) +
                                                        " bytes, got " + std::to_string(workspace_bytes));
        if ((reinterpret_cast<uintptr_t>(workspace) & 7) != 0)
            return fail(ET_ERR_INVALID_ARGUMENT, "et_combine_bwd: workspace must be 8-byte aligned");
        const int64_t nch = rb / 16;
        const int64_t np = (nch + kWave - 1) / kWave;
        const int64_t TW = win_tokens(rb);
        const int64_t nw = (T + TW - 1) / TW;
        char* wsb = static_cast<char*>(workspace);
        double* part = reinterpret_cast<double*>(wsb);
        int32_t* order = nullptr;
        bool zero_here = true;                      // combine_bwd_vec zero-fills dlogits
        if (cap > 0 && !bwd_slot_order(T, cap, rb)) {
            order = reinterpret_cast<int32_t*>(wsb + bwd_order_offset(cap, bwd_parts(np)));
            // (blocks that zero-fill dlogits, where it is 16-byte aligned)
            const int nz = (dlogits && (reinterpret_cast<uintptr_t>(dlogits) & 15) == 0) ? kOrderZeroBlocks : 0;
            combine_bwd_order<<<dim3((unsigned)(nw + nz)), dim3(kOrderThreads), (size_t)(3 * E + 1) * 4, s>>>(
                token_offsets, token_slot, expert_offsets, (int)E, (int)T, (int)TW, cap, order, dlogits, (int)nw);
            zero_here = nz == 0;
            if (int rc = check_launch("combine_bwd_order")) return rc;
        }
        const size_t lds = (size_t)(E + 1) * 4;
        {
            // one wave per (slot, pair of pieces) for every slot the capacity
            // holds (the waves past the routed count exit at once), in a grid
            // of whole XCD rounds; with capacity 0 it only zero-fills dlogits
            const int64_t nq = (np + kWinPieces - 1) / kWinPieces;
            const int64_t blocks =
                std::max<int64_t>(1, std::min<int64_t>((cap * nq + kBwdWaves - 1) / kBwdWaves, int64_t(1) << 29));
            const int64_t grid = (blocks + kXcds - 1) / kXcds * kXcds;
            ET_SWITCH_DT(dtype, combine_bwd_vec<DT><<<dim3((unsigned)grid), dim3(kBwdWaves * kWave), 0, s>>>(
                                    dyc, ypc, slot_gate, sorted_token, order, token_slot, expert_offsets, (int)E,
                                    (int)T, nch, (uint32_t)np, cap, dypc, part, dlogits, zero_here));
            if (int rc = check_launch("combine_bwd_vec")) return rc;
        }
        if (cap == 0) return ET_OK;
        combine_bwd_finish<<<dim3((unsigned)((cap + kFinishThreads - 1) / kFinishThreads)), dim3(kFinishThreads),
                             lds, s>>>(part, (uint32_t)bwd_parts(np), slot_gate, sorted_token, token_offsets, token_slot,
                                       expert_offsets, (int)E, cap, dgate, dlogits);
        return check_launch("combine_bwd_finish");
    }
    ET_SWITCH_DT(dtype, combine_bwd_elem<DT><<<row_grid(T), dim3(kRowThreads), 0, s>>>(dyc, ypc, slot_gate, token_offsets, token_slot, expert_offsets, (int)T, (int)E, d, cap, dypc, dgate, dlogits));
    return check_launch("et_combine_bwd");
}
