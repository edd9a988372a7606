// et_route.hip -- threshold routing, histogram + exclusive-scan CSR, stable
// permutation indices, and the EMA threshold update (radix select), for gfx950.
//
// Routing runs in three launches, none of which uses atomics, so the output is
// a deterministic function of (logits, thr):
//   1. count: one thread per token (256-token chunks, one chunk per block).
//      Each thread computes its token's selection bits (sigmoid + threshold +
//      argmax fallback); per-expert counts of each wave come from one ballot per
//      expert, summed over the block's 4 waves into chunk_counts[chunk, e].
//   2. scan: column-wise exclusive scan of chunk_counts over chunks (one block
//      per 64 experts, lane = expert, coalesced rows) plus a scan of the
//      per-chunk slot totals.  Gives counts[e], chunk_base[chunk, e] and
//      chunk_slot_base[chunk].
//   3. fill: recomputes the selection bits, scans counts over experts in LDS
//      (expert_offsets), and places every selected (t, e) at
//        expert_offsets[e] + chunk_base[chunk, e] + (selected tokens of e in
//        earlier waves of the chunk) + popcount(ballot_e & lanes_below)
//      which is exactly its rank among expert e's tokens in token order.
#include "et_common.hpp"

namespace et {

constexpr int kRouteThreads = 256;
constexpr int kRouteWaves = kRouteThreads / kWave;

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

struct RouteWs {
    int32_t* chunk_counts;     // [NC * E]
    int32_t* chunk_base;       // [NC * E]
    int32_t* chunk_slots;      // [NC]
    int32_t* chunk_slot_base;  // [NC]
    size_t bytes;
};

static RouteWs route_ws_layout(void* base, int64_t T, int64_t E)
{
    const int64_t NC = (T + kRouteThreads - 1) / kRouteThreads > 0 ? (T + kRouteThreads - 1) / kRouteThreads : 1;
    RouteWs ws{};
    size_t off = 0;
    char* b = static_cast<char*>(base);
    ws.chunk_counts = reinterpret_cast<int32_t*>(b + off); off += align256(size_t(NC * E) * 4);
    ws.chunk_base = reinterpret_cast<int32_t*>(b + off); off += align256(size_t(NC * E) * 4);
    ws.chunk_slots = reinterpret_cast<int32_t*>(b + off); off += align256(size_t(NC) * 4);
    ws.chunk_slot_base = reinterpret_cast<int32_t*>(b + off); off += align256(size_t(NC) * 4);
    ws.bytes = off;
    return ws;
}

// Selection bits of one token into LDS (bits[g * kRouteThreads + tid], 32
// experts per word, expert e at bit e % 32 of word e / 32).  Returns k_t.
// VEC: E % 4 == 0, so every full 32-expert group is read with 16-byte loads.
template <bool VEC>
__device__ __forceinline__ int select_token(const float* __restrict__ row,
                                            const float* __restrict__ thr, int E, bool valid,
                                            uint32_t* bits, int tid)
{
    const int ng = (E + 31) >> 5;
    int k = 0;
    float bv = -1.0f;  // every valid score is >= 0; NaN counts as -1
    int be = 0;
    for (int g = 0; g < ng; ++g) {
        uint32_t w = 0;
        const int e0 = g * 32;
        const int n = min(32, E - e0);
        if (valid) {
            if (VEC && n == 32) {
                const float4* p4 = reinterpret_cast<const float4*>(row + e0);
                float v[32];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    float4 f = p4[q];
                    v[4 * q + 0] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
                }
#pragma unroll
                for (int b = 0; b < 32; ++b) {
                    const float s = sigmoid(v[b]);
                    if (s >= thr[e0 + b]) w |= 1u << b;
                    const float sv = (s != s) ? -1.0f : s;
                    if (sv > bv) { bv = sv; be = e0 + b; }
                }
            } else {
                for (int b = 0; b < n; ++b) {
                    const float s = sigmoid(row[e0 + b]);
                    if (s >= thr[e0 + b]) w |= 1u << b;
                    const float sv = (s != s) ? -1.0f : s;
                    if (sv > bv) { bv = sv; be = e0 + b; }
                }
            }
        }
        bits[g * kRouteThreads + tid] = w;
        k += __popc(w);
    }
    if (valid && k == 0) {
        bits[(be >> 5) * kRouteThreads + tid] |= 1u << (be & 31);
        k = 1;
    }
    return k;
}

// Per-wave, per-expert token counts of the chunk: wcnt[wave * E + e].
__device__ __forceinline__ void wave_expert_counts(const uint32_t* bits, int E, int tid,
                                                   int wave, int* wcnt)
{
    const int ng = (E + 31) >> 5;
    for (int g = 0; g < ng; ++g) {
        const uint32_t wb = bits[g * kRouteThreads + tid];
        const int n = min(32, E - g * 32);
        for (int b = 0; b < n; ++b) {
            const uint64_t bal = __ballot((wb >> b) & 1u);
            if (lane_id() == 0) wcnt[wave * E + g * 32 + b] = (int)__popcll(bal);
        }
    }
}

template <bool VEC>
__global__ __launch_bounds__(kRouteThreads) void route_count_kernel(
    const float* __restrict__ logits, const float* __restrict__ thr, int T, int E,
    int32_t* __restrict__ chunk_counts, int32_t* __restrict__ chunk_slots)
{
    extern __shared__ uint32_t smem[];
    const int ng = (E + 31) >> 5;
    uint32_t* bits = smem;                                        // [ng][256]
    int* wcnt = reinterpret_cast<int*>(smem + ng * kRouteThreads); // [4][E]
    __shared__ int wk[kRouteWaves];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t t = (int64_t)blockIdx.x * kRouteThreads + tid;
    const bool valid = t < T;
    const int k = select_token<VEC>(logits + (valid ? t : 0) * E, thr, E, valid, bits, tid);
    wave_expert_counts(bits, E, tid, wave, wcnt);
    const int ks = wave_sum_int(k);
    if (lane_id() == 0) wk[wave] = ks;
    __syncthreads();
    for (int e = tid; e < E; e += kRouteThreads)
        chunk_counts[(int64_t)blockIdx.x * E + e] = wcnt[e] + wcnt[E + e] + wcnt[2 * E + e] + wcnt[3 * E + e];
    if (tid == 0) chunk_slots[blockIdx.x] = wk[0] + wk[1] + wk[2] + wk[3];
}

__global__ __launch_bounds__(kRouteThreads) void route_scan_kernel(
    const int32_t* __restrict__ chunk_counts, const int32_t* __restrict__ chunk_slots, int NC,
    int E, int32_t* __restrict__ counts, int32_t* __restrict__ chunk_base,
    int32_t* __restrict__ chunk_slot_base)
{
    __shared__ int part[kRouteWaves][kWave];
    __shared__ int wtot[kRouteWaves];
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int nEB = (E + kWave - 1) / kWave;
    if ((int)blockIdx.x < nEB) {
        // lane = expert, waves split the chunks into 4 contiguous ranges
        const int e = blockIdx.x * kWave + lane;
        const bool ve = e < E;
        const int R = (NC + kRouteWaves - 1) / kRouteWaves;
        const int r0 = min(NC, wave * R), r1 = min(NC, r0 + R);
        int sum = 0;
        if (ve)
            for (int r = r0; r < r1; ++r) sum += chunk_counts[(int64_t)r * E + e];
        part[wave][lane] = sum;
        __syncthreads();
        int base = 0, total = 0;
        for (int i = 0; i < kRouteWaves; ++i) {
            const int p = part[i][lane];
            if (i < wave) base += p;
            total += p;
        }
        if (ve) {
            int run = base;
            for (int r = r0; r < r1; ++r) {
                const int v = chunk_counts[(int64_t)r * E + e];
                chunk_base[(int64_t)r * E + e] = run;
                run += v;
            }
            if (wave == 0) counts[e] = total;
        }
    } else {
        // exclusive scan of the per-chunk slot totals
        const int R = (NC + kRouteThreads - 1) / kRouteThreads;
        const int r0 = min(NC, tid * R), r1 = min(NC, r0 + R);
        int sum = 0;
        for (int r = r0; r < r1; ++r) sum += chunk_slots[r];
        const int incl = wave_incl_scan(sum);
        if (lane == kWave - 1) wtot[wave] = incl;
        __syncthreads();
        int run = incl - sum;
        for (int i = 0; i < wave; ++i) run += wtot[i];
        for (int r = r0; r < r1; ++r) {
            const int v = chunk_slots[r];
            chunk_slot_base[r] = run;
            run += v;
        }
    }
}

template <bool VEC>
__global__ __launch_bounds__(kRouteThreads) void route_fill_kernel(
    const float* __restrict__ logits, const float* __restrict__ thr, int T, int E,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ chunk_base,
    const int32_t* __restrict__ chunk_slot_base, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ token_offsets, int32_t* __restrict__ sorted_token,
    float* __restrict__ slot_gate, int32_t* __restrict__ token_slot, int64_t cap)
{
    extern __shared__ uint32_t smem[];
    const int ng = (E + 31) >> 5;
    uint32_t* bits = smem;                                          // [ng][256]
    int* wbase = reinterpret_cast<int*>(smem + ng * kRouteThreads); // [4][E]
    int* eoff = wbase + kRouteWaves * E;                            // [E]
    __shared__ int wsum[kRouteWaves];

    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // A. expert_offsets = exclusive scan of counts (each thread owns 4 experts)
    int c4[4];
    int csum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = tid * 4 + i;
        c4[i] = e < E ? counts[e] : 0;
        csum += c4[i];
    }
    {
        const int incl = wave_incl_scan(csum);
        if (lane == kWave - 1) wsum[wave] = incl;
        __syncthreads();
        int run = incl - csum;
        int total = 0;
        for (int i = 0; i < kRouteWaves; ++i) {
            if (i < wave) run += wsum[i];
            total += wsum[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid * 4 + i;
            if (e < E) {
                eoff[e] = run;
                if (blockIdx.x == 0) expert_offsets[e] = run;
            }
            run += c4[i];
        }
        if (blockIdx.x == 0 && tid == 0) {
            expert_offsets[E] = total;
            token_offsets[T] = total;
        }
        __syncthreads();  // wsum is reused below
    }

    // B. selection bits and per-wave expert counts
    const int64_t t = (int64_t)blockIdx.x * kRouteThreads + tid;
    const bool valid = t < T;
    const float* row = logits + (valid ? t : 0) * E;
    const int k = select_token<VEC>(row, thr, E, valid, bits, tid);
    wave_expert_counts(bits, E, tid, wave, wbase);

    // token offsets: exclusive scan of k over the chunk
    const int kin = wave_incl_scan(k);
    if (lane == kWave - 1) wsum[wave] = kin;
    __syncthreads();
    int tok_pos = chunk_slot_base[blockIdx.x] + kin - k;
    for (int i = 0; i < wave; ++i) tok_pos += wsum[i];
    // per-wave count -> absolute slot base of (wave, e)
    for (int e = tid; e < E; e += kRouteThreads) {
        int run = eoff[e] + chunk_base[(int64_t)blockIdx.x * E + e];
        for (int i = 0; i < kRouteWaves; ++i) {
            const int c = wbase[i * E + e];
            wbase[i * E + e] = run;
            run += c;
        }
    }
    __syncthreads();
    if (valid) token_offsets[t] = tok_pos;

    // C. place every selected (t, e)
    int j = 0;
    for (int g = 0; g < ng; ++g) {
        const uint32_t wb = bits[g * kRouteThreads + tid];
        const int n = min(32, E - g * 32);
        for (int b = 0; b < n; ++b) {
            const uint32_t on = (wb >> b) & 1u;
            const uint64_t bal = __ballot(on);
            if (on) {
                const int e = g * 32 + b;
                const int64_t slot = (int64_t)wbase[wave * E + e] + rank_below(bal);
                if (slot < cap) {
                    sorted_token[slot] = (int32_t)t;
                    slot_gate[slot] = sigmoid(row[e]);
                }
                if ((int64_t)tok_pos + j < cap) token_slot[tok_pos + j] = (int32_t)slot;
                ++j;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// EMA threshold update: exact per-expert c-th largest score by 4 passes of an
// 8-bit MSB-first radix select on the score bits, then the EMA.
// ---------------------------------------------------------------------------

constexpr int kThrThreads = 256;

struct ThrWs {
    uint32_t* prefix;  // [E]  bits of the selected key fixed so far
    uint32_t* rank;    // [E]  rank still to find among keys matching prefix
    uint32_t* hist;    // [E * 256]
    size_t bytes;
};

static ThrWs thr_ws_layout(void* base, int64_t E)
{
    ThrWs ws{};
    size_t off = 0;
    char* b = static_cast<char*>(base);
    ws.prefix = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.rank = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.hist = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 256 * 4);
    ws.bytes = off;
    return ws;
}

__global__ __launch_bounds__(kThrThreads) void thr_init_kernel(int E, uint32_t c, uint32_t* prefix,
                                                               uint32_t* rank, uint32_t* hist)
{
    const int64_t i = (int64_t)blockIdx.x * kThrThreads + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kThrThreads;
    if (i < E) { prefix[i] = 0u; rank[i] = c; }
    for (int64_t j = i; j < (int64_t)E * 256; j += stride) hist[j] = 0u;
}

__device__ __forceinline__ uint32_t score_key(float l)
{
    const float s = sigmoid(l);
    return (s != s) ? 0u : f2u(s);
}

// grid (token blocks, expert groups of 64); lane = expert; LDS histogram laid
// out [digit][lane] so a wave's 64 updates always land in 64 distinct banks.
__global__ __launch_bounds__(kThrThreads) void thr_hist_kernel(
    const float* __restrict__ logits, int T, int E, int shift, int tokens_per_block,
    const uint32_t* __restrict__ prefix, uint32_t* __restrict__ hist)
{
    __shared__ uint32_t h[256 * kWave];
    const int tid = threadIdx.x;
    for (int i = tid; i < 256 * kWave; i += kThrThreads) h[i] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = blockIdx.y * kWave + lane;
    const bool ve = e < E;
    const uint32_t hmask = (shift == 24) ? 0u : (0xffffffffu << (shift + 8));
    const uint32_t pre = (ve ? prefix[e] : 0u) & hmask;
    const int64_t t0 = (int64_t)blockIdx.x * tokens_per_block;
    const int64_t t1 = min((int64_t)T, t0 + tokens_per_block);
    if (ve) {
#pragma unroll 4
        for (int64_t t = t0 + wave; t < t1; t += kThrThreads / kWave) {
            const uint32_t key = score_key(logits[t * E + e]);
            if ((key & hmask) == pre) atomicAdd(&h[((key >> shift) & 255u) * kWave + lane], 1u);
        }
    }
    __syncthreads();
    for (int i = tid; i < 256 * kWave; i += kThrThreads) {
        const uint32_t v = h[i];
        const int ee = blockIdx.y * kWave + (i & (kWave - 1));
        if (v != 0u && ee < E) atomicAdd(&hist[(int64_t)ee * 256 + (i >> 6)], v);
    }
}

// one wave per expert: find the digit holding the rank-th largest key, update
// prefix and rank, and clear the expert's histogram for the next pass.
__global__ __launch_bounds__(kThrThreads) void thr_select_kernel(int E, int shift,
                                                                 uint32_t* __restrict__ prefix,
                                                                 uint32_t* __restrict__ rank,
                                                                 uint32_t* __restrict__ hist)
{
    const int lane = lane_id();
    const int e = blockIdx.x * (kThrThreads / kWave) + (threadIdx.x >> 6);
    if (e >= E) return;
    uint32_t* he = hist + (int64_t)e * 256;
    // position p = 4*lane + i walks the bins from the top: bin = 255 - p
    uint32_t c[4];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c[i] = he[255 - (4 * lane + i)];
        tot += (int)c[i];
    }
    const int incl = wave_incl_scan(tot);
    const int excl = incl - tot;
    const int r = (int)rank[e];
    const bool mine = excl < r && r <= incl;
    const uint64_t who = __ballot(mine);
    if (mine) {
        int run = excl;
        int pos = 4 * lane + 3;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (run + (int)c[i] >= r) { pos = 4 * lane + i; break; }
            run += (int)c[i];
        }
        const uint32_t bin = 255u - (uint32_t)pos;
        prefix[e] = prefix[e] | (bin << shift);
        rank[e] = (uint32_t)(r - run);
    }
    (void)who;
#pragma unroll
    for (int i = 0; i < 4; ++i) he[255 - (4 * lane + i)] = 0u;
}

__global__ __launch_bounds__(kThrThreads) void thr_finalize_kernel(int E, const uint32_t* __restrict__ prefix,
                                                                   float* __restrict__ thr,
                                                                   float* __restrict__ stat, float m)
{
    const int e = blockIdx.x * kThrThreads + threadIdx.x;
    if (e >= E) return;
    const float st = u2f(prefix[e]);
    if (stat) stat[e] = st;
    const float one_minus_m = 1.0f - m;
    thr[e] = __builtin_fmaf(m, thr[e], one_minus_m * st);
}

static int route_smem_bytes(int E, bool fill)
{
    const int ng = (E + 31) >> 5;
    return (ng * kRouteThreads + kRouteWaves * E + (fill ? E : 0)) * 4;
}

}  // namespace et

using namespace et;

extern "C" size_t et_route_workspace_bytes(int64_t num_tokens, int64_t num_experts)
{
    if (num_tokens < 0 || num_experts < 1) return 0;
    return route_ws_layout(nullptr, num_tokens, num_experts).bytes;
}

extern "C" int et_route(const float* logits, const float* thr, int64_t T, int64_t E,
                        int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                        int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                        int64_t slot_capacity, void* workspace, size_t workspace_bytes, void* stream)
{
    if (T < 0) return fail(ET_ERR_INVALID_ARGUMENT, "et_route: num_tokens < 0");
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_route: num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (T * E >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_route: num_tokens * num_experts must be < 2^31");
    if (slot_capacity < 0) return fail(ET_ERR_INVALID_ARGUMENT, "et_route: slot_capacity < 0");
    if (!thr || !counts || !expert_offsets || !token_offsets || !workspace)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_route: null thr/counts/offsets/workspace pointer");
    if (T > 0 && !logits) return fail(ET_ERR_INVALID_ARGUMENT, "et_route: null logits");
    if (slot_capacity > 0 && (!sorted_token || !slot_gate || !token_slot))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_route: null slot array with slot_capacity > 0");
    const RouteWs ws = route_ws_layout(workspace, T, E);
    if (workspace_bytes < ws.bytes)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_route: workspace needs " + std::to_string(ws.bytes) +
                                                    " bytes, got " + std::to_string(workspace_bytes));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int NC = (int)((T + kRouteThreads - 1) / kRouteThreads > 0 ? (T + kRouteThreads - 1) / kRouteThreads : 1);
    const bool vec = (E % 4 == 0) && ((reinterpret_cast<uintptr_t>(logits) & 15) == 0);
    const int Ti = (int)T, Ei = (int)E;

    if (vec)
        route_count_kernel<true><<<dim3(NC), dim3(kRouteThreads), route_smem_bytes(Ei, false), s>>>(logits, thr, Ti, Ei, ws.chunk_counts, ws.chunk_slots);
    else
        route_count_kernel<false><<<dim3(NC), dim3(kRouteThreads), route_smem_bytes(Ei, false), s>>>(logits, thr, Ti, Ei, ws.chunk_counts, ws.chunk_slots);
    if (int rc = check_launch("route_count_kernel")) return rc;

    const int nEB = (Ei + kWave - 1) / kWave;
    route_scan_kernel<<<dim3(nEB + 1), dim3(kRouteThreads), 0, s>>>(ws.chunk_counts, ws.chunk_slots, NC, Ei, counts, ws.chunk_base, ws.chunk_slot_base);
    if (int rc = check_launch("route_scan_kernel")) return rc;

    if (vec)
        route_fill_kernel<true><<<dim3(NC), dim3(kRouteThreads), route_smem_bytes(Ei, true), s>>>(logits, thr, Ti, Ei, counts, ws.chunk_base, ws.chunk_slot_base, expert_offsets, token_offsets, sorted_token, slot_gate, token_slot, slot_capacity);
    else
        route_fill_kernel<false><<<dim3(NC), dim3(kRouteThreads), route_smem_bytes(Ei, true), s>>>(logits, thr, Ti, Ei, counts, ws.chunk_base, ws.chunk_slot_base, expert_offsets, token_offsets, sorted_token, slot_gate, token_slot, slot_capacity);
    return check_launch("route_fill_kernel");
}

extern "C" size_t et_threshold_workspace_bytes(int64_t num_tokens, int64_t num_experts)
{
    (void)num_tokens;
    if (num_experts < 1) return 0;
    return thr_ws_layout(nullptr, num_experts).bytes;
}

extern "C" int et_threshold_update(const float* logits, float* thr, int64_t T, int64_t E,
                                   int64_t k_target, float momentum, float* stat,
                                   void* workspace, size_t workspace_bytes, void* stream)
{
    if (T < 0) return fail(ET_ERR_INVALID_ARGUMENT, "et_threshold_update: num_tokens < 0");
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_threshold_update: num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (T * E >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_threshold_update: num_tokens * num_experts must be < 2^31");
    if (k_target < 1 || k_target > E)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_threshold_update: k_target must be in [1, num_experts]");
    if (!(momentum >= 0.0f && momentum <= 1.0f))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_threshold_update: momentum must be in [0, 1]");
    if (!thr || !workspace) return fail(ET_ERR_INVALID_ARGUMENT, "et_threshold_update: null thr/workspace");
    if (T > 0 && !logits) return fail(ET_ERR_INVALID_ARGUMENT, "et_threshold_update: null logits");
    const ThrWs ws = thr_ws_layout(workspace, E);
    if (workspace_bytes < ws.bytes)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_threshold_update: workspace needs " +
                                                    std::to_string(ws.bytes) + " bytes, got " +
                                                    std::to_string(workspace_bytes));
    if (T == 0) return ET_OK;
    int64_t c = (T * k_target + E - 1) / E;
    if (c < 1) c = 1;
    if (c > T) c = T;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int Ti = (int)T, Ei = (int)E;

    const int init_blocks = (int)std::min<int64_t>((E * 256 + kThrThreads - 1) / kThrThreads, 1024);
    thr_init_kernel<<<dim3(init_blocks), dim3(kThrThreads), 0, s>>>(Ei, (uint32_t)c, ws.prefix, ws.rank, ws.hist);
    if (int rc = check_launch("thr_init_kernel")) return rc;

    // about 512 blocks over the whole grid; each wave walks a strided token range
    const int egroups = (Ei + kWave - 1) / kWave;
    int64_t tblocks = std::max<int64_t>(1, 512 / egroups);
    int64_t tpb = (T + tblocks - 1) / tblocks;
    tpb = std::max<int64_t>(tpb, 64);
    tblocks = (T + tpb - 1) / tpb;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        thr_hist_kernel<<<dim3((unsigned)tblocks, egroups), dim3(kThrThreads), 0, s>>>(logits, Ti, Ei, shift, (int)tpb, ws.prefix, ws.hist);
        if (int rc = check_launch("thr_hist_kernel")) return rc;
        thr_select_kernel<<<dim3((Ei + 3) / 4), dim3(kThrThreads), 0, s>>>(Ei, shift, ws.prefix, ws.rank, ws.hist);
        if (int rc = check_launch("thr_select_kernel")) return rc;
    }
    thr_finalize_kernel<<<dim3((Ei + kThrThreads - 1) / kThrThreads), dim3(kThrThreads), 0, s>>>(Ei, ws.prefix, thr, stat, momentum);
    return check_launch("thr_finalize_kernel");
}
