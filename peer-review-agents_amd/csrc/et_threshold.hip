// et_threshold.hip -- EMA update of the per-expert routing thresholds, for
// gfx950: the exact c-th largest sigmoid score of every expert's column, then
// thr[e] = fma(momentum, thr[e], (1 - momentum) * stat[e]).
//
// Scores are ordered by their bit pattern, the key (a NaN score keys as 0; a
// score is in [0, 1], so a key is at most f2u(1.0)).  Four launches:
//   histogram pass: reads the logits and counts each score's digit
//     floor(score * 256) (255 for a score of 1, 0 for NaN) per expert, taken
//     from a fast sigmoid checked against per-digit logit bounds (the exact
//     score only where the check fails).  The digit is a monotone function of
//     the key that spreads scores over [0, 1] evenly, where the key's top
//     bits would spend most of their values on the exponent.
//   bin select (one block per expert): sums the blocks' histograms, finds the
//     digit bin that holds the c-th largest key and the rank left inside it,
//     and turns the bin's two score edges into logit bounds (select_bounds).
//   collect pass: reads the logits again.  A logit at or below the lower
//     bound scores below the bin and one at or above the upper bound above
//     it, so only the others (and NaN) have their exact key evaluated; keys in
//     the bin are listed in the block's segment of the expert's candidate list.
//   final select (one block per expert): the rank-th largest listed key, by an
//     MSB-first radix select over the bits in which the bin's keys can differ,
//     8 bits per round, each round an LDS histogram over the candidates (held
//     in LDS when they fit); then the EMA.
// On sigmoid(randn) scores the bin of the c-th largest holds about 0.5% of a
// column (some 600 keys per expert at T = 131072); ties or a narrow score
// range only make the candidate lists longer.  No pass uses a global atomic:
// a block counts in LDS and writes its histogram whole, a collect block
// appends to its own segment of the expert's list (an LDS counter per expert
// gives the index), and only the segments' contents, not their order, enter
// the result, so it is deterministic.
//   Histogram and collect blocks: grid (token blocks, 64-expert groups), 16
//     waves per block, lane = expert (coalesced row segments).  Counts are
//     16-bit in LDS, two digits to a word, written whole to
//     partial[group][block][lane][d / 2].
// The bin-select, collect and final-select passes are block functions
// (et_threshold_internal.hpp): et_threshold_update launches them as their own
// kernels, et_route_update as extra blocks of the routing's launches.
#include <algorithm>

#include "et_common.hpp"
#include "et_route_internal.hpp"
#include "et_threshold_internal.hpp"

namespace et {

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Token blocks per 64-expert group of the histogram and collect passes.
struct HistGrid {
    int64_t blocks;  // token blocks per group
    int64_t tpb;     // tokens per block
};

static HistGrid hist_grid(int64_t T, int64_t E)
{
    const int64_t groups = (E + kWave - 1) / kWave;
    HistGrid g;
    int64_t b = std::max<int64_t>(1, kHistBlocks / groups);
    b = std::max<int64_t>(b, (T + kMaxTokensPerBlock - 1) / kMaxTokensPerBlock);
    g.tpb = std::max<int64_t>(1, (T + b - 1) / b);
    g.tpb = std::max<int64_t>(g.tpb, (int64_t)kHistWaves * kHistUT);
    g.tpb = std::min<int64_t>(g.tpb, kMaxTokensPerBlock);
    g.blocks = std::max<int64_t>(1, (T + g.tpb - 1) / g.tpb);
    return g;
}

struct ThrWs {
    uint32_t* bin;      // [E]  digit bin of the c-th largest key
    uint32_t* rank;     // [E]  its rank inside the bin (1 = the bin's largest)
    uint32_t* key;      // [E]  the statistic's key (final select)
    float* bnd;         // [2 E] logit bounds of the collect pass: (lo, hi) per expert
    uint32_t* partial;  // [groups][blocks][64][kBinWords] block histograms (16-bit counts, packed)
    uint32_t* cand;     // [E][T] keys in the bin; block b's at [b * tpb, ...)
    uint32_t* cand_n;   // [E][blocks] candidates of each collect block
    HistGrid g;
    size_t bytes;
};

static ThrWs thr_ws_layout(void* base, int64_t T, int64_t E)
{
    ThrWs ws{};
    ws.g = hist_grid(T, E);
    const int64_t groups = (E + kWave - 1) / kWave;
    size_t off = 0;
    char* b = static_cast<char*>(base);
    auto take = [&](size_t bytes) {
        void* q = b + off;
        off += align256(bytes);
        return q;
    };
    ws.bin = static_cast<uint32_t*>(take(size_t(E) * 4));
    ws.rank = static_cast<uint32_t*>(take(size_t(E) * 4));
    ws.key = static_cast<uint32_t*>(take(size_t(E) * 4));
    ws.bnd = static_cast<float*>(take(size_t(E) * 8));
    ws.partial = static_cast<uint32_t*>(take(size_t(groups * ws.g.blocks) * kHistWords * 4));
    ws.cand = static_cast<uint32_t*>(take(size_t(T * E) * 4));
    ws.cand_n = static_cast<uint32_t*>(take(size_t(E * ws.g.blocks) * 4));
    ws.bytes = off;
    return ws;
}

// LDS histogram of one block: 16-bit counts, two digits to a word, word
// (d >> 1) * kPitch + lane; a block covers at most 65535 tokens, so a half
// never carries into its neighbour.  Cleared by the block before use.
__device__ __forceinline__ void hist_add(uint32_t* h, uint32_t d, int lane)
{
    atomicAdd(&h[(d >> 1) * kPitch + lane], 1u << ((d & 1u) * 16));
}

__device__ __forceinline__ void hist_flush(const uint32_t* h, uint32_t* __restrict__ partial)
{
    uint32_t* out = partial + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kHistWords;
    for (int i = (int)threadIdx.x; i < kHistWords; i += kHistThreads) {
        const int l = i / kBinWords, j = i % kBinWords;
        out[i] = h[j * kPitch + l];
    }
}

// Histogram pass: the digit of every key of the block's tokens.  Each wave
// takes UT consecutive tokens at a time with all UT loads issued before the
// first use (addresses clamped into the matrix).
//   The digit is found in the logit domain, as routing decides selection:
// digit d holds the scores in [d / kBins, (d + 1) / kBins), so with the logit
// bounds of select_bounds, a logit l with hi(d / kBins) <= l and l <=
// lo((d + 1) / kBins) has digit d (the score's order is monotone up to 2
// steps, which those bounds allow for).  The block puts the pairs
// (hi(d / kBins), lo((d + 1) / kBins)) of every d in LDS while its first loads
// are in flight; a lane then takes d from a fast approximate sigmoid and
// checks it against its pair, and only a lane whose check fails (a logit near
// a digit edge or NaN: rare) evaluates the exact key.  So the digits are
// exactly those of score_digit(score_key(l)).
template <int UT>
__global__ __launch_bounds__(kHistThreads) void thr_hist_kernel(const float* __restrict__ logits, int T, int E,
                                                                int tpb, uint32_t* __restrict__ partial)
{
    __shared__ uint32_t h[kBinWords * kPitch];
    __shared__ float2 dtab[kBins];
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = blockIdx.y * kWave + lane;
    const bool ve = e < E;
    const int ec = min(e, E - 1);
    const int64_t t0 = (int64_t)blockIdx.x * tpb;
    const int64_t t1 = min((int64_t)T, t0 + tpb);
    // the wave's first batch of loads, then the LDS set-up under them
    int64_t tb = t0 + (int64_t)wave * UT;
    float v[UT];
    if (tb < t1) {
#pragma unroll
        for (int u = 0; u < UT; ++u) v[u] = logits[min(tb + u, t1 - 1) * E + ec];
    }
    for (int i = tid; i < kBinWords * kPitch; i += kHistThreads) h[i] = 0u;
    if (tid < kBins) {
        // thread b: the bounds of the score b / kBins (hi(0) = -inf); the
        // last digit also holds the score 1, so nothing bounds it above
        float hi, lo;
        select_bounds(bin_edge((uint32_t)tid), hi, lo);
        dtab[tid].x = hi;
        if (tid > 0) dtab[tid - 1].y = lo;
        if (tid == kBins - 1) dtab[tid].y = __builtin_huge_valf();
    }
    __syncthreads();
    for (; tb < t1; tb += (int64_t)kHistWaves * UT) {
        if (tb != t0 + (int64_t)wave * UT) {
#pragma unroll
            for (int u = 0; u < UT; ++u) v[u] = logits[min(tb + u, t1 - 1) * E + ec];
        }
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            if (!ve || tb + u >= t1) continue;
            const float l = v[u];
            // approximate digit (a NaN converts to 0 and fails the check)
            const float sa = __builtin_amdgcn_rcpf(1.0f + __expf(-l));
            const uint32_t da = min((uint32_t)(sa * (float)kBins), (uint32_t)kBins - 1u);
            const float2 b = dtab[da];
            const bool ok = l >= b.x && l <= b.y;
            uint32_t d = da;
            if (__ballot(!ok) != 0ull) {         // (skipped by the whole wave when every check holds)
                if (!ok) d = score_digit(score_key(l));
            }
            hist_add(h, d, lane);
        }
    }
    __syncthreads();
    hist_flush(h, partial);
}

template <int UT>
__global__ __launch_bounds__(kHistThreads) void thr_collect_kernel(
    const float* __restrict__ logits, int T, int E, int tpb, const uint32_t* __restrict__ bin,
    const float* __restrict__ bnd, uint32_t* __restrict__ cand, uint32_t* __restrict__ cand_n)
{
    thr_collect_block<UT>((int)blockIdx.x, (int)blockIdx.y, (int)gridDim.x, logits, T, E, tpb, bin, bnd, cand,
                          cand_n);
}

// The bin select's own kernel (thr_bin_block: et_threshold_internal.hpp).
__global__ __launch_bounds__(kSelectThreads) void thr_bin_kernel(int nblocks,
                                                                 const uint32_t* __restrict__ partial, uint32_t c,
                                                                 uint32_t* __restrict__ bin,
                                                                 uint32_t* __restrict__ rank, float* __restrict__ bnd)
{
    thr_bin_block((int)blockIdx.x, nblocks, partial, c, bin, rank, bnd);
}

// The final select's own kernel (thr_final_block: et_threshold_internal.hpp).
__global__ __launch_bounds__(kSelectThreads) void thr_final_kernel(
    int nblocks, int T, int tpb, const uint32_t* __restrict__ bin, const uint32_t* __restrict__ rank,
    uint32_t* __restrict__ key_out, const uint32_t* __restrict__ cand, const uint32_t* __restrict__ cand_n,
    float* __restrict__ thr, float* __restrict__ stat, float m)
{
    __shared__ uint32_t lds[kFinalLdsWords<kSelectThreads, kFinalLdsKeys>];
    thr_final_block<kSelectThreads, kFinalLdsKeys>((int)blockIdx.x, nblocks, T, tpb, bin, rank, key_out, cand, cand_n,
                                                   thr, stat, m, lds);
}

// The passes on stream s; the final select applies the EMA (and writes stat).
static int thr_passes(const float* logits, int64_t T, int64_t E, int64_t k_target, float* thr, float* stat,
                      float momentum, const ThrWs& ws, hipStream_t s)
{
    const int64_t c = thr_rank(T, E, k_target);
    const int Ti = (int)T, Ei = (int)E;
    const unsigned groups = (unsigned)((E + kWave - 1) / kWave);
    const dim3 grid((unsigned)ws.g.blocks, groups);
    const int tpb = (int)ws.g.tpb, nb = (int)ws.g.blocks;
    thr_hist_kernel<kHistUT><<<grid, dim3(kHistThreads), 0, s>>>(logits, Ti, Ei, tpb, ws.partial);
    if (int rc = check_launch("thr_hist_kernel")) return rc;
    thr_bin_kernel<<<dim3(Ei), dim3(kSelectThreads), 0, s>>>(nb, ws.partial, (uint32_t)c, ws.bin, ws.rank,
                                                               ws.bnd);
    if (int rc = check_launch("thr_bin_kernel")) return rc;
    thr_collect_kernel<kHistUT><<<grid, dim3(kHistThreads), 0, s>>>(logits, Ti, Ei, tpb, ws.bin, ws.bnd, ws.cand,
                                                                     ws.cand_n);
    if (int rc = check_launch("thr_collect_kernel")) return rc;
    thr_final_kernel<<<dim3(Ei), dim3(kSelectThreads), 0, s>>>(nb, Ti, tpb, ws.bin, ws.rank, ws.key, ws.cand,
                                                                ws.cand_n, thr, stat, momentum);
    return check_launch("thr_final_kernel");
}

// Argument checks of the EMA update (host only).
static int thr_check(const char* fn, const float* logits, float* thr, int64_t T, int64_t E, int64_t k_target,
                     float momentum, void* workspace, size_t workspace_bytes)
{
    const std::string f(fn);
    if (T < 0) return fail(ET_ERR_INVALID_ARGUMENT, f + ": num_tokens < 0");
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, f + ": num_experts must be in [1, " + std::to_string(ET_MAX_EXPERTS) + "]");
    if (T * E >= (int64_t(1) << 31)) return fail(ET_ERR_INVALID_ARGUMENT, f + ": num_tokens * num_experts must be < 2^31");
    if (k_target < 1 || k_target > E) return fail(ET_ERR_INVALID_ARGUMENT, f + ": k_target must be in [1, num_experts]");
    if (!(momentum >= 0.0f && momentum <= 1.0f)) return fail(ET_ERR_INVALID_ARGUMENT, f + ": momentum must be in [0, 1]");
    if (!thr || !workspace) return fail(ET_ERR_INVALID_ARGUMENT, f + ": null thr/workspace");
    if (T > 0 && !logits) return fail(ET_ERR_INVALID_ARGUMENT, f + ": null logits");
    const size_t need = thr_ws_layout(nullptr, T, E).bytes;
    if (workspace_bytes < need)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, f + ": workspace needs " + std::to_string(need) + " bytes, got " +
                                                    std::to_string(workspace_bytes));
    return ET_OK;
}

// Byte ranges [a, a + na) and [b, b + nb) overlap.
static bool overlaps(const void* a, size_t na, const void* b, size_t nb)
{
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + nb && y < x + na;
}

}  // namespace et

using namespace et;

extern "C" size_t et_threshold_workspace_bytes(int64_t num_tokens, int64_t num_experts)
{
    if (num_tokens < 0 || num_experts < 1) return 0;
    return thr_ws_layout(nullptr, num_tokens, num_experts).bytes;
}

extern "C" int et_threshold_update(const float* logits, float* thr, int64_t T, int64_t E,
                                   int64_t k_target, float momentum, float* stat,
                                   void* workspace, size_t workspace_bytes, void* stream)
{
    if (int rc = thr_check("et_threshold_update", logits, thr, T, E, k_target, momentum, workspace, workspace_bytes))
        return rc;
    if (T == 0) return ET_OK;
    return thr_passes(logits, T, E, k_target, thr, stat, momentum, thr_ws_layout(workspace, T, E),
                      static_cast<hipStream_t>(stream));
}

extern "C" int et_route_update(const float* logits, float* thr, int64_t T, int64_t E, int32_t* counts,
                               int32_t* expert_offsets, int32_t* token_offsets, int32_t* sorted_token,
                               float* slot_gate, int32_t* token_slot, int64_t slot_capacity, void* route_workspace,
                               size_t route_workspace_bytes, int64_t k_target, float momentum, float* stat,
                               void* thr_workspace, size_t thr_workspace_bytes, void* stream)
{
    const char* fn = "et_route_update";
    if (int rc = route_check(fn, logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                             token_slot, slot_capacity))
        return rc;
    if (!route_workspace) return fail(ET_ERR_INVALID_ARGUMENT, "et_route_update: null route workspace");
    const size_t rneed = et_route_workspace_bytes(T, E);
    if (route_workspace_bytes < rneed)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_route_update: route workspace needs " + std::to_string(rneed) +
                                                    " bytes, got " + std::to_string(route_workspace_bytes));
    if (int rc = thr_check(fn, logits, thr, T, E, k_target, momentum, thr_workspace, thr_workspace_bytes)) return rc;
    if (overlaps(route_workspace, rneed, thr_workspace, thr_ws_layout(nullptr, T, E).bytes))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_route_update: the route and threshold workspaces overlap");
    // The routing reads thr before the update writes it: both on `stream`.
    // On the pair-list path (up to 256 experts) the update's passes run beside
    // the routing's: histogram; count with the bin select; scan with the
    // collect pass; place with the final select (or place, then the final
    // select, where the route tiles hold fewer than 16 groups).
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const ThrWs ws = thr_ws_layout(thr_workspace, T, E);
    if (T > 0 && E <= 4 * kWave && route_uses_pairs(T, E)) {
        const unsigned groups = (unsigned)((E + kWave - 1) / kWave);
        const dim3 grid((unsigned)ws.g.blocks, groups);
        const int Ti = (int)T, Ei = (int)E, tpb = (int)ws.g.tpb, nb = (int)ws.g.blocks;
        thr_hist_kernel<kHistUT><<<grid, dim3(kHistThreads), 0, s>>>(logits, Ti, Ei, tpb, ws.partial);
        if (int rc = check_launch("thr_hist_kernel")) return rc;
        if (int rc = route_update_count_bin(logits, thr, T, E, route_workspace, ws.partial, nb,
                                            (uint32_t)thr_rank(T, E, k_target), ws.bin, ws.rank, ws.bnd, s))
            return rc;
        if (int rc = route_update_scan_collect(T, E, route_workspace, logits, nb, tpb, ws.bin, ws.bnd, ws.cand,
                                               ws.cand_n, s))
            return rc;
        if (route_update_pairs_final(T, E))
            return route_update_place_final(T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                                            token_slot, slot_capacity, route_workspace, nb, tpb, ws.bin, ws.rank,
                                            ws.key, ws.cand, ws.cand_n, thr, stat, momentum, s);
        if (int rc = route_update_place(T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                                        token_slot, slot_capacity, route_workspace, s))
            return rc;
        thr_final_kernel<<<dim3((unsigned)Ei), dim3(kSelectThreads), 0, s>>>(nb, Ti, tpb, ws.bin, ws.rank, ws.key,
                                                                            ws.cand, ws.cand_n, thr, stat, momentum);
        return check_launch("thr_final_kernel");
    }
    if (int rc = et_route(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                          token_slot, slot_capacity, route_workspace, route_workspace_bytes, stream))
        return rc;
    if (T == 0) return ET_OK;
    return thr_passes(logits, T, E, k_target, thr, stat, momentum, ws, s);
}
