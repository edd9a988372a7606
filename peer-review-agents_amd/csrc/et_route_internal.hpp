// et_route_internal.hpp -- the selection rule (device) and the host-side
// launchers of the routing kernels shared by the logit-input routing
// (et_route.hip) and the fused router producer (et_router.hip).  Not part of
// the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "et_common.hpp"

namespace et {

// ---------------------------------------------------------------------------
// the selection rule, shared by every routing kernel (device)
// ---------------------------------------------------------------------------

// Thresholds of the lane's experts e = 64 g + lane; NaN past E, so that lane
// never selects.
template <int GM>
__device__ __forceinline__ void load_thresholds(const float* __restrict__ thr, int E, int G, float (&th)[GM])
{
    const int lane = lane_id();
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        th[g] = (g < G && e < E) ? thr[e] : __builtin_nanf("");
    }
}

// Selection of one token: m[g] = ballot(score >= thr) over group g, sc[g] =
// the lane's score.  A token with no expert gets the argmax expert (NaN lowest,
// ties to the lowest expert index; lanes past E hold NaN, so an all-NaN token
// goes to expert 0).  Returns the token's expert count (wave-uniform).  Scores
// are sigmoids, so never negative: their bit patterns order like the values.
// Logit-domain bounds of the test sigmoid(l) >= th, for one expert.  The
// specified sigmoid is monotone up to 2 order steps: over all non-NaN floats,
// bits(s(l)) >= bits(max_{l' <= l} s(l')) - 2, and s(l) >= +0 (exhaustive
// check over all 2^32 floats; scores are non-negative, so their bit patterns
// order like their values).  Hence a logit hi with bits(s(hi)) >= bits(th) + 2
// gives s(l) >= th for every l >= hi, and a logit lo with bits(s(lo)) + 2 <
// bits(th) gives s(l) < th for every l <= lo.  Both are found by stepping out
// from an approximate logit of th, each candidate checked with the exact
// sigmoid; a bound that is not found is NaN and decides nothing.  Logits
// strictly between the bounds, and NaN logits, need the exact score.
//   th NaN or > 1: nothing is selected (hi = NaN, lo = +inf).
//   th <= 0:       every non-NaN logit is selected (hi = -inf, lo = NaN).
// The searches stay loops (not unrolled): the bounds are computed once per
// wave or block, and 48 inlined sigmoids would crowd the instruction cache.
__device__ __forceinline__ void select_bounds(float th, float& hi, float& lo)
{
    const float inf = __builtin_huge_valf();
    const float nan = __builtin_nanf("");
    if (!(th <= 1.0f)) { hi = nan; lo = inf; return; }
    if (th <= 0.0f) { hi = -inf; lo = nan; return; }
    const uint32_t tb = f2u(th);
    const float l0 = th < 1.0f ? __logf(th) - __logf(1.0f - th) : 20.0f;   // approximate logit of th
    const float s0 = __builtin_fmaxf(__builtin_fabsf(l0) * 0x1p-18f, 0x1p-20f);
    hi = nan;
    float step = s0;
#pragma unroll 1
    for (int it = 0; it < 24; ++it) {
        const float h = l0 + step;
        if (f2u(sigmoid(h)) >= tb + 2u) { hi = h; break; }
        step *= 4.0f;
    }
    lo = nan;
    step = s0;
#pragma unroll 1
    for (int it = 0; it < 24; ++it) {
        const float g = l0 - step;
        if (f2u(sigmoid(g)) + 2u < tb) { lo = g; break; }
        step *= 4.0f;
    }
}

// The threshold part of the rule: scores, ballots and the expert count, with
// no fallback (the count may be 0).
template <int GM>
__device__ __forceinline__ int select_scores(const float (&lg)[GM], const float (&th)[GM], int G,
                                             uint64_t (&m)[GM], float (&sc)[GM])
{
    int k = 0;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        sc[g] = sigmoid(lg[g]);
        m[g] = (g < G) ? (uint64_t)__ballot(sc[g] >= th[g]) : 0ull;
        k += (int)__popcll(m[g]);
    }
    return k;
}

// The fallback part: m = the argmax expert of the scores sc (NaN lowest, ties
// to the lowest expert index).  Argmax by two DPP reductions (no LDS round
// trips).  Keys order the scores (all >= 0) by their bits, with NaN below
// every score; each lane keeps its best group, the lowest on ties.  The wave
// max of the keys is the best score; the wave max of ~e over the lanes holding
// it is the lowest expert index with that score.
template <int GM>
__device__ __forceinline__ void select_fallback(const float (&sc)[GM], int G, uint64_t (&m)[GM])
{
    const int lane = lane_id();
    uint32_t bk = 0u;
    int be = lane;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        if (g < G) {
            const uint32_t key = (sc[g] != sc[g]) ? 0u : f2u(sc[g]) + 1u;
            if (key > bk) { bk = key; be = g * kWave + lane; }
        }
    }
    const uint32_t top = wave_max_u32_dpp(bk);
    be = (int)~wave_max_u32_dpp(bk == top ? ~(uint32_t)be : 0u);
#pragma unroll
    for (int g = 0; g < GM; ++g) m[g] = (g == (be >> 6)) ? (1ull << (be & (kWave - 1))) : 0ull;
}

template <int GM>
__device__ __forceinline__ int select_token(const float (&lg)[GM], const float (&th)[GM], int G,
                                            uint64_t (&m)[GM], float (&sc)[GM])
{
    int k = select_scores<GM>(lg, th, G, m, sc);
    if (k == 0) {
        select_fallback<GM>(sc, G, m);
        k = 1;
    }
    return k;
}

// ---------------------------------------------------------------------------
// host-side launchers
// ---------------------------------------------------------------------------

// Argument checks of et_route (host only; `fn` names the entry point in the
// error message).  Returns ET_OK or the error code, with et_last_error set.
int route_check(const char* fn, const float* logits, const float* thr, int64_t T, int64_t E,
                const int32_t* counts, const int32_t* expert_offsets, const int32_t* token_offsets,
                const int32_t* sorted_token, const float* slot_gate, const int32_t* token_slot,
                int64_t slot_capacity);

// et_route takes the pair-list path on (T, E) (T > 0): its pair lists fit
// the 1 GiB bound; otherwise the two-read kernels.
bool route_uses_pairs(int64_t T, int64_t E);

// Column-wise exclusive scan of the per-block expert counts (NB rows of E)
// into counts[E] and block_base[NB * E], and of the per-block slot totals
// into block_slot_base[NB].
int launch_route_scan(const int32_t* block_counts, const int32_t* block_slots, int NB, int E, int32_t* counts,
                      int32_t* block_base, int32_t* block_slot_base, hipStream_t s);

// Routing outputs from per-token selection masks.  Tokens are split into
// route groups of 16 (group q = tokens [16 q, 16 q + 16)), gpt groups per
// block tile (NB tiles).  Token t's selection is masks[t * nwords + e / 32]
// bit e % 32 (nwords = ceil(E / 32)); group q's routed gates are stored in
// token order, ascending expert within a token, from gate_ws[q * 16 * E].
// group_counts / group_slots are the producer's per-group expert counts and
// slot totals; counts, block_base and block_slot_base come from
// launch_route_scan over the tiles.
int launch_route_fill_masks(const uint32_t* masks, const float* gate_ws, int T, int E, int gpt, int NB,
                            const int32_t* counts, const int32_t* group_counts, const int32_t* block_base,
                            const int32_t* group_slots, const int32_t* block_slot_base, int32_t* expert_offsets,
                            int32_t* token_offsets, int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                            int64_t cap, hipStream_t s);

}  // namespace et
