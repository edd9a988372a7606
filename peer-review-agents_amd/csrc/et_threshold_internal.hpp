// et_threshold_internal.hpp -- what the EMA threshold update shares with the
// routing file: its digit constants and score keys, its bin-select, collect
// and final-select passes as per-block device functions (run by their own
// kernels in et_threshold.hip and, for et_route_update, inside the routing's
// count, scan and place launches in et_route.hip), and those routing
// launches.  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "et_common.hpp"
#include "et_route_internal.hpp"

namespace et {

constexpr int kDigitBits = 8;
constexpr int kBins = 1 << kDigitBits;      // histogram digits: floor(score * kBins)
constexpr int kBinWords = kBins / 2;        // two 16-bit counts to a word
constexpr int kHistWaves = 16;
constexpr int kHistThreads = kHistWaves * kWave;
constexpr int64_t kHistBlocks = 256;        // blocks of a pass (whole grid)
constexpr int kHistUT = 16;                 // tokens in flight per wave
constexpr int64_t kMaxTokensPerBlock = 65535;  // LDS counts are 16-bit
constexpr int kPitch = kWave + 1;           // LDS words per digit pair (padded)
constexpr int kHistWords = kWave * kBinWords;  // words of one block histogram
constexpr int kSelectThreads = 1024;
constexpr int kSelectSplit = kSelectThreads / kBinWords;   // bin-select threads per word
constexpr int kSelectRound = 8;             // partial-histogram loads in flight per select thread
constexpr int kFinalLdsKeys = 12288;        // candidates the final select holds in LDS (48 KiB)

// The key of a logit: the bits of its score, NaN as 0 (at most f2u(1.0)).
__device__ __forceinline__ uint32_t score_key(float l)
{
    const float sc = sigmoid(l);
    return (sc != sc) ? 0u : f2u(sc);
}

// The histogram digit of a key: floor(score * kBins), kBins - 1 for a score
// of 1.  (score * kBins is exact, and the conversion truncates.)
__device__ __forceinline__ uint32_t score_digit(uint32_t key)
{
    return min((uint32_t)(u2f(key) * (float)kBins), (uint32_t)kBins - 1u);
}

// The score at the lower edge of digit bin b, b / kBins (exact).
__device__ __forceinline__ float bin_edge(uint32_t b) { return (float)b * (1.0f / (float)kBins); }

// Wave 0 of a select block: the bin of the rank-th largest key (rank r >= 1)
// given NB bin counts cnt(bin) (NB = 64, 128 or 256), bins walked from the
// top.  The lane that holds it returns true with the bin and the rank left
// inside the bin.
template <int NB, typename F>
__device__ __forceinline__ bool find_digit(F cnt, int r, uint32_t& bin, int& rank_in)
{
    constexpr int PER = NB / kWave;
    const int lane = lane_id();
    // position p = PER*lane + i walks the bins from the top: bin = NB - 1 - p
    uint32_t c[PER];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        c[i] = cnt(NB - 1 - (PER * lane + i));
        tot += (int)c[i];
    }
    const int incl = wave_incl_scan(tot);
    const int excl = incl - tot;
    if (!(excl < r && r <= incl)) return false;
    int run = excl;
    int pos = PER * lane + PER - 1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        if (run + (int)c[i] >= r) { pos = PER * lane + i; break; }
        run += (int)c[i];
    }
    bin = (uint32_t)(NB - 1 - pos);
    rank_in = r - run;
    return true;
}

// Bin select, one block per expert: counts[d] = the sum of the expert's block
// histograms (kSelectSplit threads per word of two digits, each over every
// kSelectSplit-th block, all loads of a round issued together; the two 16-bit
// halves are added separately), then wave 0 finds the digit bin that holds the
// c-th largest key, and the logit bounds of the bin's scores [b / kBins,
// (b + 1) / kBins).
// Block e (kSelectThreads threads) of the bin select.
__device__ __forceinline__ void thr_bin_block(int e, int nblocks, const uint32_t* __restrict__ partial, uint32_t c,
                                              uint32_t* __restrict__ bin, uint32_t* __restrict__ rank,
                                              float* __restrict__ bnd)
{
    __shared__ uint32_t part[kSelectSplit][kBins];
    const int tid = threadIdx.x;
    const int q = tid / kBinWords, j = tid % kBinWords;
    const uint32_t* src = partial + (int64_t)(e >> 6) * nblocks * kHistWords + (e & 63) * kBinWords + j;
    uint32_t lo = 0u, hi = 0u;
    for (int b0 = q; b0 < nblocks; b0 += kSelectRound * kSelectSplit) {
        uint32_t v[kSelectRound];
#pragma unroll
        for (int i = 0; i < kSelectRound; ++i)
            v[i] = src[(int64_t)min(b0 + i * kSelectSplit, nblocks - 1) * kHistWords];
#pragma unroll
        for (int i = 0; i < kSelectRound; ++i) {
            const uint32_t w = (b0 + i * kSelectSplit < nblocks) ? v[i] : 0u;
            lo += w & 0xffffu;
            hi += w >> 16;
        }
    }
    part[q][2 * j] = lo;
    part[q][2 * j + 1] = hi;
    __syncthreads();
    if (tid >= kWave) return;
    auto pass_count = [&](int b) {
        uint32_t n = 0u;
#pragma unroll
        for (int k = 0; k < kSelectSplit; ++k) n += part[k][b];
        return n;
    };
    uint32_t b;
    int rin;
    if (find_digit<kBins>(pass_count, (int)c, b, rin)) {
        bin[e] = b;
        rank[e] = (uint32_t)rin;
        // a logit at or below lo_a scores below bin_edge(b); one at or above
        // hi_b scores at least bin_edge(b + 1) (nothing is above the last
        // bin, and a NaN bound decides nothing: comparisons with it are false)
        float hi_a, lo_a, hi_b, lo_b;
        select_bounds(bin_edge(b), hi_a, lo_a);
        select_bounds(bin_edge(b + 1u), hi_b, lo_b);
        bnd[2 * e] = lo_a;
        bnd[2 * e + 1] = b == (uint32_t)kBins - 1u ? __builtin_nanf("") : hi_b;
    }
}

// Collect pass: the keys in bin[e], into the block's segment of the expert's
// list, cand[e][t0 + i] (i from an LDS counter, so i < t1 - t0); the block's
// count goes to cand_n[e][block].  A logit at or below bnd[2e] scores below
// the bin, one at or above bnd[2e + 1] above it; only the others (and NaN)
// have their key evaluated.
// Block (bx, by) of a grid of nbx token blocks by 64-expert groups, kHistThreads threads.
template <int UT>
__device__ __forceinline__ void thr_collect_block(int bx, int by, int nbx, const float* __restrict__ logits, int T,
                                                  int E, int tpb, const uint32_t* __restrict__ bin,
                                                  const float* __restrict__ bnd, uint32_t* __restrict__ cand,
                                                  uint32_t* __restrict__ cand_n)
{
    __shared__ uint32_t cn[kWave];
    const int tid = threadIdx.x;
    if (tid < kWave) cn[tid] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = by * kWave + lane;
    const bool ve = e < E;
    const int ec = min(e, E - 1);
    const uint32_t b1 = bin[ec];
    const float lo = bnd[2 * ec], hi = bnd[2 * ec + 1];
    const int64_t t0 = (int64_t)bx * tpb;
    const int64_t t1 = min((int64_t)T, t0 + tpb);
    for (int64_t tb = t0 + (int64_t)wave * UT; tb < t1; tb += (int64_t)kHistWaves * UT) {
        float v[UT];
#pragma unroll
        for (int u = 0; u < UT; ++u) v[u] = logits[min(tb + u, t1 - 1) * E + ec];
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            if (!ve || tb + u >= t1 || v[u] <= lo || v[u] >= hi) continue;
            const uint32_t key = score_key(v[u]);
            if (score_digit(key) == b1) {
                const uint32_t i = atomicAdd(&cn[lane], 1u);
                cand[(int64_t)e * T + t0 + i] = key;
            }
        }
    }
    __syncthreads();
    if (tid < kWave && ve) cand_n[(int64_t)e * nbx + bx] = cn[tid];
}

// Final select, one block per expert: the rank-th largest listed key.  The
// bin's keys lie in [klo, khi] and share the bits above the highest bit in
// which klo and khi differ; the rest are fixed 8 at a time from the top, each
// round an LDS histogram of the next digit over the candidates that match the
// bits fixed so far.  The candidate segments are walked up to NT
// at a time: a block-wide scan of their counts places them, and thread i of a
// round finds its segment by binary search.  With at most KEYS
// candidates the first walk copies them into LDS and every round reads them
// there; otherwise every round walks the segments again.  Then the EMA; the
// statistic's key is also left in key[e].  Block e of NT threads, whose LDS
// (kFinalLdsWords<NT, KEYS> words at lds) holds up to KEYS candidates.
template <int NT, int KEYS> constexpr int kFinalLdsWords = 256 + NT + NT / kWave + 3 + KEYS;

template <int NT, int KEYS>
__device__ __forceinline__ void thr_final_block(int e, int nblocks, int T, int tpb, const uint32_t* __restrict__ bin,
                                                const uint32_t* __restrict__ rank, uint32_t* __restrict__ key_out,
                                                const uint32_t* __restrict__ cand,
                                                const uint32_t* __restrict__ cand_n, float* __restrict__ thr,
                                                float* __restrict__ stat, float m, uint32_t* lds)
{
    uint32_t* hist = lds;                        // [256]
    uint32_t* seg_end = hist + 256;              // [NT] inclusive scan of a round's segment counts
    uint32_t* wsum = seg_end + NT;               // [NT / 64]
    uint32_t* sel = wsum + NT / kWave;           // [2] the bits fixed so far and the rank inside them
    uint32_t* n_all = sel + 2;                   // [1]
    uint32_t* ck = n_all + 1;                    // [KEYS]
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const uint32_t b1 = bin[e];
    const uint32_t klo = f2u(bin_edge(b1));
    const uint32_t khi = b1 == (uint32_t)kBins - 1u ? f2u(1.0f) : f2u(bin_edge(b1 + 1u)) - 1u;
    const uint32_t diff = klo ^ khi;
    const int nbits = diff ? 32 - __builtin_clz(diff) : 0;   // at most 30
    if (tid == 0) {
        sel[0] = klo & ~((1u << nbits) - 1u);
        sel[1] = rank[e];
    }
    const uint32_t* cl = cand + (int64_t)e * T;
    const uint32_t* cnt = cand_n + (int64_t)e * nblocks;

    // fn(i, key) for every listed key (i = its index in the concatenated list)
    auto walk = [&](auto fn) {
        uint32_t done = 0u;
        for (int b0 = 0; b0 < nblocks; b0 += NT) {
            const int nc = min(NT, nblocks - b0);
            const uint32_t n = tid < nc ? cnt[b0 + tid] : 0u;
            const uint32_t incl = (uint32_t)wave_incl_scan((int)n);
            if (lane_id() == kWave - 1) wsum[wave] = incl;
            __syncthreads();
            uint32_t below = 0u;
            for (int w = 0; w < wave; ++w) below += wsum[w];
            seg_end[tid] = below + incl;
            __syncthreads();
            const uint32_t total = seg_end[nc - 1];
            for (uint32_t i = tid; i < total; i += NT) {
                int lo = 0, hi = nc - 1;                 // the first segment that ends past i
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (seg_end[mid] > i) hi = mid; else lo = mid + 1;
                }
                const uint32_t start = lo ? seg_end[lo - 1] : 0u;
                fn(done + i, cl[(int64_t)(b0 + lo) * tpb + (i - start)]);
            }
            done += total;
            __syncthreads();
        }
        return done;
    };
    // the number of candidates, and a copy in LDS when they fit
    {
        const uint32_t total = walk([&](uint32_t i, uint32_t k) {
            if (i < (uint32_t)KEYS) ck[i] = k;
        });
        if (tid == 0) n_all[0] = total;
        __syncthreads();
    }
    const uint32_t total = n_all[0];
    const bool in_lds = total <= (uint32_t)KEYS;
    for (int sh = nbits; sh > 0; sh -= 8) {
        const int lo_sh = sh > 8 ? sh - 8 : 0;
        if (tid < 256) hist[tid] = 0u;
        __syncthreads();
        const uint32_t fixed = sel[0];
        const uint32_t hmask = ~((1u << sh) - 1u);
        const uint32_t dmask = (1u << (sh - lo_sh)) - 1u;
        auto count = [&](uint32_t, uint32_t k) {
            if ((k & hmask) == fixed) atomicAdd(&hist[(k >> lo_sh) & dmask], 1u);
        };
        if (in_lds) {
            for (uint32_t i = tid; i < total; i += NT) count(i, ck[i]);
        } else {
            walk(count);
        }
        __syncthreads();
        if (tid < kWave) {
            uint32_t b;
            int rin;
            if (find_digit<256>([&](int d) { return hist[d]; }, (int)sel[1], b, rin)) {
                sel[0] = fixed | (b << lo_sh);
                sel[1] = (uint32_t)rin;
            }
        }
        __syncthreads();
    }
    if (tid != 0) return;
    // every bit is fixed: sel[0] is the statistic's key
    const uint32_t p = sel[0];
    key_out[e] = p;
    const float st = u2f(p);
    if (stat) stat[e] = st;
    const float one_minus_m = 1.0f - m;
    thr[e] = __builtin_fmaf(m, thr[e], one_minus_m * st);
}

// The rank of the statistic: c = ceil(T * k_target / E), within [1, T].
inline int64_t thr_rank(int64_t T, int64_t E, int64_t k_target)
{
    int64_t c = (T * k_target + E - 1) / E;
    if (c < 1) c = 1;
    if (c > T) c = T;
    return c;
}

// et_route's launches on the pair-list path (route_uses_pairs(T, E), at most
// 256 experts, arguments and workspace already checked, T > 0), for
// et_route_update, which runs the EMA update's passes beside them: its bin
// select (over nbx histogram blocks per 64-expert group, statistic rank c) in
// the count's launch, and its collect pass (token blocks of tpb tokens) in the
// scan's.
int route_update_count_bin(const float* logits, const float* thr, int64_t T, int64_t E, void* workspace,
                           const uint32_t* partial, int nbx, uint32_t c, uint32_t* bin, uint32_t* rank,
                           float* bnd, hipStream_t s);
int route_update_scan_collect(int64_t T, int64_t E, void* workspace, const float* logits, int nbx, int tpb,
                              const uint32_t* bin, const float* bnd, uint32_t* cand, uint32_t* cand_n,
                              hipStream_t s);
int route_update_place(int64_t T, int64_t E, int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                       int32_t* sorted_token, float* slot_gate, int32_t* token_slot, int64_t slot_capacity,
                       void* workspace, hipStream_t s);
// Where the routing's tiles hold 16 route groups (T of at least 32768 tokens),
// the place launch also runs the update's final select (over the collect
// pass's nbx token blocks of tpb tokens), which applies the EMA to thr.
bool route_update_pairs_final(int64_t T, int64_t E);
int route_update_place_final(int64_t T, int64_t E, int32_t* counts, int32_t* expert_offsets,
                             int32_t* token_offsets, int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                             int64_t slot_capacity, void* workspace, int nbx, int tpb, const uint32_t* bin,
                             const uint32_t* rank, uint32_t* key, const uint32_t* cand, const uint32_t* cand_n,
                             float* thr, float* stat, float m, hipStream_t s);

}  // namespace et
