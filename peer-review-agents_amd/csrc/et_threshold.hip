// et_threshold.hip -- EMA update of the per-expert routing thresholds, for
// gfx950: the exact c-th largest sigmoid score of every expert's column by an
// MSB-first radix select over the score bits, then
// thr[e] = fma(momentum, thr[e], (1 - momentum) * stat[e]).
//
// A score is in [0, 1] (NaN keys as 0), so its bit pattern (the key) is below
// 2^30: bits 31 and 30 are always 0 and the select works on the 30 bits
// below.  Two histogram passes fix bits 29-22 and 21-14, a collect pass lists
// the keys that match those 16 bits (a few hundred per expert on C5-like
// data), and the final select takes bits 13-7 and 6-0 from those lists, then
// applies the EMA.  No pass uses a global atomic: a block counts in LDS and
// writes its histogram whole, a collect block appends to its own segment of
// the expert's list (an LDS counter per expert gives the index), and only the
// segments' contents, not their order, enter the result, so it is
// deterministic.
//   key pass: reads the logits, computes every key once, stores its top 16
//     bits (bits 29-14, as uint16) and counts bits 29-22.
//   prefix pass: reads the 16-bit keys and counts bits 21-14 of those whose
//     bits 29-22 match.
//   collect pass: reads the logits again.  The 16 fixed bits bound the key to
//     [K, K + 2^14), i.e. the score to [u2f(K), u2f(K + 2^14)); select_bounds
//     turns the two ends into logit bounds, so only logits near that range
//     (or NaN) have their exact key evaluated, and those whose top 16 bits
//     match are listed.
//   Histogram blocks: grid (token blocks, 64-expert groups), 16 waves per
//     block, lane = expert (coalesced row segments).  Counts are 16-bit in LDS,
//     two digits to a word, written whole to partial[group][block][lane][d / 2].
//   Select blocks (one per expert) sum the partial histograms and find the
//   digit that holds the rank-th largest matching key.
#include <algorithm>
#include <mutex>

#include "et_common.hpp"
#include "et_route_internal.hpp"

namespace et {

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

constexpr int kHistWaves = 16;
constexpr int kHistThreads = kHistWaves * kWave;
constexpr int64_t kHistBlocks = 256;        // blocks of a pass (whole grid)
constexpr int kHistUTLogits = 8;            // tokens in flight per wave, passes over the logits
constexpr int kHistUTKeys = 16;             // tokens in flight per wave, the prefix pass
constexpr int64_t kMaxTokensPerBlock = 65535;  // LDS counts are 16-bit
constexpr int kPitch = kWave + 1;           // LDS words per digit pair (padded)
constexpr int kHistWords = kWave * 128;     // words of one block histogram (two 16-bit counts each)
constexpr int kSelectThreads = 1024;
constexpr int kSelectSplit = kSelectThreads / 128;
constexpr int kSelectRound = 8;             // partial-histogram loads in flight per select thread
constexpr int kShift1 = 22;                 // the key pass's digit: bits 29-22
constexpr int kShift2 = 14;                 // the prefix pass's digit: bits 21-14

// Token blocks per 64-expert group of a pass.
struct HistGrid {
    int64_t blocks;  // token blocks per group
    int64_t tpb;     // tokens per block
};

static HistGrid hist_grid(int64_t T, int64_t E, int ut)
{
    const int64_t groups = (E + kWave - 1) / kWave;
    HistGrid g;
    int64_t b = std::max<int64_t>(1, kHistBlocks / groups);
    b = std::max<int64_t>(b, (T + kMaxTokensPerBlock - 1) / kMaxTokensPerBlock);
    g.tpb = std::max<int64_t>(1, (T + b - 1) / b);
    g.tpb = std::max<int64_t>(g.tpb, (int64_t)kHistWaves * ut);
    g.tpb = std::min<int64_t>(g.tpb, kMaxTokensPerBlock);
    g.blocks = std::max<int64_t>(1, (T + g.tpb - 1) / g.tpb);
    return g;
}

struct ThrWs {
    uint32_t* prefix;   // [E]  bits of the selected key fixed so far
    uint32_t* rank;     // [E]  rank still to find among keys matching prefix
    float* bnd;         // [2 E] logit bounds of the collect pass: (lo, hi) per expert
    uint16_t* k16;      // [T * E] bits 29-14 of every key
    uint32_t* partial;  // [groups][blocks][64][128] block histograms of one pass (16-bit counts, packed)
    uint32_t* cand;     // [E][T] keys matching the 16-bit prefix; block b's at [b * tpb, ...)
    uint32_t* cand_n;   // [E][blocks] candidates of each collect block
    HistGrid g1, g2;    // grids of the passes over the logits and of the prefix pass
    size_t bytes;
};

static ThrWs thr_ws_layout(void* base, int64_t T, int64_t E)
{
    ThrWs ws{};
    ws.g1 = hist_grid(T, E, kHistUTLogits);
    ws.g2 = hist_grid(T, E, kHistUTKeys);
    const int64_t groups = (E + kWave - 1) / kWave;
    const int64_t nb = std::max(ws.g1.blocks, ws.g2.blocks);
    size_t off = 0;
    char* b = static_cast<char*>(base);
    ws.prefix = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.rank = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.bnd = reinterpret_cast<float*>(b + off); off += align256(size_t(E) * 8);
    ws.k16 = reinterpret_cast<uint16_t*>(b + off); off += align256(size_t(T * E) * 2);
    ws.partial = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(groups * nb) * kHistWords * 4);
    ws.cand = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(T * E) * 4);
    ws.cand_n = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E * ws.g1.blocks) * 4);
    ws.bytes = off;
    return ws;
}

// The key of a logit: the bits of its score, NaN as 0 (below 2^30).
__device__ __forceinline__ uint32_t score_key(float l)
{
    const float sc = sigmoid(l);
    return (sc != sc) ? 0u : f2u(sc);
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
        const int l = i >> 7, j = i & 127;
        out[i] = h[j * kPitch + l];
    }
}

// Key pass: every key of the block's tokens; its top 16 bits to k16, bits
// 29-22 counted.  Each wave takes UT consecutive tokens at a time with all
// UT loads issued before the first use (addresses clamped into the matrix).
template <int UT>
__global__ __launch_bounds__(kHistThreads) void thr_key_kernel(const float* __restrict__ logits,
                                                               uint16_t* __restrict__ k16, int T, int E, int tpb,
                                                               uint32_t* __restrict__ partial)
{
    __shared__ uint32_t h[128 * kPitch];
    const int tid = threadIdx.x;
    for (int i = tid; i < 128 * kPitch; i += kHistThreads) h[i] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = blockIdx.y * kWave + lane;
    const bool ve = e < E;
    const int ec = min(e, E - 1);
    const int64_t t0 = (int64_t)blockIdx.x * tpb;
    const int64_t t1 = min((int64_t)T, t0 + tpb);
    for (int64_t tb = t0 + (int64_t)wave * UT; tb < t1; tb += (int64_t)kHistWaves * UT) {
        float v[UT];
#pragma unroll
        for (int u = 0; u < UT; ++u) v[u] = logits[min(tb + u, t1 - 1) * E + ec];
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            const int64_t t = tb + u;
            if (!ve || t >= t1) continue;
            const uint32_t key = score_key(v[u]);
            k16[t * E + e] = (uint16_t)(key >> kShift2);
            hist_add(h, key >> kShift1, lane);
        }
    }
    __syncthreads();
    hist_flush(h, partial);
}

// Prefix pass: bits 21-14 of the keys whose bits 29-22 match prefix[e].
template <int UT>
__global__ __launch_bounds__(kHistThreads) void thr_prefix_kernel(const uint16_t* __restrict__ k16, int T, int E,
                                                                  int tpb, const uint32_t* __restrict__ prefix,
                                                                  uint32_t* __restrict__ partial)
{
    __shared__ uint32_t h[128 * kPitch];
    const int tid = threadIdx.x;
    for (int i = tid; i < 128 * kPitch; i += kHistThreads) h[i] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = blockIdx.y * kWave + lane;
    const bool ve = e < E;
    const int ec = min(e, E - 1);
    const uint32_t pre = prefix[ec] >> kShift1;   // bits 29-22
    const int64_t t0 = (int64_t)blockIdx.x * tpb;
    const int64_t t1 = min((int64_t)T, t0 + tpb);
    for (int64_t tb = t0 + (int64_t)wave * UT; tb < t1; tb += (int64_t)kHistWaves * UT) {
        uint32_t v[UT];
#pragma unroll
        for (int u = 0; u < UT; ++u) v[u] = k16[min(tb + u, t1 - 1) * E + ec];
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            if (!ve || tb + u >= t1) continue;
            if ((v[u] >> 8) == pre) hist_add(h, v[u] & 255u, lane);
        }
    }
    __syncthreads();
    hist_flush(h, partial);
}

// Collect pass: the keys whose bits 29-14 match prefix[e], into the block's
// segment of the expert's list, cand[e][t0 + i] (i from an LDS counter, so
// i < t1 - t0); the block's count goes to cand_n[e][block].  A logit at or
// below bnd[2e] has a key below the range, one at or above bnd[2e + 1] a key
// above it; only the others (and NaN) have their key evaluated.
template <int UT>
__global__ __launch_bounds__(kHistThreads) void thr_collect_kernel(
    const float* __restrict__ logits, int T, int E, int tpb, const uint32_t* __restrict__ prefix,
    const float* __restrict__ bnd, uint32_t* __restrict__ cand, uint32_t* __restrict__ cand_n)
{
    __shared__ uint32_t cn[kWave];
    const int tid = threadIdx.x;
    if (tid < kWave) cn[tid] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = blockIdx.y * kWave + lane;
    const bool ve = e < E;
    const int ec = min(e, E - 1);
    const uint32_t pre = prefix[ec] >> kShift2;   // bits 29-14
    const float lo = bnd[2 * ec], hi = bnd[2 * ec + 1];
    const int64_t t0 = (int64_t)blockIdx.x * tpb;
    const int64_t t1 = min((int64_t)T, t0 + tpb);
    for (int64_t tb = t0 + (int64_t)wave * UT; tb < t1; tb += (int64_t)kHistWaves * UT) {
        float v[UT];
#pragma unroll
        for (int u = 0; u < UT; ++u) v[u] = logits[min(tb + u, t1 - 1) * E + ec];
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            const int64_t t = tb + u;
            if (!ve || t >= t1 || v[u] <= lo || v[u] >= hi) continue;
            const uint32_t key = score_key(v[u]);
            if ((key >> kShift2) == pre) {
                const uint32_t i = atomicAdd(&cn[lane], 1u);
                cand[(int64_t)e * T + t0 + i] = key;
            }
        }
    }
    __syncthreads();
    if (tid < kWave && ve) cand_n[(int64_t)e * gridDim.x + blockIdx.x] = cn[tid];
}

// Wave 0 of a select block: the bin of the rank-th largest key (rank r >= 1)
// given NB bin counts cnt(bin) (NB = 256 or 128), bins walked from the top.
// The lane that holds it returns true with the bin and the rank left inside
// the bin.
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

// One block per expert: counts[d] = the sum of the expert's block histograms
// (kSelectSplit threads per word of two digits, each over every
// kSelectSplit-th block, all loads of a round issued together; the two 16-bit
// halves are added separately), then wave 0 finds the digit that holds the
// rank-th largest matching key.  FIRST (bits 29-22): from the empty prefix and
// rank c0.  Otherwise (bits 21-14) the 16 fixed bits also give the collect
// pass its logit bounds.
template <bool FIRST>
__global__ __launch_bounds__(kSelectThreads) void thr_select_kernel(int E, int nblocks,
                                                                    const uint32_t* __restrict__ partial,
                                                                    uint32_t* __restrict__ prefix,
                                                                    uint32_t* __restrict__ rank, uint32_t c0,
                                                                    float* __restrict__ bnd)
{
    __shared__ uint32_t part[kSelectSplit][256];
    const int e = blockIdx.x;
    const int tid = threadIdx.x;
    const int q = tid >> 7, j = tid & 127;
    const uint32_t* src = partial + (int64_t)(e >> 6) * nblocks * kHistWords + (e & 63) * 128 + j;
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
    auto pass_count = [&](int bin) {
        uint32_t c = 0u;
#pragma unroll
        for (int k = 0; k < kSelectSplit; ++k) c += part[k][bin];
        return c;
    };
    uint32_t bin;
    int rin;
    if (find_digit<256>(pass_count, FIRST ? (int)c0 : (int)rank[e], bin, rin)) {
        if (FIRST) {
            prefix[e] = bin << kShift1;
        } else {
            const uint32_t p = prefix[e] | (bin << kShift2);
            prefix[e] = p;
            // keys in [p, p + 2^14): a logit at or below lo_a scores below
            // u2f(p), one at or above hi_b at or above u2f(p + 2^14)
            float hi_a, lo_a, hi_b, lo_b;
            select_bounds(u2f(p), hi_a, lo_a);
            select_bounds(u2f(p + (1u << kShift2)), hi_b, lo_b);
            // (a NaN bound decides nothing: comparisons with it are false)
            bnd[2 * e] = lo_a;
            bnd[2 * e + 1] = hi_b;
        }
        rank[e] = (uint32_t)rin;
    }
}

// Final select, one block per expert: bits 13-7, then bits 6-0, of the rank-th
// largest listed key, each from an LDS histogram over the expert's candidate
// segments; then the EMA (with thr) or the statistic left in prefix with rank
// 0 marking it found (without).  The segments are taken up to kSelectThreads
// blocks at a time: a block-wide scan of their counts places them, and thread
// i of a round finds its segment by binary search.
__global__ __launch_bounds__(kSelectThreads) void thr_final_kernel(
    int E, int nblocks, int T, int tpb, uint32_t* __restrict__ prefix, uint32_t* __restrict__ rank,
    const uint32_t* __restrict__ cand, const uint32_t* __restrict__ cand_n, float* __restrict__ thr,
    float* __restrict__ stat, float m)
{
    __shared__ uint32_t hist[128];
    __shared__ uint32_t seg_end[kSelectThreads];  // inclusive scan of a round's segment counts
    __shared__ uint32_t wsum[kSelectThreads / kWave];
    __shared__ uint32_t sel[2];                  // the bits fixed so far and the rank inside them
    const int e = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    if (tid == 0) {
        sel[0] = prefix[e];
        sel[1] = rank[e];
    }
    const uint32_t* cl = cand + (int64_t)e * T;
    const uint32_t* cnt = cand_n + (int64_t)e * nblocks;
    for (int step = 0; step < 2; ++step) {
        const int shift = step == 0 ? 7 : 0;
        if (tid < 128) hist[tid] = 0u;
        __syncthreads();
        const uint32_t fixed = sel[0];
        const uint32_t mask = step == 0 ? 0xffffc000u : 0xffffff80u;
        for (int b0 = 0; b0 < nblocks; b0 += kSelectThreads) {
            const int nc = min(kSelectThreads, nblocks - b0);
            const uint32_t n = tid < nc ? cnt[b0 + tid] : 0u;
            const uint32_t incl = (uint32_t)wave_incl_scan((int)n);
            if (lane_id() == kWave - 1) wsum[wave] = incl;
            __syncthreads();
            uint32_t below = 0u;
            for (int w = 0; w < wave; ++w) below += wsum[w];
            seg_end[tid] = below + incl;
            __syncthreads();
            const uint32_t total = seg_end[nc - 1];
            for (uint32_t i = tid; i < total; i += kSelectThreads) {
                int lo = 0, hi = nc - 1;                 // the first segment that ends past i
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (seg_end[mid] > i) hi = mid; else lo = mid + 1;
                }
                const uint32_t start = lo ? seg_end[lo - 1] : 0u;
                const uint32_t key = cl[(int64_t)(b0 + lo) * tpb + (i - start)];
                if ((key & mask) == fixed) atomicAdd(&hist[(key >> shift) & 127u], 1u);
            }
            __syncthreads();
        }
        if (tid < kWave) {
            uint32_t bin;
            int rin;
            if (find_digit<128>([&](int b) { return hist[b]; }, (int)sel[1], bin, rin)) {
                sel[0] = fixed | (bin << shift);
                sel[1] = (uint32_t)rin;
            }
        }
        __syncthreads();
    }
    if (tid != 0) return;
    // every bit is fixed: sel[0] is the statistic (rank 0 marks it found)
    const uint32_t p = sel[0];
    prefix[e] = p;
    rank[e] = 0u;
    if (thr) {
        const float st = u2f(p);
        if (stat) stat[e] = st;
        const float one_minus_m = 1.0f - m;
        thr[e] = __builtin_fmaf(m, thr[e], one_minus_m * st);
    }
}

// The EMA of the statistics a stat-only run left in prefix (where rank is 0),
// with the final select's arithmetic.
__global__ __launch_bounds__(256) void thr_apply_kernel(int E, const uint32_t* __restrict__ prefix,
                                                        const uint32_t* __restrict__ rank, float* __restrict__ thr,
                                                        float* __restrict__ stat, float m)
{
    const int e = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (e >= E || rank[e] != 0u) return;
    const float st = u2f(prefix[e]);
    if (stat) stat[e] = st;
    const float one_minus_m = 1.0f - m;
    thr[e] = __builtin_fmaf(m, thr[e], one_minus_m * st);
}

// The passes on stream s.  With thr, the final select also applies the EMA
// (and writes stat); without, the statistics stay in ws.prefix for
// thr_apply_kernel.
static int thr_passes(const float* logits, int64_t T, int64_t E, int64_t k_target, float* thr, float* stat,
                      float momentum, const ThrWs& ws, hipStream_t s)
{
    int64_t c = (T * k_target + E - 1) / E;
    if (c < 1) c = 1;
    if (c > T) c = T;
    const int Ti = (int)T, Ei = (int)E;
    const unsigned groups = (unsigned)((E + kWave - 1) / kWave);
    const dim3 grid1((unsigned)ws.g1.blocks, groups), grid2((unsigned)ws.g2.blocks, groups);
    thr_key_kernel<kHistUTLogits><<<grid1, dim3(kHistThreads), 0, s>>>(logits, ws.k16, Ti, Ei, (int)ws.g1.tpb,
                                                                        ws.partial);
    if (int rc = check_launch("thr_key_kernel")) return rc;
    thr_select_kernel<true><<<dim3(Ei), dim3(kSelectThreads), 0, s>>>(Ei, (int)ws.g1.blocks, ws.partial, ws.prefix,
                                                                       ws.rank, (uint32_t)c, ws.bnd);
    if (int rc = check_launch("thr_select_kernel")) return rc;
    thr_prefix_kernel<kHistUTKeys><<<grid2, dim3(kHistThreads), 0, s>>>(ws.k16, Ti, Ei, (int)ws.g2.tpb, ws.prefix,
                                                                         ws.partial);
    if (int rc = check_launch("thr_prefix_kernel")) return rc;
    thr_select_kernel<false><<<dim3(Ei), dim3(kSelectThreads), 0, s>>>(Ei, (int)ws.g2.blocks, ws.partial,
                                                                        ws.prefix, ws.rank, 0u, ws.bnd);
    if (int rc = check_launch("thr_select_kernel")) return rc;
    thr_collect_kernel<kHistUTLogits><<<grid1, dim3(kHistThreads), 0, s>>>(logits, Ti, Ei, (int)ws.g1.tpb, ws.prefix,
                                                                            ws.bnd, ws.cand, ws.cand_n);
    if (int rc = check_launch("thr_collect_kernel")) return rc;
    thr_final_kernel<<<dim3(Ei), dim3(kSelectThreads), 0, s>>>(Ei, (int)ws.g1.blocks, Ti, (int)ws.g1.tpb, ws.prefix,
                                                                ws.rank, ws.cand, ws.cand_n, thr, stat, momentum);
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

// The library's second stream on each device (default priority), with the
// two events that fork work onto it and join it back; created on first use.
// Used only while the caller's stream is being captured into a HIP graph and
// the side stream is not part of another capture.
struct SideStream {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kSideDevices = 64;
static std::mutex g_side_mu;
static SideStream g_side[kSideDevices];

static int side_stream(const char* fn, SideStream** out)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(ET_ERR_LAUNCH, std::string(fn) + ": hipGetDevice: " + hipGetErrorString(e));
    if (dev < 0 || dev >= kSideDevices)
        return fail(ET_ERR_UNSUPPORTED, std::string(fn) + ": device index " + std::to_string(dev) + " beyond " +
                                            std::to_string(kSideDevices));
    SideStream& ss = g_side[dev];
    if (!ss.s) {
        hipStream_t s = nullptr;
        hipEvent_t f = nullptr, j = nullptr;
        e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&f, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&j, hipEventDisableTiming);
        if (e != hipSuccess)
            return fail(ET_ERR_LAUNCH, std::string(fn) + ": creating the side stream: " + hipGetErrorString(e));
        ss.s = s;
        ss.fork = f;
        ss.join = j;
    }
    *out = &ss;
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
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto route = [&](void) {
        return et_route(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                        token_slot, slot_capacity, route_workspace, route_workspace_bytes, stream);
    };
    if (T == 0) return route();
    const ThrWs ws = thr_ws_layout(thr_workspace, T, E);

    // Issued eagerly, or while the side stream is busy with another capture:
    // the routing, then the update applying the EMA in its final select (the
    // routing has read thr by then), all on `stream`.
    // (the legacy default stream is never captured)
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = s ? hipStreamIsCapturing(s, &cap) : hipSuccess;
    if (e != hipSuccess) return fail(ET_ERR_LAUNCH, std::string("et_route_update: hipStreamIsCapturing: ") + hipGetErrorString(e));
    std::unique_lock<std::mutex> lock(g_side_mu);
    SideStream* ss = nullptr;
    bool fork = false;
    if (cap == hipStreamCaptureStatusActive) {
        if (int rc = side_stream(fn, &ss)) return rc;
        hipStreamCaptureStatus side_cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(ss->s, &side_cap);
        if (e != hipSuccess) return fail(ET_ERR_LAUNCH, std::string("et_route_update: hipStreamIsCapturing: ") + hipGetErrorString(e));
        fork = side_cap == hipStreamCaptureStatusNone;
    }
    if (!fork) {
        lock.unlock();
        if (int rc = route()) return rc;
        return thr_passes(logits, T, E, k_target, thr, stat, momentum, ws, s);
    }
    // Under capture: the statistic reads only the logits, so its passes run on
    // the side stream beside the routing (a parallel branch of the graph);
    // `stream` then joins it and applies the EMA after the routing read thr.
    e = hipEventRecord(ss->fork, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(ss->s, ss->fork, 0);
    if (e != hipSuccess) return fail(ET_ERR_LAUNCH, std::string("et_route_update: fork: ") + hipGetErrorString(e));
    const int rc_stat = thr_passes(logits, T, E, k_target, nullptr, nullptr, momentum, ws, ss->s);
    const int rc_route = rc_stat ? ET_OK : route();
    // join (also after a failed launch, so the side stream is never left
    // forked from a capture), then the EMA write, after the routing read thr
    e = hipEventRecord(ss->join, ss->s);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, ss->join, 0);
    if (e != hipSuccess) return fail(ET_ERR_LAUNCH, std::string("et_route_update: join: ") + hipGetErrorString(e));
    if (rc_stat) return rc_stat;
    if (rc_route) return rc_route;
    thr_apply_kernel<<<dim3((unsigned)((E + 255) / 256)), dim3(256), 0, s>>>((int)E, ws.prefix, ws.rank, thr, stat,
                                                                             momentum);
    return check_launch("thr_apply_kernel");
}
