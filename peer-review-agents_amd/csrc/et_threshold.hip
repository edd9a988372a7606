// et_threshold.hip -- EMA update of the per-expert routing thresholds, for
// gfx950: the exact c-th largest sigmoid score of every expert's column by an
// 8-bit MSB-first radix select over the score bits, then
// thr[e] = fma(momentum, thr[e], (1 - momentum) * stat[e]).
//
// Three histogram passes and three select launches fix the top three 8-bit
// digits; the third pass also copies out the keys that still match after two
// digits (a few hundred per expert on C5-like data), and the last select
// takes the fourth digit from those candidate lists in LDS, then applies the
// EMA.  No pass uses a global atomic: a histogram block appends its
// candidates to its own segment of the expert's list (an LDS counter per
// expert gives the index), and only the segments' contents, not their order,
// enter the result, so it is deterministic.
//   histogram: grid (token blocks, 64-expert groups), 16 waves per block,
//     lane = expert (coalesced 256-byte row segments).  The first pass reads
//     the logits, computes every score key once and stores the keys; the later
//     passes read the keys.  A block counts the digits of the keys that match
//     the prefix fixed so far in an LDS histogram of 16-bit counts and writes
//     it whole, two counts per word, to partial[group][block][lane][digit / 2]
//     (digit d in the half d % 2).
//   select: one block per expert sums the expert's partial histograms, finds
//     the digit that holds the rank-th largest matching key, and narrows the
//     prefix and the rank for the next pass; the last one then histograms the
//     expert's candidates by their lowest byte and fixes the statistic.
#include <algorithm>
#include <mutex>

#include "et_common.hpp"
#include "et_route_internal.hpp"

namespace et {

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

constexpr int kHistWaves = 16;
constexpr int kHistThreads = kHistWaves * kWave;
constexpr int64_t kHistBlocksFirst = 256;   // blocks of the score pass (whole grid)
constexpr int kHistUTFirst = 8;             // tokens in flight per wave, score pass
constexpr int64_t kHistBlocksKeys = 256;    // blocks of the key passes (whole grid)
constexpr int kHistUTKeys = 16;             // tokens in flight per wave, key passes
constexpr int64_t kMaxTokensPerBlock = 65535;  // LDS counts are 16-bit
constexpr int kPitch = kWave + 1;           // LDS words per digit pair (padded)
constexpr int kHistWords = kWave * 128;     // words of one block histogram (two 16-bit counts each)
constexpr int kSelectThreads = 1024;
constexpr int kSelectSplit = kSelectThreads / 128;
constexpr int kSelectRound = 8;             // partial-histogram loads in flight per select thread

// Token blocks per 64-expert group of a histogram pass.
struct HistGrid {
    int64_t blocks;  // token blocks per group
    int64_t tpb;     // tokens per block
};

static HistGrid hist_grid(int64_t T, int64_t E, int64_t target_blocks, int ut)
{
    const int64_t groups = (E + kWave - 1) / kWave;
    HistGrid g;
    int64_t b = std::max<int64_t>(1, target_blocks / groups);
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
    uint32_t* keys;     // [T * E] score keys (bit patterns of the scores; NaN -> 0)
    uint32_t* partial;  // [groups][blocks][64][128] block histograms of one pass (16-bit counts, packed)
    uint32_t* cand;     // [E][T] keys matching the two-digit prefix; block b's at [b * tpb, ...)
    uint32_t* cand_n;   // [E][blocks] candidates of each block of the third pass
    HistGrid g1, g2;    // grids of the score pass and of the key passes
    size_t bytes;
};

static ThrWs thr_ws_layout(void* base, int64_t T, int64_t E)
{
    ThrWs ws{};
    ws.g1 = hist_grid(T, E, kHistBlocksFirst, kHistUTFirst);
    ws.g2 = hist_grid(T, E, kHistBlocksKeys, kHistUTKeys);
    const int64_t groups = (E + kWave - 1) / kWave;
    const int64_t nb = std::max(ws.g1.blocks, ws.g2.blocks);
    size_t off = 0;
    char* b = static_cast<char*>(base);
    ws.prefix = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.rank = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.keys = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(T * E) * 4);
    ws.partial = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(groups * nb) * kHistWords * 4);
    ws.cand = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(T * E) * 4);
    ws.cand_n = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E * ws.g2.blocks) * 4);
    ws.bytes = off;
    return ws;
}

// One digit-histogram pass.  Each wave takes UT consecutive tokens at a time,
// with all UT loads issued before the first use (addresses clamped into the
// matrix).  FIRST: the input is the logits and the key of every score is
// stored; otherwise the input is the stored keys.  LDS counts are 16-bit, two
// digits to a word (word (d >> 1) * kPitch + lane, half d & 1); a block covers
// at most 65535 tokens, so a half never carries into its neighbour.
// COMPACT (the third pass): every key that matches the two-digit prefix is
// also stored in the block's segment of its expert's candidate list,
// cand[e][t0 + i] for the block's tokens [t0, t1) (i from an LDS counter, so
// i < t1 - t0), and the block's count goes to cand_n[e][block].
template <bool FIRST, bool COMPACT, int UT>
__global__ __launch_bounds__(kHistThreads) void thr_hist_kernel(
    const float* __restrict__ logits, uint32_t* __restrict__ keys, int T, int E, int shift,
    int tokens_per_block, const uint32_t* __restrict__ prefix, uint32_t* __restrict__ partial,
    uint32_t* __restrict__ cand, uint32_t* __restrict__ cand_n)
{
    __shared__ uint32_t h[128 * kPitch];
    __shared__ uint32_t cn[kWave];
    const int tid = threadIdx.x;
    for (int i = tid; i < 128 * kPitch; i += kHistThreads) h[i] = 0u;
    if (COMPACT && tid < kWave) cn[tid] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = blockIdx.y * kWave + lane;
    const bool ve = e < E;
    const int ec = min(e, E - 1);
    const uint32_t hmask = (shift == 24) ? 0u : (0xffffffffu << (shift + 8));
    const uint32_t pre = (shift == 24) ? 0u : (prefix[ec] & hmask);
    const int64_t t0 = (int64_t)blockIdx.x * tokens_per_block;
    const int64_t t1 = min((int64_t)T, t0 + tokens_per_block);
    for (int64_t tb = t0 + (int64_t)wave * UT; tb < t1; tb += (int64_t)kHistWaves * UT) {
        uint32_t v[UT];
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            const int64_t tc = min(tb + u, t1 - 1);
            v[u] = FIRST ? f2u(logits[tc * E + ec]) : keys[tc * E + ec];
        }
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            const int64_t t = tb + u;
            if (!ve || t >= t1) continue;
            uint32_t key = v[u];
            if (FIRST) {
                const float sc = sigmoid(u2f(key));
                key = (sc != sc) ? 0u : f2u(sc);
                keys[t * E + e] = key;
            }
            if ((key & hmask) == pre) {
                const uint32_t d = (key >> shift) & 255u;
                atomicAdd(&h[(d >> 1) * kPitch + lane], 1u << ((d & 1u) * 16));
                if (COMPACT) {
                    const uint32_t i = atomicAdd(&cn[lane], 1u);
                    cand[(int64_t)e * T + t0 + i] = key;
                }
            }
        }
    }
    __syncthreads();
    uint32_t* out = partial + ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kHistWords;
    for (int i = tid; i < kHistWords; i += kHistThreads) {
        const int l = i >> 7, j = i & 127;
        out[i] = h[j * kPitch + l];
    }
    if (COMPACT && tid < kWave && ve) cand_n[(int64_t)e * gridDim.x + blockIdx.x] = cn[tid];
}

// Wave 0 of a select block: the bin of the rank-th largest key (rank r >= 1)
// given the bin counts cnt(bin), bins walked from the top.  The lane that
// holds it returns true with the bin and the rank left inside the bin.
template <typename F>
__device__ __forceinline__ bool find_digit(F cnt, int r, uint32_t& bin, int& rank_in)
{
    const int lane = lane_id();
    // position p = 4*lane + i walks the bins from the top: bin = 255 - p
    uint32_t c[4];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c[i] = cnt(255 - (4 * lane + i));
        tot += (int)c[i];
    }
    const int incl = wave_incl_scan(tot);
    const int excl = incl - tot;
    if (!(excl < r && r <= incl)) return false;
    int run = excl;
    int pos = 4 * lane + 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (run + (int)c[i] >= r) { pos = 4 * lane + i; break; }
        run += (int)c[i];
    }
    bin = 255u - (uint32_t)pos;
    rank_in = r - run;
    return true;
}

// One block per expert: counts[d] = the sum of the expert's block histograms
// (kSelectSplit threads per word of two digits, each over every
// kSelectSplit-th block, all loads of a round issued together; the two 16-bit
// halves are added separately), then wave 0 finds the digit that holds the
// rank-th largest matching key.  FINAL (the third select, shift 8): the digit
// found fixes 24 bits; the block then counts the lowest byte of the expert's
// candidates that match them (LDS histogram), wave 0 finds the last digit,
// and the statistic goes into the EMA.  The candidate segments are taken up
// to kSelectThreads blocks at a time: a block-wide scan of their counts
// places them, and thread i of a round finds its segment by binary search.
template <bool FINAL>
__global__ __launch_bounds__(kSelectThreads) void thr_select_kernel(
    int E, int shift, int nblocks, const uint32_t* __restrict__ partial, uint32_t* __restrict__ prefix,
    uint32_t* __restrict__ rank, uint32_t c0, float* __restrict__ thr, float* __restrict__ stat, float m,
    const uint32_t* __restrict__ cand, const uint32_t* __restrict__ cand_n, int T, int tpb)
{
    __shared__ uint32_t part[kSelectSplit][256];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t seg_end[kSelectThreads];  // FINAL: inclusive scan of a round's segment counts
    __shared__ uint32_t wsum[kSelectThreads / kWave];
    __shared__ uint32_t sel[2];                  // FINAL: the 24-bit prefix and the rank inside it
    const int e = blockIdx.x;
    const int tid = threadIdx.x;
    if (FINAL) {
        if (tid < 256) hist[tid] = 0u;
        if (tid == 0) { sel[0] = 0xffffffffu; sel[1] = 0u; }
    }
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
    auto pass_count = [&](int bin) {
        uint32_t c = 0u;
#pragma unroll
        for (int k = 0; k < kSelectSplit; ++k) c += part[k][bin];
        return c;
    };
    if (!FINAL) {
        if (tid >= kWave) return;
        // the first pass starts from the empty prefix and rank c0
        const bool first = shift == 24;
        uint32_t bin;
        int rin;
        if (find_digit(pass_count, first ? (int)c0 : (int)rank[e], bin, rin)) {
            prefix[e] = (first ? 0u : prefix[e]) | (bin << shift);
            rank[e] = (uint32_t)rin;
        }
        return;
    }
    if (tid < kWave) {
        uint32_t bin;
        int rin;
        if (find_digit(pass_count, (int)rank[e], bin, rin)) {
            sel[0] = prefix[e] | (bin << 8);
            sel[1] = (uint32_t)rin;
        }
    }
    __syncthreads();
    const uint32_t p24 = sel[0];
    const uint32_t* cl = cand + (int64_t)e * T;
    const uint32_t* cnt = cand_n + (int64_t)e * nblocks;
    const int wave = tid >> 6;
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
            if ((key & 0xffffff00u) == p24) atomicAdd(&hist[key & 255u], 1u);
        }
        __syncthreads();
    }
    if (tid >= kWave) return;
    uint32_t bin;
    int rin;
    if (find_digit([&](int b) { return hist[b]; }, (int)sel[1], bin, rin)) {
        // every bit is fixed: p is the statistic (rank 0 marks it found)
        const uint32_t p = p24 | bin;
        prefix[e] = p;
        rank[e] = 0u;
        if (thr) {
            const float st = u2f(p);
            if (stat) stat[e] = st;
            const float one_minus_m = 1.0f - m;
            thr[e] = __builtin_fmaf(m, thr[e], one_minus_m * st);
        }
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

// The radix-select passes on stream s.  With thr, the last select also
// applies the EMA (and writes stat); without, the statistics stay in
// ws.prefix for thr_apply_kernel.
static int thr_passes(const float* logits, int64_t T, int64_t E, int64_t k_target, float* thr, float* stat,
                      float momentum, const ThrWs& ws, hipStream_t s)
{
    int64_t c = (T * k_target + E - 1) / E;
    if (c < 1) c = 1;
    if (c > T) c = T;
    const int Ti = (int)T, Ei = (int)E;
    const unsigned groups = (unsigned)((E + kWave - 1) / kWave);
    for (int pass = 0; pass < 3; ++pass) {
        const int shift = 24 - 8 * pass;
        const HistGrid& g = pass == 0 ? ws.g1 : ws.g2;
        const dim3 grid((unsigned)g.blocks, groups);
        if (pass == 0)
            thr_hist_kernel<true, false, kHistUTFirst><<<grid, dim3(kHistThreads), 0, s>>>(
                logits, ws.keys, Ti, Ei, shift, (int)g.tpb, ws.prefix, ws.partial, ws.cand, ws.cand_n);
        else if (pass == 1)
            thr_hist_kernel<false, false, kHistUTKeys><<<grid, dim3(kHistThreads), 0, s>>>(
                logits, ws.keys, Ti, Ei, shift, (int)g.tpb, ws.prefix, ws.partial, ws.cand, ws.cand_n);
        else
            thr_hist_kernel<false, true, kHistUTKeys><<<grid, dim3(kHistThreads), 0, s>>>(
                logits, ws.keys, Ti, Ei, shift, (int)g.tpb, ws.prefix, ws.partial, ws.cand, ws.cand_n);
        if (int rc = check_launch("thr_hist_kernel")) return rc;
        if (pass < 2)
            thr_select_kernel<false><<<dim3(Ei), dim3(kSelectThreads), 0, s>>>(
                Ei, shift, (int)g.blocks, ws.partial, ws.prefix, ws.rank, (uint32_t)c, thr, stat, momentum, ws.cand,
                ws.cand_n, Ti, (int)ws.g2.tpb);
        else
            thr_select_kernel<true><<<dim3(Ei), dim3(kSelectThreads), 0, s>>>(
                Ei, shift, (int)g.blocks, ws.partial, ws.prefix, ws.rank, (uint32_t)c, thr, stat, momentum, ws.cand,
                ws.cand_n, Ti, (int)ws.g2.tpb);
        if (int rc = check_launch("thr_select_kernel")) return rc;
    }
    return ET_OK;
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
    if (route_workspace_bytes < et_route_workspace_bytes(T, E))
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_route_update: route workspace needs " +
                                                    std::to_string(et_route_workspace_bytes(T, E)) + " bytes, got " +
                                                    std::to_string(route_workspace_bytes));
    if (int rc = thr_check(fn, logits, thr, T, E, k_target, momentum, thr_workspace, thr_workspace_bytes)) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (T == 0)
        return et_route(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate, token_slot,
                        slot_capacity, route_workspace, route_workspace_bytes, stream);
    const ThrWs ws = thr_ws_layout(thr_workspace, T, E);
    std::lock_guard<std::mutex> lock(g_side_mu);
    SideStream* ss = nullptr;
    if (int rc = side_stream(fn, &ss)) return rc;
    // fork: the statistic reads only the logits, so it runs beside the routing
    hipError_t e = hipEventRecord(ss->fork, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(ss->s, ss->fork, 0);
    if (e != hipSuccess) return fail(ET_ERR_LAUNCH, std::string("et_route_update: fork: ") + hipGetErrorString(e));
    const int rc_stat = thr_passes(logits, T, E, k_target, nullptr, nullptr, momentum, ws, ss->s);
    const int rc_route = rc_stat ? ET_OK
                                 : et_route(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token,
                                            slot_gate, token_slot, slot_capacity, route_workspace,
                                            route_workspace_bytes, stream);
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
