// et_threshold.hip -- EMA update of the per-expert routing thresholds, for
// gfx950: the exact c-th largest sigmoid score of every expert's column by an
// 8-bit MSB-first radix select over the score bits, then
// thr[e] = fma(momentum, thr[e], (1 - momentum) * stat[e]).
//
// The first histogram pass computes every score key once (lane = expert,
// coalesced reads of the logits) and stores the keys; the three later passes
// read the keys.  Per-block histograms live in LDS laid out [digit][lane], so
// a wave's 64 updates land in distinct banks, and are added into the global
// histogram with atomics on the non-zero bins (integer counts: the result does
// not depend on their order).  Each block adds into one of kHistReplicas
// copies of the histogram (block index modulo the count), which divides the
// number of atomics that contend for one address; the select pass sums the
// copies.
#include <algorithm>

#include "et_common.hpp"

namespace et {

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// ---------------------------------------------------------------------------
// EMA threshold update: exact per-expert c-th largest score by 4 passes of an
// 8-bit MSB-first radix select on the score bits, then the EMA.
// ---------------------------------------------------------------------------

constexpr int kThrThreads = 256;
constexpr int kHistReplicas = 8;

struct ThrWs {
    uint32_t* prefix;  // [E]  bits of the selected key fixed so far
    uint32_t* rank;    // [E]  rank still to find among keys matching prefix
    uint32_t* hist;    // [kHistReplicas][E][256]
    uint32_t* keys;    // [T * E] score keys (bit patterns of the scores; NaN -> 0)
    size_t bytes;
};

static ThrWs thr_ws_layout(void* base, int64_t T, int64_t E)
{
    ThrWs ws{};
    size_t off = 0;
    char* b = static_cast<char*>(base);
    ws.prefix = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.rank = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(E) * 4);
    ws.hist = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(kHistReplicas) * E * 256 * 4);
    ws.keys = reinterpret_cast<uint32_t*>(b + off); off += align256(size_t(T * E) * 4);
    ws.bytes = off;
    return ws;
}

__global__ __launch_bounds__(kThrThreads) void thr_init_kernel(int E, uint32_t c, uint32_t* prefix,
                                                               uint32_t* rank, uint32_t* hist)
{
    const int64_t i = (int64_t)blockIdx.x * kThrThreads + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kThrThreads;
    if (i < E) { prefix[i] = 0u; rank[i] = c; }
    for (int64_t j = i; j < (int64_t)kHistReplicas * E * 256; j += stride) hist[j] = 0u;
}

// One digit-histogram pass.  Grid (token blocks, 64-expert groups), 16 waves
// per block; lane = expert.  Each wave takes UT consecutive tokens at a time,
// with all UT loads issued before the first use (addresses clamped into the
// matrix).  FIRST: the input is the logits; the key of every score is stored.
// Otherwise the input is the stored keys.
constexpr int kHistWaves = 16;
constexpr int kHistThreads = kHistWaves * kWave;
constexpr int kHistUT = 8;

template <bool FIRST>
__global__ __launch_bounds__(kHistThreads) void thr_hist_kernel(
    const float* __restrict__ logits, uint32_t* __restrict__ keys, int T, int E, int shift,
    int tokens_per_block, const uint32_t* __restrict__ prefix, uint32_t* __restrict__ hist)
{
    __shared__ uint32_t h[256 * kWave];
    const int tid = threadIdx.x;
    for (int i = tid; i < 256 * kWave; i += kHistThreads) h[i] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = tid >> 6;
    const int e = blockIdx.y * kWave + lane;
    const bool ve = e < E;
    const int ec = min(e, E - 1);
    const uint32_t hmask = (shift == 24) ? 0u : (0xffffffffu << (shift + 8));
    const uint32_t pre = prefix[ec] & hmask;
    const int64_t t0 = (int64_t)blockIdx.x * tokens_per_block;
    const int64_t t1 = min((int64_t)T, t0 + tokens_per_block);
    for (int64_t tb = t0 + (int64_t)wave * kHistUT; tb < t1; tb += (int64_t)kHistWaves * kHistUT) {
        uint32_t v[kHistUT];
#pragma unroll
        for (int u = 0; u < kHistUT; ++u) {
            const int64_t tc = min(tb + u, t1 - 1);
            v[u] = FIRST ? f2u(logits[tc * E + ec]) : keys[tc * E + ec];
        }
#pragma unroll
        for (int u = 0; u < kHistUT; ++u) {
            const int64_t t = tb + u;
            if (!ve || t >= t1) continue;
            uint32_t key = v[u];
            if (FIRST) {
                const float sc = sigmoid(u2f(key));
                key = (sc != sc) ? 0u : f2u(sc);
                keys[t * E + e] = key;
            }
            if ((key & hmask) == pre) atomicAdd(&h[((key >> shift) & 255u) * kWave + lane], 1u);
        }
    }
    __syncthreads();
    uint32_t* hr = hist + (int64_t)(blockIdx.x % kHistReplicas) * E * 256;
    for (int i = tid; i < 256 * kWave; i += kHistThreads) {
        const uint32_t v = h[i];
        const int ee = blockIdx.y * kWave + (i & (kWave - 1));
        if (v != 0u && ee < E) atomicAdd(&hr[(int64_t)ee * 256 + (i >> 6)], v);
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
    // position p = 4*lane + i walks the bins from the top: bin = 255 - p; each
    // count is the sum over the histogram copies
    uint32_t c[4];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t v[kHistReplicas];
#pragma unroll
        for (int r = 0; r < kHistReplicas; ++r) v[r] = hist[((int64_t)r * E + e) * 256 + 255 - (4 * lane + i)];
        c[i] = 0u;
#pragma unroll
        for (int r = 0; r < kHistReplicas; ++r) c[i] += v[r];
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
    for (int r = 0; r < kHistReplicas; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) hist[((int64_t)r * E + e) * 256 + 255 - (4 * lane + i)] = 0u;
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
    const ThrWs ws = thr_ws_layout(workspace, T, E);
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

    // about one 1024-thread block per CU over the whole grid
    const int egroups = (Ei + kWave - 1) / kWave;
    int64_t tblocks = std::max<int64_t>(1, 256 / egroups);
    int64_t tpb = (T + tblocks - 1) / tblocks;
    tpb = std::max<int64_t>(tpb, (int64_t)kHistWaves * kHistUT);
    tblocks = (T + tpb - 1) / tpb;
    const dim3 grid((unsigned)tblocks, egroups);
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        if (pass == 0)
            thr_hist_kernel<true><<<grid, dim3(kHistThreads), 0, s>>>(logits, ws.keys, Ti, Ei, shift, (int)tpb, ws.prefix, ws.hist);
        else
            thr_hist_kernel<false><<<grid, dim3(kHistThreads), 0, s>>>(logits, ws.keys, Ti, Ei, shift, (int)tpb, ws.prefix, ws.hist);
        if (int rc = check_launch("thr_hist_kernel")) return rc;
        thr_select_kernel<<<dim3((Ei + 3) / 4), dim3(kThrThreads), 0, s>>>(Ei, shift, ws.prefix, ws.rank, ws.hist);
        if (int rc = check_launch("thr_select_kernel")) return rc;
    }
    thr_finalize_kernel<<<dim3((Ei + kThrThreads - 1) / kThrThreads), dim3(kThrThreads), 0, s>>>(Ei, ws.prefix, thr, stat, momentum);
    return check_launch("thr_finalize_kernel");
}
