// et_threshold.hip -- EMA update of the per-expert routing thresholds, for
// gfx950: the exact c-th largest sigmoid score of every expert's column by an
// 8-bit MSB-first radix select over the score bits, then
// thr[e] = fma(momentum, thr[e], (1 - momentum) * stat[e]).
#include <algorithm>

#include "et_common.hpp"

namespace et {

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

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

}  // namespace et

using namespace et;

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
