// et_route.hip -- threshold routing, histogram + exclusive-scan CSR, and the
// stable permutation indices, for gfx950.  Three launches, none with atomics,
// so the output is a deterministic function of (logits, thr).
//
// Lane = expert.  A wave walks a run of consecutive tokens in order.  For each
// token, lane l of expert group g (64 experts per group) reads
// logits[t, 64 g + l] -- one coalesced 256-byte row segment per group -- and
// computes the sigmoid score; the ballot of score >= thr is the token's
// selection mask over the group.  Per-expert counts and slot positions then
// live in the lane's registers.
//
//   1. count: per wave, the number of tokens routed to each expert and the
//      wave's slot total; the block's waves also add their rows in LDS into the
//      block's row.
//   2. scan: column-wise exclusive scan of the block rows over blocks (lane =
//      expert, 16 waves split the rows) plus a scan of the block slot totals.
//   3. fill: an exclusive scan of counts over experts gives expert_offsets.
//      A wave's first slot of expert e is expert_offsets[e] + the block's base
//      + the counts of earlier waves in the block.  The wave replays its tokens
//      and lane e writes the slot of each (t, e) at its running position, so an
//      expert's slots are in token order.  The token-major entry of (t, e) is
//      the token's offset plus the number of selected experts below e.
#include <algorithm>
#include <mutex>

#include "et_common.hpp"
#include "et_route_internal.hpp"

namespace et {

constexpr int kRouteWaves = 8;                        // waves per block, count and fill
constexpr int kRouteThreads = kRouteWaves * kWave;
constexpr int kScanWaves = 16;
constexpr int kScanThreads = kScanWaves * kWave;
constexpr int64_t kRouteTargetBlocks = 512;           // keeps the block scan short

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Work split of one routing call: tokens per wave, waves and blocks.
struct RoutePlan {
    int G;        // 64-expert groups
    int64_t tw;   // tokens per wave
    int64_t NW;   // waves (>= 1)
    int64_t NB;   // blocks
};

static RoutePlan route_plan(int64_t T, int64_t E)
{
    RoutePlan p;
    p.G = (int)((E + kWave - 1) / kWave);
    const int64_t per_block = (T + kRouteTargetBlocks - 1) / kRouteTargetBlocks;
    p.tw = std::max<int64_t>(16, (per_block + kRouteWaves - 1) / kRouteWaves);
    p.NW = std::max<int64_t>(1, (T + p.tw - 1) / p.tw);
    p.NB = (p.NW + kRouteWaves - 1) / kRouteWaves;
    return p;
}

struct RouteWs {
    int32_t* wave_counts;      // [NW * E]
    int32_t* block_counts;     // [NB * E]
    int32_t* block_base;       // [NB * E]
    int32_t* wave_slots;       // [NW]
    int32_t* block_slots;      // [NB]
    int32_t* block_slot_base;  // [NB]
    size_t bytes;
};

static RouteWs route_ws_layout(void* base, const RoutePlan& p, int64_t E)
{
    RouteWs ws{};
    size_t off = 0;
    char* b = static_cast<char*>(base);
    auto take = [&](int64_t n) {
        int32_t* q = reinterpret_cast<int32_t*>(b + off);
        off += align256(size_t(n) * 4);
        return q;
    };
    ws.wave_counts = take(p.NW * E);
    ws.block_counts = take(p.NB * E);
    ws.block_base = take(p.NB * E);
    ws.wave_slots = take(p.NW);
    ws.block_slots = take(p.NB);
    ws.block_slot_base = take(p.NB);
    ws.bytes = off;
    return ws;
}

// Logits of UT consecutive tokens starting at tb < t1 (NaN past t1 or past
// E).  Addresses are clamped into the matrix so that every load is issued
// unconditionally, all before the first use; a guarded load would complete
// before the next one issues.
template <int GM, int UT>
__device__ __forceinline__ void load_logits(const float* __restrict__ logits, int E, int G, int64_t tb,
                                            int64_t t1, float (&lg)[UT][GM])
{
    const int lane = lane_id();
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        if (g >= G) {
#pragma unroll
            for (int u = 0; u < UT; ++u) lg[u][g] = __builtin_nanf("");
            continue;
        }
        const int e = g * kWave + lane;
        const int ec = min(e, E - 1);
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            const int64_t tc = min(tb + u, t1 - 1);
            lg[u][g] = logits[tc * E + ec];
        }
#pragma unroll
        for (int u = 0; u < UT; ++u)
            if (e >= E || tb + u >= t1) lg[u][g] = __builtin_nanf("");
    }
}

template <int GM, int UT>
__global__ __launch_bounds__(kRouteThreads) void route_count_kernel(
    const float* __restrict__ logits, const float* __restrict__ thr, int T, int E, int tw, int NW,
    int32_t* __restrict__ wave_counts, int32_t* __restrict__ block_counts,
    int32_t* __restrict__ wave_slots, int32_t* __restrict__ block_slots)
{
    extern __shared__ int32_t lds[];
    int32_t* wrow = lds;                        // [kRouteWaves][E]
    int32_t* wks = lds + kRouteWaves * E;       // [kRouteWaves]
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int gw = (int)blockIdx.x * kRouteWaves + wave;
    const int G = (E + kWave - 1) / kWave;
    float th[GM];
    load_thresholds<GM>(thr, E, G, th);
    int cnt[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) cnt[g] = 0;
    int ks = 0;
    if (gw < NW) {
        const int64_t t0 = (int64_t)gw * tw;
        const int64_t t1 = std::min<int64_t>(T, t0 + tw);
        for (int64_t tb = t0; tb < t1; tb += UT) {
            float lg[UT][GM];
            load_logits<GM, UT>(logits, E, G, tb, t1, lg);
#pragma unroll
            for (int u = 0; u < UT; ++u) {
                if (tb + u >= t1) break;
                uint64_t m[GM];
                float sc[GM];
                ks += select_token<GM>(lg[u], th, G, m, sc);
#pragma unroll
                for (int g = 0; g < GM; ++g) cnt[g] += (int)((m[g] >> lane) & 1ull);
            }
        }
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            const int e = g * kWave + lane;
            if (g < G && e < E) wave_counts[(int64_t)gw * E + e] = cnt[g];
        }
        if (lane == 0) wave_slots[gw] = ks;
    }
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        if (g < G && e < E) wrow[wave * E + e] = cnt[g];
    }
    if (lane == 0) wks[wave] = ks;
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kRouteThreads) {
        int s = 0;
#pragma unroll
        for (int w = 0; w < kRouteWaves; ++w) s += wrow[w * E + e];
        block_counts[(int64_t)blockIdx.x * E + e] = s;
    }
    if (threadIdx.x == 0) {
        int s = 0;
#pragma unroll
        for (int w = 0; w < kRouteWaves; ++w) s += wks[w];
        block_slots[blockIdx.x] = s;
    }
}

// Blocks 0..G-1: exclusive scan over the NB block rows for 64 experts (lane =
// expert; wave w scans rows [w R, (w+1) R)).  Block G: exclusive scan of the
// block slot totals.
__global__ __launch_bounds__(kScanThreads) void route_scan_kernel(
    const int32_t* __restrict__ block_counts, const int32_t* __restrict__ block_slots, int NB, int E,
    int32_t* __restrict__ counts, int32_t* __restrict__ block_base, int32_t* __restrict__ block_slot_base)
{
    __shared__ int part[kScanWaves][kWave];
    __shared__ int wtot[kScanWaves];
    const int lane = lane_id();
    const int wave = (int)threadIdx.x >> 6;
    const int G = (E + kWave - 1) / kWave;
    if ((int)blockIdx.x < G) {
        const int e = (int)blockIdx.x * kWave + lane;
        const bool ve = e < E;
        const int R = (NB + kScanWaves - 1) / kScanWaves;
        const int r0 = min(NB, wave * R), r1 = min(NB, r0 + R);
        int acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0;
        const int ec = min(e, E - 1);
        for (int r = r0; r < r1; r += 8) {
            int v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = block_counts[(int64_t)min(r + i, r1 - 1) * E + ec];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] += (ve && r + i < r1) ? v[i] : 0;
        }
        int sum = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += acc[i];
        part[wave][lane] = sum;
        __syncthreads();
        int run = 0, total = 0;
        for (int i = 0; i < kScanWaves; ++i) {
            const int p = part[i][lane];
            if (i < wave) run += p;
            total += p;
        }
        if (ve) {
            for (int r = r0; r < r1; r += 8) {
                int v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = block_counts[(int64_t)min(r + i, r1 - 1) * E + e];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (r + i < r1) block_base[(int64_t)(r + i) * E + e] = run;
                    run += v[i];
                }
            }
            if (wave == 0) counts[e] = total;
        }
    } else {
        const int tid = threadIdx.x;
        const int R = (NB + kScanThreads - 1) / kScanThreads;
        const int r0 = min(NB, tid * R), r1 = min(NB, r0 + R);
        int sum = 0;
        for (int r = r0; r < r1; r += 8) {
            int v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = block_slots[min(r + i, r1 - 1)];
#pragma unroll
            for (int i = 0; i < 8; ++i) sum += (r + i < r1) ? v[i] : 0;
        }
        const int incl = wave_incl_scan(sum);
        if (lane == kWave - 1) wtot[wave] = incl;
        __syncthreads();
        int run = incl - sum;
        for (int i = 0; i < wave; ++i) run += wtot[i];
        for (int r = r0; r < r1; ++r) {
            block_slot_base[r] = run;
            run += block_slots[r];
        }
    }
}

template <int GM, int UT>
__global__ __launch_bounds__(kRouteThreads) void route_fill_kernel(
    const float* __restrict__ logits, const float* __restrict__ thr, int T, int E, int tw, int NW,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ wave_counts,
    const int32_t* __restrict__ block_base, const int32_t* __restrict__ wave_slots,
    const int32_t* __restrict__ block_slot_base, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ token_offsets, int32_t* __restrict__ sorted_token, float* __restrict__ slot_gate,
    int32_t* __restrict__ token_slot, int64_t cap)
{
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int gw = (int)blockIdx.x * kRouteWaves + wave;
    if (gw >= NW) return;
    const int G = (E + kWave - 1) / kWave;
    const int b = (int)blockIdx.x;
    const int w0 = b * kRouteWaves;

    // expert_offsets (exclusive scan of counts over experts) and the wave's
    // first slot of each of the lane's experts
    int pos[GM];
    int run = 0;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        const bool ve = g < G && e < E;
        const int c = ve ? counts[e] : 0;
        const int incl = wave_incl_scan(c);
        const int eo = run + incl - c;
        run += __builtin_amdgcn_readlane(incl, kWave - 1);
        // counts of the earlier waves of this block (all loads issued first)
        const int ec = min(e, E - 1);
        int prev[kRouteWaves - 1];
#pragma unroll
        for (int i = 0; i < kRouteWaves - 1; ++i)
            prev[i] = wave_counts[(int64_t)min(w0 + i, gw) * E + ec];
        int base = eo + block_base[(int64_t)b * E + ec];
#pragma unroll
        for (int i = 0; i < kRouteWaves - 1; ++i) base += (w0 + i < gw) ? prev[i] : 0;
        pos[g] = ve ? base : 0;
        if (ve && gw == 0) expert_offsets[e] = eo;
    }
    if (gw == 0 && lane == 0) {
        expert_offsets[E] = run;
        token_offsets[T] = run;
    }
    int tok_pos = block_slot_base[b];
    {
        int prev[kRouteWaves - 1];
#pragma unroll
        for (int i = 0; i < kRouteWaves - 1; ++i) prev[i] = wave_slots[min(w0 + i, gw)];
#pragma unroll
        for (int i = 0; i < kRouteWaves - 1; ++i) tok_pos += (w0 + i < gw) ? prev[i] : 0;
    }

    float th[GM];
    load_thresholds<GM>(thr, E, G, th);
    const int64_t t0 = (int64_t)gw * tw;
    const int64_t t1 = std::min<int64_t>(T, t0 + tw);
    for (int64_t tb = t0; tb < t1; tb += UT) {
        float lg[UT][GM];
        load_logits<GM, UT>(logits, E, G, tb, t1, lg);
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            if (tb + u >= t1) break;
            const int t = (int)(tb + u);
            uint64_t m[GM];
            float sc[GM];
            const int k = select_token<GM>(lg[u], th, G, m, sc);
            if (lane == 0) token_offsets[t] = tok_pos;
            int below = 0;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                if (g < G) {
                    if ((m[g] >> lane) & 1ull) {
                        const int rank = below + rank_below(m[g]);
                        if ((int64_t)pos[g] < cap) {
                            sorted_token[pos[g]] = t;
                            slot_gate[pos[g]] = sc[g];
                        }
                        if ((int64_t)tok_pos + rank < cap) token_slot[tok_pos + rank] = pos[g];
                        ++pos[g];
                    }
                    below += (int)__popcll(m[g]);
                }
            }
            tok_pos += k;
        }
    }
}

// Fill from selection masks (the fused router producer's output): the same
// slot assignment as route_fill_kernel, with each token's selection read from
// its mask words instead of recomputed from logits, and each routed pair's
// gate read from the producer's gate list of its 16-token route group.  Block
// b = producer tile b, wave i = route group q = b * gpt + i.
constexpr int kMaxGroupsPerTile = 16;

template <int GM, int UT>
__global__ __launch_bounds__(kMaxGroupsPerTile * kWave) void route_fill_masks_kernel(
    const uint32_t* __restrict__ masks, const float* __restrict__ gate_ws, int T, int E, int gpt,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ group_counts,
    const int32_t* __restrict__ block_base, const int32_t* __restrict__ group_slots,
    const int32_t* __restrict__ block_slot_base, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ token_offsets, int32_t* __restrict__ sorted_token, float* __restrict__ slot_gate,
    int32_t* __restrict__ token_slot, int64_t cap)
{
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int b = (int)blockIdx.x;
    const int q = b * gpt + wave;
    const int q0 = b * gpt;
    const int G = (E + kWave - 1) / kWave;
    const int nwords = (E + 31) / 32;

    int pos[GM];
    int run = 0;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        const bool ve = g < G && e < E;
        const int c = ve ? counts[e] : 0;
        const int incl = wave_incl_scan(c);
        const int eo = run + incl - c;
        run += __builtin_amdgcn_readlane(incl, kWave - 1);
        // counts of the earlier groups of this tile (all loads issued first)
        const int ec = min(e, E - 1);
        int prev[kMaxGroupsPerTile - 1];
#pragma unroll
        for (int i = 0; i < kMaxGroupsPerTile - 1; ++i) prev[i] = group_counts[(int64_t)min(q0 + i, q) * E + ec];
        int base = eo + block_base[(int64_t)b * E + ec];
#pragma unroll
        for (int i = 0; i < kMaxGroupsPerTile - 1; ++i) base += (i < wave) ? prev[i] : 0;
        pos[g] = ve ? base : 0;
        if (ve && q == 0) expert_offsets[e] = eo;
    }
    if (q == 0 && lane == 0) {
        expert_offsets[E] = run;
        token_offsets[T] = run;
    }
    int tok_pos = block_slot_base[b];
    {
        int prev[kMaxGroupsPerTile - 1];
#pragma unroll
        for (int i = 0; i < kMaxGroupsPerTile - 1; ++i) prev[i] = group_slots[min(q0 + i, q)];
#pragma unroll
        for (int i = 0; i < kMaxGroupsPerTile - 1; ++i) tok_pos += (i < wave) ? prev[i] : 0;
    }
    const int tok_pos0 = tok_pos;
    const float* gl = gate_ws + (int64_t)q * 16 * E;

    const int64_t t0 = (int64_t)q * 16;
    const int64_t t1 = std::min<int64_t>(T, t0 + 16);
    for (int64_t tb = t0; tb < t1; tb += UT) {
        // mask word of the lane's expert in each group, for UT tokens (clamped
        // loads, all issued before the first use)
        uint32_t wv[UT][GM];
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            const int wi = min(2 * g + (lane >> 5), nwords - 1);
#pragma unroll
            for (int u = 0; u < UT; ++u) wv[u][g] = masks[min(tb + u, t1 - 1) * nwords + wi];
        }
        // Three passes over the UT tokens: ranks within each token (ballots),
        // then every gate load (their list positions follow from the token
        // counts alone), then the stores -- so a batch waits for one round
        // trip to the gate list rather than one per token.
        int rk[UT][GM];                                 // rank of the lane's pair within its token, -1 if none
        int kt[UT];
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            int below = 0;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int e = g * kWave + lane;
                const bool bit = tb + u < t1 && g < G && e < E && ((wv[u][g] >> (lane & 31)) & 1u);
                const uint64_t m = (uint64_t)__ballot(bit);
                rk[u][g] = bit ? below + rank_below(m) : -1;
                below += (int)__popcll(m);
            }
            kt[u] = below;
        }
        float gate[UT][GM];
        {
            int tp = tok_pos - tok_pos0;
#pragma unroll
            for (int u = 0; u < UT; ++u) {
#pragma unroll
                for (int g = 0; g < GM; ++g) gate[u][g] = gl[min(tp + max(rk[u][g], 0), 16 * E - 1)];   // the group's list
                tp += kt[u];
            }
        }
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            if (tb + u >= t1) break;
            const int t = (int)(tb + u);
            if (lane == 0) token_offsets[t] = tok_pos;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int rank = rk[u][g];
                if (rank >= 0) {
                    if ((int64_t)pos[g] < cap) {
                        sorted_token[pos[g]] = t;
                        slot_gate[pos[g]] = gate[u][g];
                    }
                    if ((int64_t)tok_pos + rank < cap) token_slot[tok_pos + rank] = pos[g];
                    ++pos[g];
                }
            }
            tok_pos += kt[u];
        }
    }
}

// Expert-group bucket (GM) and tokens in flight per wave (UT = 32 / GM keeps
// the logits of UT tokens x GM groups in 32 VGPRs).
#define ET_SWITCH_GROUPS(G, ...)                                                            \
    if ((G) <= 1) { constexpr int GM = 1, UT = 32; __VA_ARGS__; }                          \
    else if ((G) <= 2) { constexpr int GM = 2, UT = 16; __VA_ARGS__; }                     \
    else if ((G) <= 4) { constexpr int GM = 4, UT = 8; __VA_ARGS__; }                      \
    else if ((G) <= 8) { constexpr int GM = 8, UT = 4; __VA_ARGS__; }                      \
    else { constexpr int GM = 16, UT = 2; __VA_ARGS__; }

}  // namespace et

namespace et {

int launch_route_scan(const int32_t* block_counts, const int32_t* block_slots, int NB, int E, int32_t* counts,
                      int32_t* block_base, int32_t* block_slot_base, hipStream_t s)
{
    const int G = (E + kWave - 1) / kWave;
    route_scan_kernel<<<dim3(G + 1), dim3(kScanThreads), 0, s>>>(block_counts, block_slots, NB, E, counts, block_base,
                                                                  block_slot_base);
    return check_launch("route_scan_kernel");
}

int launch_route_fill_masks(const uint32_t* masks, const float* gate_ws, int T, int E, int gpt, int NB,
                            const int32_t* counts, const int32_t* group_counts, const int32_t* block_base,
                            const int32_t* group_slots, const int32_t* block_slot_base, int32_t* expert_offsets,
                            int32_t* token_offsets, int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                            int64_t cap, hipStream_t s)
{
    if (gpt < 1 || gpt > kMaxGroupsPerTile)
        return fail(ET_ERR_INVALID_ARGUMENT, "route_fill_masks: route groups per tile must be 1..16");
    if (NB == 0) return ET_OK;
    // The producer's expert counts stop at 256 (4 groups of 64); a route
    // group is 16 tokens, so one batch covers it up to 2 groups.
    const int G = (E + kWave - 1) / kWave;
    if (G > 4) return fail(ET_ERR_INVALID_ARGUMENT, "route_fill_masks: at most 256 experts");
#define ET_FILL_MASKS(GM_, UT_)                                                                              \
    route_fill_masks_kernel<GM_, UT_><<<dim3(NB), dim3(gpt * kWave), 0, s>>>(                                \
        masks, gate_ws, T, E, gpt, counts, group_counts, block_base, group_slots, block_slot_base,           \
        expert_offsets, token_offsets, sorted_token, slot_gate, token_slot, cap)
    if (G <= 1) ET_FILL_MASKS(1, 16);
    else if (G <= 2) ET_FILL_MASKS(2, 16);
    else ET_FILL_MASKS(4, 8);
#undef ET_FILL_MASKS
    return check_launch("route_fill_masks_kernel");
}

}  // namespace et

using namespace et;

extern "C" size_t et_route_workspace_bytes(int64_t num_tokens, int64_t num_experts)
{
    if (num_tokens < 0 || num_experts < 1) return 0;
    return route_ws_layout(nullptr, route_plan(num_tokens, num_experts), num_experts).bytes;
}

// Argument checks shared by et_route and et_route_noalloc (no HIP call).
int et::route_check(const char* fn, const float* logits, const float* thr, int64_t T, int64_t E,
                       const int32_t* counts, const int32_t* expert_offsets, const int32_t* token_offsets,
                       const int32_t* sorted_token, const float* slot_gate, const int32_t* token_slot,
                       int64_t slot_capacity)
{
    const std::string f(fn);
    if (T < 0) return fail(ET_ERR_INVALID_ARGUMENT, f + ": num_tokens < 0");
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, f + ": num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (T * E >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, f + ": num_tokens * num_experts must be < 2^31");
    if (slot_capacity < 0) return fail(ET_ERR_INVALID_ARGUMENT, f + ": slot_capacity < 0");
    if (!thr || !counts || !expert_offsets || !token_offsets)
        return fail(ET_ERR_INVALID_ARGUMENT, f + ": null thr/counts/offsets pointer");
    if (T > 0 && !logits) return fail(ET_ERR_INVALID_ARGUMENT, f + ": null logits");
    if (slot_capacity > 0 && (!sorted_token || !slot_gate || !token_slot))
        return fail(ET_ERR_INVALID_ARGUMENT, f + ": null slot array with slot_capacity > 0");
    return ET_OK;
}

extern "C" int et_route(const float* logits, const float* thr, int64_t T, int64_t E,
                        int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                        int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                        int64_t slot_capacity, void* workspace, size_t workspace_bytes, void* stream)
{
    if (int rc = route_check("et_route", logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token,
                             slot_gate, token_slot, slot_capacity))
        return rc;
    if (!workspace) return fail(ET_ERR_INVALID_ARGUMENT, "et_route: null workspace pointer");
    const RoutePlan p = route_plan(T, E);
    const RouteWs ws = route_ws_layout(workspace, p, E);
    if (workspace_bytes < ws.bytes)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_route: workspace needs " + std::to_string(ws.bytes) +
                                                    " bytes, got " + std::to_string(workspace_bytes));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int Ti = (int)T, Ei = (int)E, tw = (int)p.tw, NW = (int)p.NW, NB = (int)p.NB;
    const size_t count_lds = size_t(kRouteWaves) * (E + 1) * 4;

    ET_SWITCH_GROUPS(p.G, route_count_kernel<GM, UT><<<dim3(NB), dim3(kRouteThreads), count_lds, s>>>(
                              logits, thr, Ti, Ei, tw, NW, ws.wave_counts, ws.block_counts, ws.wave_slots,
                              ws.block_slots));
    if (int rc = check_launch("route_count_kernel")) return rc;

    route_scan_kernel<<<dim3(p.G + 1), dim3(kScanThreads), 0, s>>>(ws.block_counts, ws.block_slots, NB, Ei,
                                                                    counts, ws.block_base, ws.block_slot_base);
    if (int rc = check_launch("route_scan_kernel")) return rc;

    ET_SWITCH_GROUPS(p.G, route_fill_kernel<GM, UT><<<dim3(NB), dim3(kRouteThreads), 0, s>>>(
                              logits, thr, Ti, Ei, tw, NW, counts, ws.wave_counts, ws.block_base, ws.wave_slots,
                              ws.block_slot_base, expert_offsets, token_offsets, sorted_token, slot_gate,
                              token_slot, slot_capacity));
    return check_launch("route_fill_kernel");
}

// ---------------------------------------------------------------------------
// et_route_noalloc: et_route with its workspace in a static device array
// ---------------------------------------------------------------------------
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, serving loops that forbid hipMalloc).  The routing kernels' block
// and wave counts live in `scratch`, one copy per GPU for the life of the
// process.  Its address is taken once per device with hipGetSymbolAddress
// (on the first call with that device current) and kept in g_scratch; the
// kernels receive that device address, never the host-side symbol.  Every
// region of the workspace is written by the count kernel before the scan and
// fill kernels read it, so nothing needs clearing between calls.  All calls
// on one GPU share the array: calls that overlap in time on one GPU (on
// different streams, or from different host threads) race.

namespace et {

constexpr size_t kRouteScratchBytes = ET_ROUTE_NOALLOC_SCRATCH_BYTES;
constexpr int kScratchDevices = 64;

static __device__ __align__(256) unsigned char scratch[kRouteScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch[kScratchDevices] = {};

// Device address of the current device's copy of `scratch`.
static int route_scratch(void** out)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(ET_ERR_LAUNCH, std::string("et_route_noalloc: hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kScratchDevices)
        return fail(ET_ERR_UNSUPPORTED, "et_route_noalloc: device index " + std::to_string(dev) + " beyond " +
                                            std::to_string(kScratchDevices));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(ET_ERR_LAUNCH, std::string("et_route_noalloc: hipGetSymbolAddress(scratch): ") +
                                           hipGetErrorString(e));
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return ET_OK;
}

}  // namespace et

extern "C" int et_route_noalloc(const float* logits, const float* thr, int64_t T, int64_t E,
                                int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                                int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                                int64_t slot_capacity, void* stream)
{
    if (int rc = route_check("et_route_noalloc", logits, thr, T, E, counts, expert_offsets, token_offsets,
                             sorted_token, slot_gate, token_slot, slot_capacity))
        return rc;
    const size_t need = route_ws_layout(nullptr, route_plan(T, E), E).bytes;
    if (need > kRouteScratchBytes)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL,
                    "et_route_noalloc: T=" + std::to_string(T) + ", E=" + std::to_string(E) + " needs " +
                        std::to_string(need) + " bytes of scratch; the static scratch holds " +
                        std::to_string(kRouteScratchBytes) + " (call et_route with a workspace)");
    void* ws = nullptr;
    if (int rc = route_scratch(&ws)) return rc;
    return et_route(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate, token_slot,
                    slot_capacity, ws, kRouteScratchBytes, stream);
}
