// et_route.hip -- threshold routing, histogram + exclusive-scan CSR, and the
// stable permutation indices, for gfx950.  No launch uses a global atomic, so
// the output is a deterministic function of (logits, thr).
//
// et_route (the pair-list path) reads the logits once, in three launches:
//   1. count (route_pairs_kernel): a wave walks a route group of 8 tokens with
//      lane = expert; selection is decided against per-expert logit bounds
//      (a sigmoid only between the bounds and for the argmax fallback), and
//      every routed pair is listed in token order with its logit and its
//      (token, occurrence, expert) indices; per-group expert counts and slot
//      totals, and their tile sums, follow.
//   2. segmented scan (route_segscan_kernel): the tile sums' exclusive prefix
//      within segments of up to 256 tiles, and the segment totals.
//   3. place (route_place_kernel): lane = pair; each pair's slot is its
//      expert's first slot in its group plus its occurrence index, its gate the
//      sigmoid of its logit, and a token's offset the list index of its first
//      pair; the slot-indexed outputs go out through an LDS stage in the
//      tile's expert-major order.  Expert slots come out in token order
//      (stable), token-major entries in ascending expert order.
// et_route_noalloc (the two-read path) keeps the older count / scan / fill
// kernels, whose workspace is O(E) per block and fits a small static scratch:
// the count and fill passes each read the logits, with lane = expert.
// et_route_update (et_threshold.hip) runs the EMA update's bin select, collect
// pass and final select as extra blocks of the count, scan and place launches
// (route_pairs_kernel<..., true>, upd_scan_collect_kernel,
// route_place_kernel<..., true>): a small pass beside a big one shares its
// launch without slowing it.
#include <algorithm>
#include <mutex>

#include "et_common.hpp"
#include "et_route_internal.hpp"
#include "et_threshold_internal.hpp"

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

// Logits of UT consecutive tokens starting at tb < t1, lane = expert 64 g +
// lane, with addresses clamped into the matrix: every load is issued
// unconditionally, all before the first use (a guarded load, or a select on
// a loaded value between loads, would make each wait for the previous).  Past
// t1 or past E the value is a copy of a valid logit.
template <int GM, int UT>
__device__ __forceinline__ void load_logits_raw(const float* __restrict__ logits, int E, int G, int64_t tb,
                                                int64_t t1, float (&lg)[UT][GM])
{
    const int lane = lane_id();
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int ec = min(min(g, G - 1) * kWave + lane, E - 1);
#pragma unroll
        for (int u = 0; u < UT; ++u) lg[u][g] = logits[min(tb + u, t1 - 1) * E + ec];
    }
}

// The same, then NaN past t1 or past E (the masking after all the loads).
template <int GM, int UT>
__device__ __forceinline__ void load_logits(const float* __restrict__ logits, int E, int G, int64_t tb,
                                            int64_t t1, float (&lg)[UT][GM])
{
    load_logits_raw<GM, UT>(logits, E, G, tb, t1, lg);
    const int lane = lane_id();
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
        for (int u = 0; u < UT; ++u)
            if (g >= G || g * kWave + lane >= E || tb + u >= t1) lg[u][g] = __builtin_nanf("");
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
// block slot totals.  A wave's first RW rows stay in registers between the
// sum and the prefix pass (RW from the row count, up to 16), so up to 256
// block rows take one round trip to memory for the loads and one for the
// stores; longer ranges re-read their rows.  (The two-read routing and the
// fused router producer use it; et_route's pair path scans in segments.)
template <int RW>
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
        const int ec = min(e, E - 1);
        const int rl = max(r1 - 1, 0);               // a row every clamped load may read
        int v[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) v[i] = block_counts[min(r0 + i, rl) * E + ec];
        int sum = 0;
#pragma unroll
        for (int i = 0; i < RW; ++i) sum += (r0 + i < r1) ? v[i] : 0;
        for (int r = r0 + RW; r < r1; r += RW) {
            int w[RW];
#pragma unroll
            for (int i = 0; i < RW; ++i) w[i] = block_counts[min(r + i, rl) * E + ec];
#pragma unroll
            for (int i = 0; i < RW; ++i) sum += (r + i < r1) ? w[i] : 0;
        }
        part[wave][lane] = ve ? sum : 0;
        __syncthreads();
        int run = 0, total = 0;
        for (int i = 0; i < kScanWaves; ++i) {
            const int p = part[i][lane];
            if (i < wave) run += p;
            total += p;
        }
        if (ve) {
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                if (r0 + i < r1) block_base[(r0 + i) * E + e] = run;
                run += (r0 + i < r1) ? v[i] : 0;
            }
            for (int r = r0 + RW; r < r1; r += RW) {
                int w[RW];
#pragma unroll
                for (int i = 0; i < RW; ++i) w[i] = block_counts[min(r + i, rl) * E + e];
#pragma unroll
                for (int i = 0; i < RW; ++i) {
                    if (r + i < r1) block_base[(r + i) * E + e] = run;
                    run += (r + i < r1) ? w[i] : 0;
                }
            }
            if (wave == 0) counts[e] = total;
        }
    } else {
        const int tid = threadIdx.x;
        const int R = (NB + kScanThreads - 1) / kScanThreads;
        const int r0 = min(NB, tid * R), r1 = min(NB, r0 + R);
        const int rl = max(NB - 1, 0);
        int sum = 0;
        for (int r = r0; r < r1; r += 8) {
            int v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = block_slots[min(r + i, rl)];
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

// ---------------------------------------------------------------------------
// The single-read path of et_route: selection masks and routed gates
// ---------------------------------------------------------------------------
//
// Tokens are split into route groups of 16 (group q = tokens [16 q, 16 q +
// 16)), gpt groups per block tile; wave i of block b walks group q = b * gpt
// + i.  The count kernel is the only pass that reads the logits: it decides
// each token's selection, writes it as a bit mask (masks[t * nwords + e / 32],
// bit e % 32), lists the routed pairs' gates in token order (ascending expert
// within a token) from gate_ws[q * 16 * E], and writes the per-group expert
// counts and slot totals and their tile sums.  The scan and the mask fill
// (route_fill_masks_kernel) then place every pair without the logits.
//
// Selection is decided in the logit domain: select_bounds gives each expert a
// logit hi above which the score clears the threshold and a logit lo below
// which it does not, so the exact sigmoid is evaluated only for logits
// between the two (or NaN) -- none at all in most waves.  A token with no
// expert takes select_fallback on exact scores.  The routed pairs' logits are
// collected in a wave-private LDS list at their gate positions and turned
// into gates 64 at a time (one sigmoid per lane), so a wave evaluates about
// (routed pairs) / 64 sigmoids instead of one per (token, expert).  The
// selection, gates and fallback are those of select_token bit for bit.
constexpr int kMaxGroupsPerTile = 16;

// LDS list capacity of one wave: the list is flushed whenever it holds 64 or
// more entries, and a token adds at most 64 * GM; one more entry takes the
// writes of lanes that have nothing to list.
template <int GM> constexpr int kPairList = kWave * (GM + 1) + 1;

// Route groups per tile at most, by expert-group bucket (LDS within 64 KiB).
template <int GM> constexpr int kMaxGpt = GM > 8 ? 4 : GM > 4 ? 8 : kMaxGroupsPerTile;

// Fill from selection masks (et_route's count kernel or the fused router
// producer): the slot assignment of route_fill_kernel, with each token's
// selection read from its mask words and each routed pair's gate from its
// group's gate list.  Block b = tile b, wave i = route group q = b * gpt + i.
// Every independent load of a wave -- the expert counts, its group's counts
// and slot total, the tile's bases, its first mask words and first gates --
// is issued before the first use, so the prologue costs one round trip to
// memory; the prefix over the tile's earlier groups then goes through LDS.
// The wave walks its tokens with lane = expert, as the two-read fill does,
// but lists each routed pair (its slot and token, in token-major order) in a
// wave-private LDS list instead of storing it from the expert's lane; the
// list is written out 64 pairs at a time with lane = pair, so every store
// instruction carries 64 pairs (token_slot contiguously; sorted_token and
// slot_gate at the slots) and the gates are read contiguously, one chunk of
// 64 ahead.
__device__ __noinline__ void flush_pairs(int* ps, int* pt, int lc, const float* __restrict__ gl, float gate0,
                                         int count, int n, int tok_pos, int64_t cap,
                                         int32_t* __restrict__ sorted_token, float* __restrict__ slot_gate,
                                         int32_t* __restrict__ token_slot)
{
    // pairs [0, count) are written out (gate0 = this lane's gate of the first
    // 64); [count, n) move to the front
    const int lane = lane_id();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    for (int j0 = 0; j0 < count; j0 += kWave) {
        const int j = j0 + lane;
        if (j < count) {
            const int slot = ps[j];
            const int tok = pt[j];
            const float gate = j0 == 0 ? gate0 : gl[j];
            if ((int64_t)tok_pos + j < cap) token_slot[tok_pos + j] = slot;
            if ((int64_t)slot < cap) {
                sorted_token[slot] = tok;
                slot_gate[slot] = gate;
            }
        }
    }
    if (count < n) {
        const int rs = ps[min(count + lane, lc - 1)];
        const int rt = pt[min(count + lane, lc - 1)];
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        if (lane < n - count) {
            ps[lane] = rs;
            pt[lane] = rt;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

template <int GM, int UT>
__global__ __launch_bounds__(kMaxGpt<GM> * kWave) void route_fill_masks_kernel(
    const uint32_t* __restrict__ masks, const float* __restrict__ gate_ws, int T, int E, int gpt,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ group_counts,
    const int32_t* __restrict__ block_base, const int32_t* __restrict__ group_slots,
    const int32_t* __restrict__ block_slot_base, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ token_offsets, int32_t* __restrict__ sorted_token, float* __restrict__ slot_gate,
    int32_t* __restrict__ token_slot, int64_t cap)
{
    constexpr int LC = kPairList<GM>;
    constexpr int DUMMY = LC - 1;
    extern __shared__ int lds_i[];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int b = (int)blockIdx.x;
    const int q = b * gpt + wave;
    const int G = (E + kWave - 1) / kWave;
    const int nwords = (E + 31) / 32;
    int* red = lds_i;                          // [gpt][E] group counts, then [gpt] slot totals
    int* ps = lds_i + gpt * (E + 1) + wave * 2 * LC;   // slots of the listed pairs
    int* pt = ps + LC;                                  // their tokens
    const int64_t t0 = (int64_t)q * 16;
    const int64_t t1 = std::min<int64_t>(T, t0 + 16);
    const float* gl = gate_ws + (int64_t)q * 16 * E;
    const int gl_last = 16 * E - 1;

    // every independent load first
    int cnt_e[GM], cnt_q[GM], bb[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int ec = min(min(g, G - 1) * kWave + lane, E - 1);
        cnt_e[g] = counts[ec];
        cnt_q[g] = group_counts[(int64_t)q * E + ec];
        bb[g] = block_base[(int64_t)b * E + ec];
    }
    const int slots_q = group_slots[q];
    const int tile_slot_base = block_slot_base[b];
    uint32_t wv[UT][GM];
    if (t0 < t1) {
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            const int wi = min(2 * g + (lane >> 5), nwords - 1);
#pragma unroll
            for (int u = 0; u < UT; ++u) wv[u][g] = masks[min(t0 + u, t1 - 1) * nwords + wi];
        }
    }
    float gpre = gl[min(lane, gl_last)];       // gates of the first chunk of 64 pairs

    // the tile's earlier groups, through LDS
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        if (g < G && e < E) red[wave * E + e] = cnt_q[g];
    }
    if (lane == 0) red[gpt * E + wave] = slots_q;
    __syncthreads();
    int pos[GM];
    int run = 0;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        const bool ve = g < G && e < E;
        const int c = ve ? cnt_e[g] : 0;
        const int incl = wave_incl_scan(c);
        const int eo = run + incl - c;
        run += __builtin_amdgcn_readlane(incl, kWave - 1);
        int base = eo + bb[g];
        for (int i = 0; i < wave; ++i) base += ve ? red[i * E + e] : 0;
        pos[g] = ve ? base : 0;
        if (ve && q == 0) expert_offsets[e] = eo;
    }
    if (q == 0 && lane == 0) {
        expert_offsets[E] = run;
        token_offsets[T] = run;
    }
    int tok_pos = tile_slot_base;
    for (int i = 0; i < wave; ++i) tok_pos += red[gpt * E + i];

    int toff = 0;        // lane u: token_offsets of token t0 + u
    int lp = 0;          // pairs of the group so far
    int pend = 0;        // of which still listed
    for (int64_t tb = t0; tb < t1; tb += UT) {
        if (tb != t0) {
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int wi = min(2 * g + (lane >> 5), nwords - 1);
#pragma unroll
                for (int u = 0; u < UT; ++u) wv[u][g] = masks[min(tb + u, t1 - 1) * nwords + wi];
            }
        }
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            if (tb + u >= t1) break;
            const int t = (int)(tb + u);
            toff = lane == (int)(t - t0) ? tok_pos + lp : toff;
            int below = pend;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int e = g * kWave + lane;
                const bool bit = g < G && e < E && ((wv[u][g] >> (lane & 31)) & 1u);
                const uint64_t m = (uint64_t)__ballot(bit);
                const int at = bit ? below + rank_below(m) : DUMMY;
                ps[at] = pos[g];
                pt[at] = t;
                pos[g] += bit ? 1 : 0;
                below += (int)__popcll(m);
            }
            const int k = below - pend;
            pend += k;
            lp += k;
            if (pend >= kWave) {
                const int full = pend & ~(kWave - 1);
                const int done = lp - pend;
                flush_pairs(ps, pt, LC, gl + done, gpre, full, pend, tok_pos + done, cap, sorted_token, slot_gate,
                            token_slot);
                gpre = gl[min(done + full + lane, gl_last)];
                pend -= full;
            }
        }
    }
    if (pend > 0) {
        const int done = lp - pend;
        flush_pairs(ps, pt, LC, gl + done, gpre, pend, pend, tok_pos + done, cap, sorted_token, slot_gate,
                    token_slot);
    }
    if ((int64_t)lane < t1 - t0) token_offsets[t0 + lane] = toff;
}

// ---------------------------------------------------------------------------
// et_route's pair-list path
// ---------------------------------------------------------------------------
//
// The count kernel (route_pairs_kernel) is the only pass over the logits.
// Per route group of kPairGroup tokens it lists every routed pair in token
// order (ascending expert within a token) as {logit bits, occ | u << 5 |
// e << 9}: u the token's index in the group, occ the number of earlier tokens
// of the group routed to the same expert e.  It also writes the group's expert
// counts and slot total, and their tile sums.  After the scan, the place
// kernel (route_place_kernel) turns the lists into the outputs with lane =
// pair: slot = (the expert's first slot in this group) + occ, from a
// per-expert table in LDS, gate = sigmoid(logit) -- one sigmoid per pair, 64
// pairs per instruction -- and a token's offset = the list index of its first
// pair (every token has at least one).
//
// Fewer tokens per wave give more waves, whose serial instruction streams are
// what bounds the count kernel: kPairGroup = 8.
constexpr int kPairGroup = 8;
constexpr int kInfoTok = 5;      // occ: bits 0-4 (the running count reaches kPairGroup)
constexpr int kInfoExpert = 9;   // u: bits 5-8, e (< 1024): bits 9-18

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// (m >> lane) & 1 ? b : a, reading the wave-uniform mask m as the lane
// select of one v_cndmask (the compiler otherwise moves m into vector
// registers and tests the lane's bit with shifts).
__device__ __forceinline__ int mask_select(uint64_t m, int a, int b)
{
    int r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(m));
    return r;
}

// v + ((m >> lane) & 1): the mask as the carry-in of one add.
__device__ __forceinline__ uint32_t add_mask_bit(uint32_t v, uint64_t m)
{
    uint32_t r;
    uint64_t carry;
    asm("v_addc_co_u32_e64 %0, %1, %2, 0, %3" : "=v"(r), "=s"(carry) : "v"(v), "s"(m));
    return r;
}

// popcount(m & lanes below this one) + base
__device__ __forceinline__ int rank_below_plus(uint64_t m, int base)
{
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)base));
}

// One walk of a wave over its route group.  EXACT = false decides every
// selection by the logit bounds and gives up (returns true, leaving the group
// unfinished) when a batch holds a logit between an expert's bounds (or NaN);
// it evaluates sigmoids only for the argmax fallback of a token with no
// expert.  EXACT = true evaluates the exact score where the bounds do not
// decide, and always finishes.  Both take the fallback on exact scores.  FULL: the group has all kPairGroup tokens (no bound
// checks).  The list (two words per entry) is flushed to `gp` in whole chunks
// of 64 entries as it fills.  info[g] runs as (e << kInfoExpert) + (count so
// far).  With GM <= 2 every expert group exists (G == GM).
template <int GM, int UT, bool EXACT, bool FULL>
__device__ __forceinline__ bool route_walk(const float* __restrict__ logits, int E, int Grt, int64_t t0, int nu_rt,
                                           float (&lg)[UT][GM], const float (&th)[GM], const float (&hi)[GM],
                                           const float (&lo)[GM], const bool (&ve)[GM], uint32_t* list, int dummy,
                                           u32x2_t* __restrict__ gp, uint32_t (&info)[GM], int& lp)
{
    const int lane = lane_id();
    const int G = GM <= 2 ? GM : Grt;
    const int nu = FULL ? kPairGroup : nu_rt;
#pragma unroll
    for (int g = 0; g < GM; ++g) info[g] = (uint32_t)(g * kWave + lane) << kInfoExpert;
    lp = 0;
    int pend = 0;
    for (int ub = 0; ub < nu; ub += UT) {
        if (ub != 0 || (EXACT && UT < kPairGroup)) load_logits_raw<GM, UT>(logits, E, G, t0 + ub, t0 + nu, lg);
        uint64_t ambm = 0ull;     // lanes that met an ambiguous logit in the batch
#pragma unroll
        for (int u = 0; u < UT; ++u) {
            if (!FULL && ub + u >= nu) break;
            const int uu = ub + u;
            uint64_t mm[GM];
            int k = 0;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                mm[g] = 0ull;
                if (g < G) {
                    const float l = lg[u][g];
                    if (EXACT) {
                        const bool sure = l >= hi[g];
                        const bool amb = ve[g] && !sure && !(l <= lo[g]);
                        bool sel = sure;
                        if (__ballot(amb) != 0ull) sel = amb ? sigmoid(l) >= th[g] : sure;
                        mm[g] = (uint64_t)__ballot(sel);
                    } else {
                        // a lane past E has hi = NaN and lo = +inf: never
                        // selected, never ambiguous (unless its copied logit
                        // is NaN, which only sends the group to the exact walk)
                        mm[g] = (uint64_t)__ballot(l >= hi[g]);
                        ambm |= (uint64_t)__ballot(!(l <= lo[g])) & ~mm[g];
                    }
                    k += (int)__popcll(mm[g]);
                }
            }
            if (k == 0) {
                // the argmax fallback on exact scores (in the bounds walk too:
                // if the batch also met an ambiguous logit, the exact walk
                // redoes the group)
                float sc[GM];
#pragma unroll
                for (int g = 0; g < GM; ++g) sc[g] = ve[g] ? sigmoid(lg[u][g]) : __builtin_nanf("");
                select_fallback<GM>(sc, G, mm);
                k = 1;
            }
            int below = pend;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                if (g < G) {
                    const int at = mask_select(mm[g], dummy, rank_below_plus(mm[g], below));
                    list[2 * at] = f2u(lg[u][g]);
                    list[2 * at + 1] = info[g] | ((uint32_t)uu << kInfoTok);
                    info[g] = add_mask_bit(info[g], mm[g]);
                    below += (int)__popcll(mm[g]);
                }
            }
            pend += k;
            lp += k;
            if (pend >= kWave) {
                // whole chunks of 64 to the group's list; the rest to the front
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                const u32x2_t* l2 = reinterpret_cast<const u32x2_t*>(list);
                const int full = pend & ~(kWave - 1);
                u32x2_t* dst = gp + (lp - pend);
                for (int j0 = 0; j0 < full; j0 += kWave) dst[j0 + lane] = l2[j0 + lane];
                const u32x2_t v = l2[min(full + lane, dummy)];
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                if (lane < pend - full) reinterpret_cast<u32x2_t*>(list)[lane] = v;
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
                pend -= full;
            }
        }
        if (!EXACT && ambm != 0ull) return true;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (lane < pend) gp[(lp - pend) + lane] = reinterpret_cast<const u32x2_t*>(list)[lane];
    return false;
}

// The EMA update's bin select as the first `nblocks` blocks of the count
// launch of et_route_update (BIN = true): blocks [0, nblocks) select (one
// expert each, 1024 threads), the rest count tile blockIdx.x - nblocks.
struct BinRole {
    const uint32_t* partial;
    uint32_t* bin;
    uint32_t* rank;
    float* bnd;
    int nbx;
    int nblocks;
    uint32_t c;
};

template <int GM, int UT, bool BIN = false>
__global__ __launch_bounds__(kMaxGpt<GM> * kWave, GM <= 2 ? 8 : 1) void route_pairs_kernel(
    const float* __restrict__ logits, const float* __restrict__ thr, int T, int E, int gpt,
    u32x2_t* __restrict__ pairs, uint8_t* __restrict__ group_counts, int32_t* __restrict__ group_slots,
    int32_t* __restrict__ block_counts, int32_t* __restrict__ block_slots, BinRole br)
{
    constexpr int LC = kPairList<GM>;
    extern __shared__ float lds_f[];
    int tile = (int)blockIdx.x;
    if constexpr (BIN) {
        static_assert(kMaxGpt<GM> * kWave == kSelectThreads, "the bin-select blocks fill the launch's blocks");
        if (tile < br.nblocks) {
            thr_bin_block(tile, br.nbx, br.partial, br.c, br.bin, br.rank, br.bnd);
            return;
        }
        tile -= br.nblocks;
        if ((int)threadIdx.x >= gpt * kWave) return;   // the tile's gpt waves count
    }
    float* bth = lds_f;                      // [GM * 64] thresholds, by (group, lane)
    float* bhi = bth + GM * kWave;           // [GM * 64] logit bounds
    float* blo = bhi + GM * kWave;
    uint32_t* lists = reinterpret_cast<uint32_t*>(blo + GM * kWave);   // [gpt][2 LC]; then the tile sums (int)
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int G = (E + kWave - 1) / kWave;
    const int64_t q = (int64_t)tile * gpt + wave;
    const int64_t t0 = q * kPairGroup;
    const int64_t t1 = std::min<int64_t>(T, t0 + kPairGroup);

    // the thresholds this wave turns into bounds, then the group's logits, so
    // the bounds wait only for the thresholds (lanes past E keep a copy of a
    // valid logit: their bounds never select)
    float thw[GM];
#pragma unroll
    for (int i = 0; i < GM; ++i) {
        const int g = wave + i * gpt;
        const int e = g * kWave + lane;
        thw[i] = (g < G && e < E) ? thr[e] : __builtin_nanf("");
    }
    float lg[UT][GM];
    if (t0 < t1) load_logits_raw<GM, UT>(logits, E, G, t0, t1, lg);
#pragma unroll
    for (int i = 0; i < GM; ++i) {
        const int g = wave + i * gpt;
        if (g < G) {
            float h, l;
            select_bounds(thw[i], h, l);
            bth[g * kWave + lane] = thw[i];
            bhi[g * kWave + lane] = h;
            blo[g * kWave + lane] = l;
        }
    }
    __syncthreads();
    float th[GM], hi[GM], lo[GM];
    bool ve[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const bool vg = g < G;
        th[g] = vg ? bth[g * kWave + lane] : __builtin_nanf("");
        hi[g] = vg ? bhi[g * kWave + lane] : __builtin_nanf("");
        lo[g] = vg ? blo[g * kWave + lane] : __builtin_nanf("");
        ve[g] = vg && g * kWave + lane < E;
    }

    uint32_t* list = lists + wave * 2 * LC;
    u32x2_t* gp = pairs + q * kPairGroup * (int64_t)E;
    const int nu = (int)std::max<int64_t>(0, t1 - t0);
    uint32_t info[GM];
    int lp;
    bool redo;
    if (nu == kPairGroup)
        redo = route_walk<GM, UT, false, true>(logits, E, G, t0, nu, lg, th, hi, lo, ve, list, LC - 1, gp, info, lp);
    else
        redo = route_walk<GM, UT, false, false>(logits, E, G, t0, nu, lg, th, hi, lo, ve, list, LC - 1, gp, info, lp);
    if (redo) route_walk<GM, UT, true, false>(logits, E, G, t0, nu, lg, th, hi, lo, ve, list, LC - 1, gp, info, lp);
    int cnt[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) cnt[g] = (int)(info[g] & ((1u << kInfoTok) - 1u));

#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        if (g < G && e < E) group_counts[q * E + e] = (uint8_t)cnt[g];   // <= kPairGroup
    }
    if (lane == 0) group_slots[q] = lp;

    // tile sums through LDS (over the lists, which every wave has finished)
    int* red = reinterpret_cast<int*>(lists);
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        if (g < G && e < E) red[wave * E + e] = cnt[g];
    }
    if (lane == 0) red[gpt * E + wave] = lp;
    __syncthreads();
    for (int e = (int)threadIdx.x; e < E; e += gpt * kWave) {
        int sum = 0;
        for (int i = 0; i < gpt; ++i) sum += red[i * E + e];
        block_counts[(int64_t)tile * E + e] = sum;
    }
    if (threadIdx.x == 0) {
        int sum = 0;
        for (int i = 0; i < gpt; ++i) sum += red[gpt * E + i];
        block_slots[tile] = sum;
    }
}

// Segmented scan of the pair path.  Tiles are split into segments of RS
// consecutive tiles (RS <= kSegTiles).  Block (s, g), g < G: lane = expert of
// group g, wave w scans RW = ceil(RS / 16) tiles of segment s, writes each
// tile's exclusive prefix within the segment to block_base and the segment's
// totals to seg_counts[s][e].  Block (s, G): the same for the tile slot totals
// (block_slot_base within the segment, seg_slots[s]).  Every block takes one
// round trip for its loads and one for its stores; the place kernel adds the
// totals of the earlier segments.
constexpr int kSegTiles = 256;

// Block (seg, gy) of the scan, kScanThreads threads.
__device__ __forceinline__ void route_segscan_block(
    int seg, int gy, const int32_t* __restrict__ block_counts, const int32_t* __restrict__ block_slots, int NB,
    int E, int RS, int32_t* __restrict__ block_base, int32_t* __restrict__ seg_counts,
    int32_t* __restrict__ block_slot_base, int32_t* __restrict__ seg_slots)
{
    __shared__ int part[kScanWaves][kWave];
    __shared__ int wtot[kScanWaves];
    const int lane = lane_id();
    const int wave = (int)threadIdx.x >> 6;
    const int G = (E + kWave - 1) / kWave;
    const int s0 = seg * RS, s1 = min(NB, s0 + RS);
    if (gy < G) {
        const int e = gy * kWave + lane;
        const bool ve = e < E;
        const int ec = min(e, E - 1);
        const int RW = (RS + kScanWaves - 1) / kScanWaves;
        const int r0 = min(s1, s0 + wave * RW), r1 = min(s1, r0 + RW);
        const int rl = max(r1 - 1, 0);
        int v[kSegTiles / kScanWaves];
#pragma unroll
        for (int i = 0; i < kSegTiles / kScanWaves; ++i) v[i] = block_counts[min(r0 + i, rl) * E + ec];
        int sum = 0;
#pragma unroll
        for (int i = 0; i < kSegTiles / kScanWaves; ++i) sum += (r0 + i < r1) ? v[i] : 0;
        part[wave][lane] = ve ? sum : 0;
        __syncthreads();
        int run = 0, total = 0;
        for (int i = 0; i < kScanWaves; ++i) {
            const int p = part[i][lane];
            if (i < wave) run += p;
            total += p;
        }
        if (ve) {
#pragma unroll
            for (int i = 0; i < kSegTiles / kScanWaves; ++i) {
                if (r0 + i < r1) block_base[(r0 + i) * E + e] = run;
                run += (r0 + i < r1) ? v[i] : 0;
            }
            if (wave == 0) seg_counts[seg * E + e] = total;
        }
    } else {
        const int tid = (int)threadIdx.x;
        const int r = s0 + tid;
        const int v = r < s1 ? block_slots[r] : 0;
        const int incl = wave_incl_scan(v);
        if (lane == kWave - 1) wtot[wave] = incl;
        __syncthreads();
        int run = incl - v;
        int total = 0;
        for (int i = 0; i < kScanWaves; ++i) {
            if (i < wave) run += wtot[i];
            total += wtot[i];
        }
        if (r < s1) block_slot_base[r] = run;
        if (tid == 0) seg_slots[seg] = total;
    }
}

__global__ __launch_bounds__(kScanThreads) void route_segscan_kernel(
    const int32_t* __restrict__ block_counts, const int32_t* __restrict__ block_slots, int NB, int E, int RS,
    int32_t* __restrict__ block_base, int32_t* __restrict__ seg_counts, int32_t* __restrict__ block_slot_base,
    int32_t* __restrict__ seg_slots)
{
    route_segscan_block((int)blockIdx.x, (int)blockIdx.y, block_counts, block_slots, NB, E, RS, block_base,
                        seg_counts, block_slot_base, seg_slots);
}

// et_route_update's scan launch: blocks [0, ncol) run the EMA update's
// collect pass (token block b % nbx of 64-expert group b / nbx), the rest the
// segmented scan, block ncol + seg * (G + 1) + gy.  Both read only what earlier
// launches wrote, and each role fills a 1024-thread block.
static_assert(kScanThreads == kHistThreads, "the scan and collect blocks have one size");

__global__ __launch_bounds__(kScanThreads) void upd_scan_collect_kernel(
    int ncol, int nbx, const float* __restrict__ logits, int T, int E, int tpb, const uint32_t* __restrict__ bin,
    const float* __restrict__ bnd, uint32_t* __restrict__ cand, uint32_t* __restrict__ cand_n,
    const int32_t* __restrict__ block_counts, const int32_t* __restrict__ block_slots, int NB, int RS,
    int32_t* __restrict__ block_base, int32_t* __restrict__ seg_counts, int32_t* __restrict__ block_slot_base,
    int32_t* __restrict__ seg_slots)
{
    const int b = (int)blockIdx.x;
    if (b < ncol) {
        thr_collect_block<kHistUT>(b % nbx, b / nbx, nbx, logits, T, E, tpb, bin, bnd, cand, cand_n);
        return;
    }
    const int G1 = (E + kWave - 1) / kWave + 1;
    route_segscan_block((b - ncol) / G1, (b - ncol) % G1, block_counts, block_slots, NB, E, RS, block_base,
                        seg_counts, block_slot_base, seg_slots);
}

// Place kernel: block b = tile b; wave i handles the tile's route groups
// q = b * gpt + PG * i + j, j < PG (PG = 2, or 1 for one-group tiles), one
// after the other.  Wave 0 works out what the whole tile shares -- the expert
// totals (over every scan segment), expert_offsets, and the tile's first slot
// per expert and first token-major index (its prefix within its segment plus
// the earlier segments) -- and leaves it in LDS; each wave then adds the
// counts of the tile's earlier groups (also through LDS), keeps its current
// group's first slot per expert in an LDS table, and places the group's pairs
// 64 at a time.  Every independent load of a wave (its groups' counts and
// slot totals, their first 64 list entries) goes out first.
// Token-major outputs (token_slot, token_offsets) are written as the pairs
// are placed.  The slot-indexed ones (sorted_token, slot_gate) are staged in
// LDS in the tile's own expert-major order -- expert e's pairs of the tile
// are its slots [tbase[e], tbase[e] + n_e), at stage positions [loff[e],
// loff[e] + n_e) with loff the exclusive scan of the tile's expert counts --
// and written out by the whole block with lane = stage position, so one store
// instruction covers a few contiguous runs of slots rather than 64 scattered
// ones.  A tile with more than kStage pairs writes them directly.
constexpr int kPlaceGroups = 2;
constexpr int kStage = 2048;
constexpr int kXcds = 8;           // accelerator complex dies of an MI355X

// The EMA update's final select as the first blocks of the place launch of
// et_route_update (FIN = true, tiles of kMaxGroupsPerTile groups): blocks
// [0, E) select (one expert each, with the place blocks' kPlaceThreads
// threads), blocks [E, nblocks) (to a multiple of 8) do nothing, and block
// nblocks + i places the tiles that block i places without them.
constexpr int kPlaceThreads = kMaxGroupsPerTile / 2 * kWave;   // 8 waves, 2 route groups each
constexpr int kPairFinalKeys = 6144;   // candidates the paired final select holds in LDS
struct FinalRole {
    const uint32_t* bin;
    const uint32_t* rank;
    uint32_t* key;
    const uint32_t* cand;
    const uint32_t* cand_n;
    float* thr;
    float* stat;
    float m;
    int E, nblocks, nbx, T, tpb;
};

template <int GM, bool FIN = false>
__global__ __launch_bounds__(kMaxGpt<GM> * kWave / 2) void route_place_kernel(
    const u32x2_t* __restrict__ pairs, int T, int E, int gpt, int PG, int S, int RS,
    const int32_t* __restrict__ seg_counts, const int32_t* __restrict__ seg_slots,
    const uint8_t* __restrict__ group_counts, const int32_t* __restrict__ block_base,
    const int32_t* __restrict__ group_slots, const int32_t* __restrict__ block_slot_base,
    const int32_t* __restrict__ block_counts, const int32_t* __restrict__ block_slots, int32_t* __restrict__ counts,
    int32_t* __restrict__ expert_offsets, int32_t* __restrict__ token_offsets, int32_t* __restrict__ sorted_token,
    float* __restrict__ slot_gate, int32_t* __restrict__ token_slot, int64_t cap, FinalRole fr)
{
    extern __shared__ int lds_i[];
    if constexpr (FIN) {
        static_assert(kMaxGpt<GM> * kWave / 2 == kPlaceThreads, "the final-select blocks fill the launch's blocks");
        if ((int)blockIdx.x < fr.nblocks) {
            if ((int)blockIdx.x < fr.E)
                thr_final_block<kPlaceThreads, kPairFinalKeys>((int)blockIdx.x, fr.nbx, fr.T, fr.tpb, fr.bin, fr.rank,
                                                               fr.key, fr.cand, fr.cand_n, fr.thr, fr.stat, fr.m,
                                                               reinterpret_cast<uint32_t*>(lds_i));
            return;
        }
    }
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    // Blocks go to the 8 XCDs in turn (block i to XCD i % 8).  With a whole
    // number of tiles per XCD, XCD x takes tiles [x n, (x + 1) n): its writes
    // to an expert's slots then form one contiguous range, whose cache lines
    // fill in that XCD's L2 instead of being written back in pieces by several.
    const int nb = (int)gridDim.x - (FIN ? fr.nblocks : 0);
    const int bx = (int)blockIdx.x - (FIN ? fr.nblocks : 0);
    const int b = (nb % kXcds == 0) ? (bx % kXcds) * (nb / kXcds) + bx / kXcds : bx;
    const int g0 = PG * wave;                       // the wave's first group within the tile
    const int G = (E + kWave - 1) / kWave;
    const int nwave = (int)blockDim.x / kWave;
    int* red = lds_i;                               // [gpt][E] group counts, then [gpt] slot totals
    int* tbase = lds_i + gpt * (E + 1);             // [E] the tile's first slot per expert, then [1] token-major
    int* loff = tbase + E + 1;                      // [E] the tile's expert-major stage offsets
    int2* ptab0 = reinterpret_cast<int2*>(lds_i + ((loff + E - lds_i + 1) & ~1));   // (8-byte aligned)
    int2* ptab = ptab0 + wave * E;                  // the current group's (first slot, stage position)
    int* st_slot = reinterpret_cast<int*>(ptab0 + nwave * E);   // [kStage] stage
    int* st_tok = st_slot + kStage;
    float* st_gate = reinterpret_cast<float*>(st_tok + kStage);
    const int gp_last = kPairGroup * E - 1;
    const int tile_pairs = block_slots[b];
    const bool staged = tile_pairs <= kStage;       // block-uniform

    int cnt_q[kPlaceGroups][GM], lp[kPlaceGroups];
    u32x2_t pr[kPlaceGroups];
#pragma unroll
    for (int j = 0; j < kPlaceGroups; ++j) {
        const int q = b * gpt + g0 + min(j, PG - 1);
#pragma unroll
        for (int g = 0; g < GM; ++g)
            cnt_q[j][g] = group_counts[(int64_t)q * E + min(min(g, G - 1) * kWave + lane, E - 1)];
        lp[j] = group_slots[q];
        pr[j] = pairs[(int64_t)q * kPairGroup * E + min(lane, gp_last)];
    }

    if (wave == 0) {
        const int seg = b / RS;
        int cnt_e[GM], bb[GM], tc[GM];
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            bb[g] = block_base[(int64_t)b * E + min(min(g, G - 1) * kWave + lane, E - 1)];
            tc[g] = block_counts[(int64_t)b * E + min(min(g, G - 1) * kWave + lane, E - 1)];
            cnt_e[g] = 0;
        }
        int tile_slot_base = block_slot_base[b];
        constexpr int SC = GM <= 2 ? 16 : 4;       // segments per round of loads
        for (int c0 = 0; c0 < S; c0 += SC) {
            int sv[GM][SC], ssl[SC];
#pragma unroll
            for (int i = 0; i < SC; ++i) {
                const int sg = min(c0 + i, S - 1);
                ssl[i] = seg_slots[sg];
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    sv[g][i] = seg_counts[sg * E + min(min(g, G - 1) * kWave + lane, E - 1)];
            }
#pragma unroll
            for (int i = 0; i < SC; ++i) {
                const bool in = c0 + i < S, before = c0 + i < seg;
                tile_slot_base += before ? ssl[i] : 0;
#pragma unroll
                for (int g = 0; g < GM; ++g) {
                    cnt_e[g] += in ? sv[g][i] : 0;
                    bb[g] += before ? sv[g][i] : 0;
                }
            }
        }
        int run = 0, lrun = 0;
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            const int e = g * kWave + lane;
            const bool ve = g < G && e < E;
            const int c = ve ? cnt_e[g] : 0;
            const int incl = wave_incl_scan(c);
            const int eo = run + incl - c;
            run += __builtin_amdgcn_readlane(incl, kWave - 1);
            const int n = ve ? tc[g] : 0;
            const int lincl = wave_incl_scan(n);
            if (ve) loff[e] = lrun + lincl - n;
            lrun += __builtin_amdgcn_readlane(lincl, kWave - 1);
            if (ve) tbase[e] = eo + bb[g];
            if (ve && b == 0) {
                expert_offsets[e] = eo;
                counts[e] = c;
            }
        }
        if (lane == 0) {
            tbase[E] = tile_slot_base;
            if (b == 0) {
                expert_offsets[E] = run;
                token_offsets[T] = run;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kPlaceGroups; ++j) {
        if (j < PG) {
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int e = g * kWave + lane;
                if (g < G && e < E) red[(g0 + j) * E + e] = cnt_q[j][g];
            }
            if (lane == 0) red[gpt * E + g0 + j] = lp[j];
        }
    }
    __syncthreads();
    int base[GM], lbase[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        base[g] = 0;
        lbase[g] = 0;
        if (g < G && e < E) {
            int pre = 0;
            for (int i = 0; i < g0; ++i) pre += red[i * E + e];
            base[g] = tbase[e] + pre;
            lbase[g] = loff[e] + pre;
        }
    }
    int tok_pos = tbase[E];
    for (int i = 0; i < g0; ++i) tok_pos += red[gpt * E + i];

#pragma unroll
    for (int j = 0; j < kPlaceGroups; ++j) {
        if (j >= PG) break;
        const int q = b * gpt + g0 + j;
        const int64_t t0 = (int64_t)q * kPairGroup;
        const u32x2_t* gp = pairs + (int64_t)q * kPairGroup * E;
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            const int e = g * kWave + lane;
            if (g < G && e < E) ptab[e] = make_int2(base[g], lbase[g]);
            base[g] += cnt_q[j][g];
            lbase[g] += cnt_q[j][g];
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        u32x2_t nx = pr[j];
        int u_prev = -1;     // token index of the previous chunk's last pair
        for (int j0 = 0; j0 < lp[j]; j0 += kWave) {
            const u32x2_t cur = nx;
            if (j0 + kWave < lp[j]) nx = gp[min(j0 + kWave + lane, gp_last)];
            const int jj = j0 + lane;
            const uint32_t info = cur.y;
            const int u = (int)((info >> kInfoTok) & 15u);
            const int u_left = __shfl_up(u, 1, kWave);
            if (jj < lp[j]) {
                // a token's first pair gives its offset
                if (u != (lane == 0 ? u_prev : u_left)) token_offsets[t0 + u] = tok_pos + jj;
                const int2 pt = ptab[info >> kInfoExpert];
                const int occ = (int)(info & ((1u << kInfoTok) - 1u));
                const int slot = pt.x + occ;
                if ((int64_t)tok_pos + jj < cap) token_slot[tok_pos + jj] = slot;
                const float gate = sigmoid(u2f(cur.x));
                if (staged) {
                    const int at = pt.y + occ;
                    st_slot[at] = slot;
                    st_tok[at] = (int)(t0 + u);
                    st_gate[at] = gate;
                } else if ((int64_t)slot < cap) {
                    sorted_token[slot] = (int)(t0 + u);
                    slot_gate[slot] = gate;
                }
            }
            u_prev = __builtin_amdgcn_readlane(u, kWave - 1);
        }
        tok_pos += lp[j];
    }
    if (!staged) return;
    __syncthreads();
    for (int i = (int)threadIdx.x; i < tile_pairs; i += (int)blockDim.x) {
        const int slot = st_slot[i];
        if ((int64_t)slot < cap) {
            sorted_token[slot] = st_tok[i];
            slot_gate[slot] = st_gate[i];
        }
    }
}

// Expert-group bucket (GM) and tokens in flight per wave (UT = 32 / GM keeps
// the logits of UT tokens x GM groups in 32 VGPRs).
#define ET_SWITCH_GROUPS(G, ...)                                                            \
    if ((G) <= 1) { constexpr int GM = 1, UT = 32; (void)UT; __VA_ARGS__; }                 \
    else if ((G) <= 2) { constexpr int GM = 2, UT = 16; (void)UT; __VA_ARGS__; }            \
    else if ((G) <= 4) { constexpr int GM = 4, UT = 8; (void)UT; __VA_ARGS__; }             \
    else if ((G) <= 8) { constexpr int GM = 8, UT = 4; (void)UT; __VA_ARGS__; }             \
    else { constexpr int GM = 16, UT = 2; (void)UT; __VA_ARGS__; }

}  // namespace et

namespace et {

int launch_route_scan(const int32_t* block_counts, const int32_t* block_slots, int NB, int E, int32_t* counts,
                      int32_t* block_base, int32_t* block_slot_base, hipStream_t s)
{
    const int G = (E + kWave - 1) / kWave;
    const int R = (NB + kScanWaves - 1) / kScanWaves;
#define ET_SCAN(RW_) route_scan_kernel<RW_><<<dim3(G + 1), dim3(kScanThreads), 0, s>>>( \
        block_counts, block_slots, NB, E, counts, block_base, block_slot_base)
    if (R <= 8) ET_SCAN(8);
    else ET_SCAN(16);
#undef ET_SCAN
    return check_launch("route_scan_kernel");
}

int launch_route_fill_masks(const uint32_t* masks, const float* gate_ws, int T, int E, int gpt, int NB,
                            const int32_t* counts, const int32_t* group_counts, const int32_t* block_base,
                            const int32_t* group_slots, const int32_t* block_slot_base, int32_t* expert_offsets,
                            int32_t* token_offsets, int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                            int64_t cap, hipStream_t s)
{
    // A route group is 16 tokens, so one batch of tokens covers it up to 2
    // expert groups; beyond, batches keep UT * GM = 32.  The pair lists take
    // 2 * kPairList<GM> ints per wave: up to 16 waves with 256 experts or
    // fewer, 8 up to 512 and 4 beyond (at most 64 KiB).
    const int G = (E + kWave - 1) / kWave;
    if (gpt < 1 || gpt > (G > 8 ? kMaxGpt<16> : G > 4 ? kMaxGpt<8> : kMaxGpt<4>))
        return fail(ET_ERR_INVALID_ARGUMENT, "route_fill_masks: too many route groups per tile");
    if (NB == 0) return ET_OK;
#define ET_FILL_MASKS(GM_, UT_)                                                                              \
    route_fill_masks_kernel<GM_, UT_>                                                                        \
        <<<dim3(NB), dim3(gpt * kWave), size_t(gpt) * (E + 1 + 2 * kPairList<GM_>) * 4, s>>>(               \
        masks, gate_ws, T, E, gpt, counts, group_counts, block_base, group_slots, block_slot_base,           \
        expert_offsets, token_offsets, sorted_token, slot_gate, token_slot, cap)
    if (G <= 1) ET_FILL_MASKS(1, 16);
    else if (G <= 2) ET_FILL_MASKS(2, 16);
    else if (G <= 4) ET_FILL_MASKS(4, 8);
    else if (G <= 8) ET_FILL_MASKS(8, 4);
    else ET_FILL_MASKS(16, 2);
#undef ET_FILL_MASKS
    return check_launch("route_fill_masks_kernel");
}

// Workspace of the pair-list path: tiles of gpt route groups of kPairGroup tokens.
// Enough tiles to give each CU one where T allows (gpt up to 16, fewer with
// more than 256 experts, which keeps the kernels' LDS within 64 KiB).
struct PairPlan {
    int G;
    int64_t gpt, ntiles, ngroups;
    int64_t nseg, seg_tiles;   // scan segments and tiles per segment
};

static PairPlan pair_plan(int64_t T, int64_t E)
{
    PairPlan p;
    p.G = (int)((E + kWave - 1) / kWave);
    const int64_t max_gpt = p.G > 8 ? kMaxGpt<16> : p.G > 4 ? kMaxGpt<8> : kMaxGpt<4>;
    // (a power of two, so the place kernel's waves split a tile's groups evenly)
    const int64_t per_tile = kPairGroup * 256;        // tokens per tile for 256 tiles
    const int64_t want = std::max<int64_t>(1, std::min<int64_t>(max_gpt, (T + per_tile - 1) / per_tile));
    p.gpt = 1;
    while (p.gpt * 2 <= want) p.gpt *= 2;
    p.ntiles = std::max<int64_t>(1, (T + kPairGroup * p.gpt - 1) / (kPairGroup * p.gpt));
    p.ngroups = p.ntiles * p.gpt;
    p.nseg = (p.ntiles + kSegTiles - 1) / kSegTiles;
    p.seg_tiles = (p.ntiles + p.nseg - 1) / p.nseg;
    return p;
}

struct PairWs {
    u32x2_t* pairs;            // [ngroups * kPairGroup * E] each group's routed pairs, token order
    uint8_t* group_counts;     // [ngroups * E] (at most kPairGroup each)
    int32_t* block_counts;     // [ntiles * E]
    int32_t* block_base;       // [ntiles * E]
    int32_t* group_slots;      // [ngroups]
    int32_t* block_slots;      // [ntiles]
    int32_t* block_slot_base;  // [ntiles]
    int32_t* seg_counts;       // [nseg * E]
    int32_t* seg_slots;        // [nseg]
    size_t bytes;
};

static PairWs pair_ws_layout(void* base, const PairPlan& p, int64_t E)
{
    PairWs ws{};
    size_t off = 0;
    char* b = static_cast<char*>(base);
    auto take = [&](int64_t words) {
        void* q = b + off;
        off += align256(size_t(words) * 4);
        return q;
    };
    ws.pairs = static_cast<u32x2_t*>(take(2 * p.ngroups * kPairGroup * E));
    ws.group_counts = static_cast<uint8_t*>(take((p.ngroups * E + 3) / 4));
    ws.block_counts = static_cast<int32_t*>(take(p.ntiles * E));
    ws.block_base = static_cast<int32_t*>(take(p.ntiles * E));
    ws.group_slots = static_cast<int32_t*>(take(p.ngroups));
    ws.block_slots = static_cast<int32_t*>(take(p.ntiles));
    ws.block_slot_base = static_cast<int32_t*>(take(p.ntiles));
    ws.seg_counts = static_cast<int32_t*>(take(p.nseg * E));
    ws.seg_slots = static_cast<int32_t*>(take(p.nseg));
    ws.bytes = off;
    return ws;
}

// The count pass of the pair-list path on stream s.
static int pairs_count(const float* logits, const float* thr, int64_t T, int64_t E, const PairPlan& p,
                       const PairWs& ws, hipStream_t s)
{
    const int Ti = (int)T, Ei = (int)E, gpt = (int)p.gpt, NB = (int)p.ntiles;
    ET_SWITCH_GROUPS(p.G, {
        constexpr int UTM = UT > kPairGroup ? kPairGroup : UT;   // a route group's tokens at most
        const size_t lds = size_t(3 * GM * kWave) * 4 +
                           std::max(size_t(gpt) * kPairList<GM> * 8, size_t(gpt) * (E + 1) * 4);
        route_pairs_kernel<GM, UTM><<<dim3(NB), dim3(gpt * kWave), lds, s>>>(
            logits, thr, Ti, Ei, gpt, ws.pairs, ws.group_counts, ws.group_slots, ws.block_counts,
            ws.block_slots, BinRole{});
    });
    return check_launch("route_pairs_kernel");
}

// The place pass of the pair-list path on stream s.
static int pairs_place(int64_t T, int64_t E, int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                       int32_t* sorted_token, float* slot_gate, int32_t* token_slot, int64_t slot_capacity,
                       const PairPlan& p, const PairWs& ws, hipStream_t s)
{
    const int Ti = (int)T, Ei = (int)E, gpt = (int)p.gpt, NB = (int)p.ntiles;
    const int S = (int)p.nseg, RS = (int)p.seg_tiles;
    ET_SWITCH_GROUPS(p.G, {
        const int PG = gpt >= kPlaceGroups ? kPlaceGroups : 1;
        const int nwave = gpt / PG;
        const size_t lds = (size_t(gpt) * (E + 1) + 2 * size_t(E) + 2 + 2 * size_t(nwave) * E + 3 * kStage) * 4;
        route_place_kernel<GM><<<dim3(NB), dim3(nwave * kWave), lds, s>>>(
            ws.pairs, Ti, Ei, gpt, PG, S, RS, ws.seg_counts, ws.seg_slots, ws.group_counts, ws.block_base,
            ws.group_slots, ws.block_slot_base, ws.block_counts, ws.block_slots, counts, expert_offsets,
            token_offsets, sorted_token, slot_gate, token_slot, slot_capacity, FinalRole{});
    });
    return check_launch("route_place_kernel");
}

// The three launches of et_route on stream s (arguments checked).
static int route_pairs_path(const float* logits, const float* thr, int64_t T, int64_t E, int32_t* counts,
                            int32_t* expert_offsets, int32_t* token_offsets, int32_t* sorted_token,
                            float* slot_gate, int32_t* token_slot, int64_t slot_capacity, const PairPlan& p,
                            const PairWs& ws, hipStream_t s)
{
    if (int rc = pairs_count(logits, thr, T, E, p, ws, s)) return rc;
    const int S = (int)p.nseg, RS = (int)p.seg_tiles;
    route_segscan_kernel<<<dim3(S, p.G + 1), dim3(kScanThreads), 0, s>>>(
        ws.block_counts, ws.block_slots, (int)p.ntiles, (int)E, RS, ws.block_base, ws.seg_counts,
        ws.block_slot_base, ws.seg_slots);
    if (int rc = check_launch("route_segscan_kernel")) return rc;
    return pairs_place(T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate, token_slot,
                       slot_capacity, p, ws, s);
}

int route_update_count_bin(const float* logits, const float* thr, int64_t T, int64_t E, void* workspace,
                           const uint32_t* partial, int nbx, uint32_t c, uint32_t* bin, uint32_t* rank,
                           float* bnd, hipStream_t s)
{
    const PairPlan p = pair_plan(T, E);
    const PairWs ws = pair_ws_layout(workspace, p, E);
    if (p.G > 4) return fail(ET_ERR_INVALID_ARGUMENT, "route_update_count_bin: more than 256 experts");
    const int Ti = (int)T, Ei = (int)E, gpt = (int)p.gpt, NB = (int)p.ntiles;
    const BinRole br{partial, bin, rank, bnd, nbx, Ei, c};
    ET_SWITCH_GROUPS(p.G, {
        if constexpr (GM <= 4) {
            const size_t lds = size_t(3 * GM * kWave) * 4 +
                               std::max(size_t(gpt) * kPairList<GM> * 8, size_t(gpt) * (E + 1) * 4);
            route_pairs_kernel<GM, kPairGroup, true><<<dim3(Ei + NB), dim3(kSelectThreads), lds, s>>>(
                logits, thr, Ti, Ei, gpt, ws.pairs, ws.group_counts, ws.group_slots, ws.block_counts,
                ws.block_slots, br);
        }
    });
    return check_launch("route_pairs_kernel (with the bin select)");
}

int route_update_scan_collect(int64_t T, int64_t E, void* workspace, const float* logits, int nbx, int tpb,
                              const uint32_t* bin, const float* bnd, uint32_t* cand, uint32_t* cand_n,
                              hipStream_t s)
{
    const PairPlan p = pair_plan(T, E);
    const PairWs ws = pair_ws_layout(workspace, p, E);
    const int S = (int)p.nseg, RS = (int)p.seg_tiles;
    const int ncol = nbx * p.G;
    upd_scan_collect_kernel<<<dim3((unsigned)(ncol + S * (p.G + 1))), dim3(kScanThreads), 0, s>>>(
        ncol, nbx, logits, (int)T, (int)E, tpb, bin, bnd, cand, cand_n, ws.block_counts, ws.block_slots,
        (int)p.ntiles, RS, ws.block_base, ws.seg_counts, ws.block_slot_base, ws.seg_slots);
    return check_launch("upd_scan_collect_kernel");
}

bool route_update_pairs_final(int64_t T, int64_t E)
{
    const PairPlan p = pair_plan(T, E);
    return p.G <= 4 && p.gpt == kMaxGroupsPerTile;
}

int route_update_place_final(int64_t T, int64_t E, int32_t* counts, int32_t* expert_offsets,
                             int32_t* token_offsets, int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                             int64_t slot_capacity, void* workspace, int nbx, int tpb, const uint32_t* bin,
                             const uint32_t* rank, uint32_t* key, const uint32_t* cand, const uint32_t* cand_n,
                             float* thr, float* stat, float m, hipStream_t s)
{
    const PairPlan p = pair_plan(T, E);
    const PairWs ws = pair_ws_layout(workspace, p, E);
    if (!route_update_pairs_final(T, E))
        return fail(ET_ERR_INVALID_ARGUMENT, "route_update_place_final: tiles below 16 route groups");
    const int Ti = (int)T, Ei = (int)E, gpt = (int)p.gpt, NB = (int)p.ntiles;
    const int S = (int)p.nseg, RS = (int)p.seg_tiles;
    const int nfin = (Ei + kXcds - 1) / kXcds * kXcds;
    const FinalRole fr{bin, rank, key, cand, cand_n, thr, stat, m, Ei, nfin, nbx, Ti, tpb};
    ET_SWITCH_GROUPS(p.G, {
        if constexpr (GM <= 4) {
            const int nwave = gpt / kPlaceGroups;
            const size_t lds = std::max((size_t(gpt) * (E + 1) + 2 * size_t(E) + 2 + 2 * size_t(nwave) * E +
                                         3 * kStage) * 4,
                                        size_t(kFinalLdsWords<kPlaceThreads, kPairFinalKeys>) * 4);
            route_place_kernel<GM, true><<<dim3(nfin + NB), dim3(kPlaceThreads), lds, s>>>(
                ws.pairs, Ti, Ei, gpt, kPlaceGroups, S, RS, ws.seg_counts, ws.seg_slots, ws.group_counts,
                ws.block_base, ws.group_slots, ws.block_slot_base, ws.block_counts, ws.block_slots, counts,
                expert_offsets, token_offsets, sorted_token, slot_gate, token_slot, slot_capacity, fr);
        }
    });
    return check_launch("route_place_kernel (with the final select)");
}

int route_update_place(int64_t T, int64_t E, int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                       int32_t* sorted_token, float* slot_gate, int32_t* token_slot, int64_t slot_capacity,
                       void* workspace, hipStream_t s)
{
    const PairPlan p = pair_plan(T, E);
    return pairs_place(T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate, token_slot,
                       slot_capacity, p, pair_ws_layout(workspace, p, E), s);
}

}  // namespace et

using namespace et;

// The pair lists reserve room for every (token, expert) pair (8 bytes each),
// so above kPairWsLimit bytes of workspace et_route takes the two-read kernels
// instead: the same outputs bit for bit, from a workspace of O(E) per block.
constexpr size_t kPairWsLimit = size_t(1) << 30;

static size_t pair_ws_bytes(int64_t T, int64_t E) { return pair_ws_layout(nullptr, pair_plan(T, E), E).bytes; }
static size_t two_read_ws_bytes(int64_t T, int64_t E) { return route_ws_layout(nullptr, route_plan(T, E), E).bytes; }
static bool use_pairs(int64_t T, int64_t E) { return pair_ws_bytes(T, E) <= kPairWsLimit; }

bool et::route_uses_pairs(int64_t T, int64_t E) { return T > 0 && E >= 1 && use_pairs(T, E); }

static int route_two_read(const float* logits, const float* thr, int64_t T, int64_t E, int32_t* counts,
                          int32_t* expert_offsets, int32_t* token_offsets, int32_t* sorted_token, float* slot_gate,
                          int32_t* token_slot, int64_t slot_capacity, void* workspace, hipStream_t s);

extern "C" size_t et_route_workspace_bytes(int64_t num_tokens, int64_t num_experts)
{
    if (num_tokens < 0 || num_experts < 1) return 0;
    return use_pairs(num_tokens, num_experts) ? pair_ws_bytes(num_tokens, num_experts)
                                              : two_read_ws_bytes(num_tokens, num_experts);
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
    const size_t need = et_route_workspace_bytes(T, E);
    if (workspace_bytes < need)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_route: workspace needs " + std::to_string(need) +
                                                    " bytes, got " + std::to_string(workspace_bytes));
    if (!use_pairs(T, E))
        return route_two_read(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                              token_slot, slot_capacity, workspace, static_cast<hipStream_t>(stream));
    const PairPlan p = pair_plan(T, E);
    const PairWs ws = pair_ws_layout(workspace, p, E);
    return route_pairs_path(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                            token_slot, slot_capacity, p, ws, static_cast<hipStream_t>(stream));
}

// The two-read routing (et_route_noalloc's path, and et_route's where the
// pair lists would exceed kPairWsLimit): a count pass and a fill pass that
// both read the logits, with a workspace of per-wave and per-block counts only
// (O(E) per block, so it fits a small static scratch at any T).  Outputs
// bit-identical to the pair path's.
static int route_two_read(const float* logits, const float* thr, int64_t T, int64_t E, int32_t* counts,
                          int32_t* expert_offsets, int32_t* token_offsets, int32_t* sorted_token, float* slot_gate,
                          int32_t* token_slot, int64_t slot_capacity, void* workspace, hipStream_t s)
{
    const RoutePlan p = route_plan(T, E);
    const RouteWs ws = route_ws_layout(workspace, p, E);
    const int Ti = (int)T, Ei = (int)E, tw = (int)p.tw, NW = (int)p.NW, NB = (int)p.NB;
    const size_t count_lds = size_t(kRouteWaves) * (E + 1) * 4;

    ET_SWITCH_GROUPS(p.G, route_count_kernel<GM, UT><<<dim3(NB), dim3(kRouteThreads), count_lds, s>>>(
                              logits, thr, Ti, Ei, tw, NW, ws.wave_counts, ws.block_counts, ws.wave_slots,
                              ws.block_slots));
    if (int rc = check_launch("route_count_kernel")) return rc;
    if (int rc = launch_route_scan(ws.block_counts, ws.block_slots, NB, Ei, counts, ws.block_base,
                                   ws.block_slot_base, s))
        return rc;
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
    return route_two_read(logits, thr, T, E, counts, expert_offsets, token_offsets, sorted_token, slot_gate,
                          token_slot, slot_capacity, ws, static_cast<hipStream_t>(stream));
}
