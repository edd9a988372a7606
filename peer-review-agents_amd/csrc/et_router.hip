// et_router.hip -- the router producer of the path on gfx950: router logits
// L[T, E] (f32) = X[T, d] (bf16) * W[E, d]^T (bf16), binary32 accumulation on
// the MFMA units (v_mfma_f32_16x16x32_bf16 up to 128 experts,
// v_mfma_f32_32x32x16_bf16 above).
//
// The GEMM is skinny (E <= 256 columns) and HBM-bound on X: X is read from HBM
// exactly once, W (E * d * 2 bytes) stays in L2 and is staged through LDS.
//
// Tiling: a block of MW waves owns 32 * MT * MW tokens (32 * MT per wave)
// and all E experts (NT groups of 32).  The K dimension advances in chunks of
// KC: the block copies W[:, chunk] into LDS (double-buffered, one barrier per
// chunk) while every wave loads its own X fragments straight from global
// memory, several chunks ahead; each k-step is one MFMA per token tile and
// expert tile.
//
// MFMA operand layouts (M x M tiles, M = 16 or 32): lane l holds
//   A: row l % M, k = 8 * (l / M) + i, i < 8      -> 16 contiguous bytes of X
//   B: col l % M, k = 8 * (l / M) + i             -> 16 contiguous bytes of W
//   C, M = 16 (k-step 32): col l % 16, acc[j] at row 4 * (l / 16) + j
//   C, M = 32 (k-step 16): col l % 32, acc[j] at row 8 * (j / 4) + 4 * (l / 32) + j % 4
// With M = 16 one X load covers 16 rows x 64 contiguous bytes instead of 32
// rows x 32 bytes, which streams faster.  On gfx950 the 16x16x32 result
// equals two 16-k steps rounded in turn, so both forms give the same bits
// (tests/test_gpu_router.py checks the rounding and the k order).  With more than 128 experts the
// 16 x 16 form's B fragments of a k-step and two token tiles per wave no
// longer fit beside the accumulators, and the 32 x 32 form is kept.
#include <algorithm>

#include "et_common.hpp"
#include "et_route_internal.hpp"

namespace et {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Word 3 of a gfx9 buffer descriptor for raw (untyped, stride 0) access.
constexpr int kBufDword3 = 0x00020000;
// A byte offset past every descriptor's num_records (< 2^31): loads return 0.
constexpr uint32_t kBufOutOfRange = 0x80000000u;

// Shape of one instantiation.  NT expert tiles of 32 (all E experts), MW
// waves per block, MT token tiles of 32 per wave (each B fragment read from
// LDS feeds MT MFMAs), an X register ring of R chunks (R - 1 in flight ahead
// of the MFMAs).  KC is the k per chunk; the double-buffered W chunk in LDS is
// 2 * NT * 32 rows * (KC + 8) bf16 (rows padded by 16 bytes so that the B
// fragment reads are free of bank conflicts).
// The two MFMA forms: tile size M, k per MFMA, and the token row (within the
// tile) of accumulator element j of a lane.
template <int M> struct RtMfma;
template <> struct RtMfma<16> {
    static constexpr int KS = 32;
    static constexpr int NACC = 4;
    typedef f32x4_t Acc;
    // Both forms are written as inline assembly with the accumulator tied in
    // place ("+a"): with the builtin, the register allocator gave some
    // products a new accumulator register and restored them with ~160
    // accumulator moves per chunk (over 1000 per tile at 8 expert tiles).  The
    // compiler does not see these as MFMAs, so the kernel waits out their
    // latency itself before it reads the accumulators.
    static __device__ __forceinline__ Acc mma(u32x4_t a, u32x4_t b, Acc c)
    {
        asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        return c;
    }
    static __device__ __forceinline__ int crow(int lane, int j) { return 4 * (lane >> 4) + j; }
    // 16-token route group (within the wave) of element j of token tile m
    static constexpr int group(int m, int /*j*/) { return m; }
};
template <> struct RtMfma<32> {
    static constexpr int KS = 16;
    static constexpr int NACC = 16;
    typedef f32x16_t Acc;
    static __device__ __forceinline__ Acc mma(u32x4_t a, u32x4_t b, Acc c)
    {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
        return c;
    }
    static __device__ __forceinline__ int crow(int lane, int j) { return 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3); }
    static constexpr int group(int m, int j) { return 2 * m + j / 8; }
};

template <int NT, int MW, int MT, int R> struct RtShape {
    static constexpr int THREADS = MW * kWave;
    static constexpr int M = NT <= 4 ? 16 : 32;   // MFMA tile
    using F = RtMfma<M>;
    static constexpr int KC = NT <= 4 ? 64 : 32;
    static constexpr int PITCH = KC + 8;        // bf16 per LDS row
    static constexpr int KSTEPS = KC / F::KS;   // MFMA k-steps per chunk
    static constexpr int TT = 32 * MT / M;      // token tiles per wave
    static constexpr int ET = 32 * NT / M;      // expert tiles
    // B fragments are read in units of ET / UPS tiles, double-buffered
    // (unit u + 1 under unit u's MFMAs)
    static constexpr int UPS = M == 16 ? 2 : 1;
    static constexpr int PF = R - 1;
    static constexpr int TOK = MW * MT * 32;    // tokens per block tile
    static constexpr int SEGS = NT * 32 * KC / 8;  // 16-byte W segments per chunk
    static constexpr int SEGS_PER_THREAD = (SEGS + THREADS - 1) / THREADS;
    static_assert(R % 2 == 0, "the W register double buffer is indexed by ring position");
};

// Outputs of the routing epilogue (ROUTE = true), by 16-token route group
// (group q = tokens [16 q, 16 q + 16)) and by block tile.
struct RouteEpilogue {
    const float* thr;          // [E]
    uint32_t* masks;           // [T * nwords], nwords = ceil(E / 32): token t's selection, bit e % 32 of word e / 32
    float* gate_ws;            // [ngroups * 16 * E]: group q's routed gates in token order, ascending expert
    int32_t* group_counts;     // [ngroups * E]
    int32_t* block_counts;     // [ntiles * E]
    int32_t* group_slots;      // [ngroups]
    int32_t* block_slots;      // [ntiles]
};

// Routing epilogue of one producer tile.  The wave's logits pass through a
// wave-private LDS buffer, 16 tokens at a time, and are then walked token by
// token with lane = expert.  Selection is decided in the logit domain by the
// per-expert bounds of select_bounds, with the exact score only for logits
// between the bounds (or NaN); tokens with no expert take select_fallback on
// exact scores.  So the selection, gates and argmax fallback are those of
// et_route (select_token) bit for bit, with far fewer sigmoids: gates are
// computed only for the routed pairs, after each 16-token group.
// acc[m][n][j] is the logit of token t0 + M m + crow(lane, j), expert
// M n + lane % M.  The waves run through it
// independently; the tile sums at the end take two block barriers (`red`
// aliases the W buffer, which every wave has finished reading once the K
// loop's last barrier has passed).
template <int NT, int MW, int MT, typename S>
__device__ __forceinline__ void route_epilogue(const typename S::F::Acc (&acc)[S::TT][S::ET], const RouteEpilogue& ro,
                                               float* rbuf, int* red, int tile, int wave, int64_t t0, int T, int E)
{
    constexpr int P = NT * 32 + 8;              // LDS row pitch (floats)
    constexpr int GM = (NT * 32 + kWave - 1) / kWave;
    constexpr int DUMMY = 16 * P - 1;           // padding of the last row: never a logit, never a list entry
    const int lane = lane_id();
    const int G = (E + kWave - 1) / kWave;
    const int nwords = (E + 31) / 32;
    float th[GM], hi[GM], lo[GM];
    load_thresholds<GM>(ro.thr, E, G, th);
#pragma unroll
    for (int g = 0; g < GM; ++g) select_bounds(th[g], hi[g], lo[g]);
    int wcnt[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) wcnt[g] = 0;
    int wslots = 0;
    using F = typename S::F;
    constexpr int M = S::M;
#pragma unroll
    for (int gi = 0; gi < 2 * MT; ++gi) {
        {
            // the 16 tokens of route group gi, one row of rbuf each
#pragma unroll
            for (int m = 0; m < S::TT; ++m)
#pragma unroll
                for (int n = 0; n < S::ET; ++n)
#pragma unroll
                    for (int j = 0; j < F::NACC; ++j)
                        if (F::group(m, j) == gi)
                            rbuf[((m * M + F::crow(lane, j)) & 15) * P + n * M + (lane & (M - 1))] = acc[m][n][j];
            // rbuf is private to this wave and a wave's LDS operations run in
            // issue order, so the fences only have to keep the compiler from
            // moving these accesses across each other.
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            const int64_t tg = t0 + gi * 16;               // first token of the route group
            const int64_t q = tg / 16;
            const int nu = (int)std::min<int64_t>(16, std::max<int64_t>(0, (int64_t)T - tg));
            // Stores go through range-checked buffer descriptors: a lane with
            // nothing to store gives an out-of-range offset and its store is
            // dropped, with no branch on the exec mask.
            const __amdgpu_buffer_rsrc_t gres =
                __builtin_amdgcn_make_buffer_rsrc(ro.gate_ws + q * 16 * (int64_t)E, (short)0, 16 * E * 4, kBufDword3);
            const __amdgpu_buffer_rsrc_t mres = __builtin_amdgcn_make_buffer_rsrc(
                ro.masks + (tg < T ? tg : 0) * nwords, (short)0, nu * nwords * 4, kBufDword3);
            int cnt[GM];
#pragma unroll
            for (int g = 0; g < GM; ++g) cnt[g] = 0;
            int lp = 0;
            // Tokens in batches of UB (selections within a batch are
            // independent); the fallback and the outputs follow in token order.
            // The routed pairs' logits are listed in rbuf at their gate
            // positions: the entries of tokens < u + 1 lie below (u + 1) * E <=
            // (u + 1) * P, i.e. in rows already read.
            constexpr int UB = 8 / GM;
#pragma unroll 1
            for (int ub = 0; ub < 16; ub += UB) {
                float lg[UB][GM];
                uint64_t mm[UB][GM];
                int kk[UB];
#pragma unroll
                for (int i = 0; i < UB; ++i) {
                    const int u = ub + i;
                    kk[i] = 0;
#pragma unroll
                    for (int g = 0; g < GM; ++g) {
                        const int e = g * kWave + lane;
                        const float v = rbuf[u * P + min(e, NT * 32 - 1)];   // in bounds for every lane
                        const bool valid = u < nu && g < G && e < E;
                        lg[i][g] = valid ? v : __builtin_nanf("");
                        const bool sure = lg[i][g] >= hi[g];
                        const bool amb = valid && !sure && !(lg[i][g] <= lo[g]);
                        bool sel = sure;
                        if (__ballot(amb) != 0ull) sel = amb ? sigmoid(lg[i][g]) >= th[g] : sure;
                        mm[i][g] = (uint64_t)__ballot(sel);
                        kk[i] += (int)__popcll(mm[i][g]);
                    }
                }
#pragma unroll
                for (int i = 0; i < UB; ++i) {
                    const int u = ub + i;
                    if (u < nu) {
                        if (kk[i] == 0) {
                            float sc[GM];
#pragma unroll
                            for (int g = 0; g < GM; ++g) sc[g] = sigmoid(lg[i][g]);
                            select_fallback<GM>(sc, G, mm[i]);
                            kk[i] = 1;
                        }
                        uint32_t word = 0u;                     // lane i < nwords writes mask word i
#pragma unroll
                        for (int g = 0; g < GM; ++g) {
                            word = lane == 2 * g ? (uint32_t)mm[i][g] : word;
                            word = lane == 2 * g + 1 ? (uint32_t)(mm[i][g] >> 32) : word;
                        }
                        __builtin_amdgcn_raw_buffer_store_b32(
                            word, mres, lane < nwords ? (uint32_t)(u * nwords + lane) * 4u : kBufOutOfRange, 0, 0);
                        int below = 0;
#pragma unroll
                        for (int g = 0; g < GM; ++g) {
                            if (g < G) {
                                const bool sel = (mm[i][g] >> lane) & 1ull;
                                const int gi = lp + below + rank_below(mm[i][g]);   // < 16 E: the group's pairs
                                rbuf[sel ? gi : DUMMY] = lg[i][g];
                                cnt[g] += sel ? 1 : 0;
                                below += (int)__popcll(mm[i][g]);
                            }
                        }
                        lp += kk[i];
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            // gates of the group's routed pairs, in list order
            for (int j0 = 0; j0 < lp; j0 += kWave) {
                const int j = j0 + lane;
                const float gate = sigmoid(rbuf[min(j, DUMMY)]);
                __builtin_amdgcn_raw_buffer_store_b32(f2u(gate), gres, j < lp ? (uint32_t)j * 4u : kBufOutOfRange, 0, 0);
            }
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int e = g * kWave + lane;
                if (g < G && e < E) ro.group_counts[q * E + e] = cnt[g];
                wcnt[g] += cnt[g];
            }
            if (lane == 0) ro.group_slots[q] = lp;
            wslots += lp;
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // rbuf is rewritten by the next group
        }
    }
    // tile sums through LDS
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int e = g * kWave + lane;
        if (g < G && e < E) red[wave * E + e] = wcnt[g];
    }
    if (lane == 0) red[MW * E + wave] = wslots;
    __syncthreads();
    for (int e = (int)threadIdx.x; e < E; e += MW * kWave) {
        int sum = 0;
#pragma unroll
        for (int i = 0; i < MW; ++i) sum += red[i * E + e];
        ro.block_counts[(int64_t)tile * E + e] = sum;
    }
    if (threadIdx.x == 0) {
        int sum = 0;
#pragma unroll
        for (int i = 0; i < MW; ++i) sum += red[MW * E + i];
        ro.block_slots[tile] = sum;
    }
    __syncthreads();
}

// A block owns TOK tokens at a time and loops over token tiles (the grid is
// capped); wave w owns tokens [t0, t0 + 32 * MT).  Every wave sums k in
// k-steps of 16, one MFMA per step, token tile and expert tile, ascending from
// k0(t) = (floor(t / 256) mod 4) * 64 * floor(d / 256) and wrapping to 0, so
// the bits of a logit depend on d and floor(t / 256) mod 4 only -- not on T,
// E or the tiling.
template <int NT, int MW, int MT, int R, bool ROUTE>
__global__ __launch_bounds__(MW * kWave) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int T, int d, int E,
    float* __restrict__ logits, RouteEpilogue ro)
{
    using S = RtShape<NT, MW, MT, R>;
    static_assert(!ROUTE || MW * NT * 32 + MW <= NT * 32 * S::PITCH, "epilogue reduction must fit the W buffer");
    __shared__ uint16_t wl[2][NT * 32 * S::PITCH];
    // routing epilogue: 16 tokens x (NT * 32 + 8) floats per wave
    __shared__ float rbuf[ROUTE ? MW * 16 * (NT * 32 + 8) : 1];
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    using F = typename S::F;
    constexpr int M = S::M;
    const int quad = lane / M;             // which 8 k of a k-step
    const int row = lane & (M - 1);
    const int nchunks = (d + S::KC - 1) / S::KC;
    const int ntiles = (int)((T + S::TOK - 1) / S::TOK);
    // Buffer loads with the hardware range check: an offset at or past a
    // descriptor's num_records returns zeros without touching memory.  So
    // rows past T (X) or past E (W) and k past d read as 0 with the choice
    // made on the address -- no select on loaded data, which would make the
    // load wait right away.
    const __amdgpu_buffer_rsrc_t wres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(w), (short)0, (int)((int64_t)E * d * 2), kBufDword3);

    static_assert(256 % S::TOK == 0, "a block tile lies inside one 256-token group");
    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t t0 = (int64_t)tile * S::TOK + (int64_t)wave * (32 * MT);
        // The k walk of token group g = t / 256 starts at k0 = (g mod 4) * 64 *
        // floor(d / 256) and wraps.  Rows are 2d bytes apart; with d a
        // multiple of a large power of two, blocks walking the same column
        // range at the same time hit a subset of the HBM channels (at C3 the
        // X stream drops from ~6.0 to ~4.7 TB/s).  Chunks past the end stay
        // past the end, so their loads read zeros.
        const int grp = (int)(((int64_t)tile * S::TOK) >> 8);
        const int rot = (grp & 3) * (d / 256) * (64 / S::KC);
        auto chunk_at = [&](int c) { return c < nchunks ? (c + rot < nchunks ? c + rot : c + rot - nchunks) : c; };
        const int64_t rows_here = max<int64_t>(0, min<int64_t>(32 * MT, (int64_t)T - t0));
        const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x + (t0 < T ? t0 : 0) * (int64_t)d), (short)0, (int)(rows_here * d * 2),
            kBufDword3);

        u32x4_t wreg[2][S::SEGS_PER_THREAD];
        auto load_w_one = [&](int c, u32x4_t (&wr)[S::SEGS_PER_THREAD], int i) {
            const int seg = min(tid + i * S::THREADS, S::SEGS - 1);
            const int e = seg / (S::KC / 8);
            const int k = chunk_at(c) * S::KC + (seg % (S::KC / 8)) * 8;
            const uint32_t off = k < d ? ((uint32_t)e * (uint32_t)d + (uint32_t)k) * 2u : kBufOutOfRange;
            wr[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wres, off, 0, 0));
        };
        auto load_w = [&](int c, u32x4_t (&wr)[S::SEGS_PER_THREAD]) {
#pragma unroll
            for (int i = 0; i < S::SEGS_PER_THREAD; ++i) load_w_one(c, wr, i);
        };
        auto store_w = [&](int buf, const u32x4_t (&wr)[S::SEGS_PER_THREAD]) {
#pragma unroll
            for (int i = 0; i < S::SEGS_PER_THREAD; ++i) {
                const int seg = tid + i * S::THREADS;
                if (S::SEGS % S::THREADS == 0 || seg < S::SEGS) {
                    const int e = seg / (S::KC / 8);
                    const int kk = (seg % (S::KC / 8)) * 8;
                    *reinterpret_cast<u32x4_t*>(&wl[buf][e * S::PITCH + kk]) = wr[i];
                }
            }
        };
        u32x4_t xr[R][S::TT][S::KSTEPS];
        auto load_x_one = [&](int c, u32x4_t (&a)[S::TT][S::KSTEPS], int m, int s) {
            const int k = chunk_at(c) * S::KC + s * F::KS + quad * 8;
            const uint32_t off = k < d ? (uint32_t)(m * M + row) * (uint32_t)d * 2u + (uint32_t)k * 2u : kBufOutOfRange;
            a[m][s] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 0, 0));
        };
        auto load_x = [&](int c, u32x4_t (&a)[S::TT][S::KSTEPS]) {
#pragma unroll
            for (int m = 0; m < S::TT; ++m)
#pragma unroll
                for (int s = 0; s < S::KSTEPS; ++s) load_x_one(c, a, m, s);
        };
        // load i of a step (W chunk segments first, then X chunk rows), so the
        // loads can be spread between the step's MFMAs in issue order
        constexpr int NLOADS = S::SEGS_PER_THREAD + S::TT * S::KSTEPS;
        auto load_one = [&](int c, int r, int i) {
            if (i < S::SEGS_PER_THREAD) load_w_one(c + 2, wreg[r & 1], i);
            else {
                const int j = i - S::SEGS_PER_THREAD;
                load_x_one(c + S::PF, xr[(r + S::PF) % R], j / S::KSTEPS, j % S::KSTEPS);
            }
        };

        typename F::Acc acc[S::TT][S::ET];
#pragma unroll
        for (int m = 0; m < S::TT; ++m)
#pragma unroll
            for (int n = 0; n < S::ET; ++n) acc[m][n] = typename F::Acc{};

        // prologue: W chunk 0 -> LDS, W chunk 1 -> wreg[1], X chunks 0 .. PF-1
        load_w(0, wreg[0]);
        load_w(1, wreg[1]);
#pragma unroll
        for (int p = 0; p < S::PF; ++p) load_x(p, xr[p]);
        store_w(0, wreg[0]);
        __syncthreads();
        // Step c: W chunk c is in LDS buffer c & 1, W chunk c + 1 in
        // wreg[(c + 1) & 1], X chunk c in xr[c % R].  r = c % R is a
        // compile-time constant in every unrolled copy, so the rings stay in
        // registers.
        auto step = [&](int c, int r) {
            // Loads complete in issue order and the scheduler must not reorder
            // these: the wait for W chunk c + 1 at the end of the step then
            // leaves X chunks c + 2 .. c + R - 1 in flight.
            // With the 16 x 16 form the loads go one after each of the
            // step's first MFMAs (issued while the MFMA runs); with the 32 x
            // 32 form they stay a block ahead of the MFMAs.
            constexpr bool SPREAD = M == 16;
            __builtin_amdgcn_sched_barrier(0);
            if (!SPREAD) {
                load_w(c + 2, wreg[r & 1]);
                __builtin_amdgcn_sched_barrier(0);
                load_x(c + S::PF, xr[(r + S::PF) % R]);
                __builtin_amdgcn_sched_barrier(0);
            }
            constexpr int UT = S::ET / S::UPS;       // expert tiles per unit
            constexpr int NU = S::UPS * S::KSTEPS;
            const uint16_t* wb = wl[r & 1];
            u32x4_t bf[2][UT];
            auto rdb = [&](int u, int b) {
                const int n0 = (u % S::UPS) * UT, s = u / S::UPS;
#pragma unroll
                for (int n = 0; n < UT; ++n)
                    bf[b][n] = *reinterpret_cast<const u32x4_t*>(
                        &wb[((n0 + n) * M + row) * S::PITCH + s * F::KS + quad * 8]);
            };
            rdb(0, 0);
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                if (u + 1 < NU) rdb(u + 1, (u + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
                const int n0 = (u % S::UPS) * UT, s = u / S::UPS;
#pragma unroll
                for (int n = 0; n < UT; ++n)
#pragma unroll
                    for (int m = 0; m < S::TT; ++m) {
                        acc[m][n0 + n] = F::mma(xr[r][m][s], bf[u & 1][n], acc[m][n0 + n]);
                        const int g = (u * UT + n) * S::TT + m;      // MFMA index within the step
                        if (SPREAD && g < NLOADS) {
                            __builtin_amdgcn_sched_barrier(0);
                            load_one(c, r, g);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                __builtin_amdgcn_sched_barrier(0);
            }
            store_w((r + 1) & 1, wreg[(r + 1) & 1]);
            __syncthreads();
        };
        // Whole groups of R steps have no exit inside, so the compiler's load
        // counters stay exact across the loop and no wait drains the X ring;
        // the last nchunks % R steps run once, guarded.
        const int nmain = nchunks - nchunks % R;
        for (int cb = 0; cb < nmain; cb += R) {
#pragma unroll
            for (int r = 0; r < R; ++r) step(cb + r, r);
        }
#pragma unroll
        for (int r = 0; r < R - 1; ++r)
            if (nmain + r < nchunks) step(nmain + r, r);

        // wait until the last products are written (at most 16 passes of 4
        // cycles after issue; 80 cycles of s_nop).  The MFMAs are inline asm,
        // so the compiler's hazard recognizer does not see them: the
        // scheduling barriers on both sides keep every read of the
        // accumulators (v_accvgpr_read, or a VALU use) after the nops.
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // epilogue: lane l writes expert n * M + l % M of its token rows per tile
        if (!ROUTE || logits != nullptr) {
#pragma unroll
            for (int m = 0; m < S::TT; ++m)
#pragma unroll
                for (int n = 0; n < S::ET; ++n) {
                    const int e = n * M + row;
#pragma unroll
                    for (int j = 0; j < F::NACC; ++j) {
                        const int64_t t = t0 + m * M + F::crow(lane, j);
                        if (t < T && e < E) logits[t * E + e] = acc[m][n][j];
                    }
                }
        }
        if constexpr (ROUTE)
            route_epilogue<NT, MW, MT, S>(acc, ro, rbuf + wave * 16 * (NT * 32 + 8), reinterpret_cast<int*>(wl[0]), tile,
                                       wave, t0, T, E);
    }
}

// X ring length: 8-16 KiB of X in flight per wave.  The 2 x 2 launch (a
// block of 128 tokens) keeps 4 chunks when rows are long (d >= 4096: 4-6%
// faster there), 2 otherwise (4-7% faster at d = 1024 and 2048, where a row
// has few chunks to hide the deeper prologue behind).
template <int NT, int MT> constexpr int kRouterRing = NT <= 4 ? 4 / MT : 4;
constexpr int64_t kRouterLongRow = 4096;

template <int NT, int MW, int MT, bool ROUTE>
static void launch_router(dim3 grid, hipStream_t s, const uint16_t* x, const uint16_t* w, int64_t T, int64_t d,
                          int64_t E, float* logits, const RouteEpilogue& ro)
{
    if constexpr (NT <= 4 && MW == 2 && MT == 2) {
        if (d >= kRouterLongRow) {
            router_logits_kernel<NT, MW, MT, 4, ROUTE>
                <<<grid, dim3(MW * kWave), 0, s>>>(x, w, (int)T, (int)d, (int)E, logits, ro);
            return;
        }
    }
    router_logits_kernel<NT, MW, MT, kRouterRing<NT, MT>, ROUTE>
        <<<grid, dim3(MW * kWave), 0, s>>>(x, w, (int)T, (int)d, (int)E, logits, ro);
}

// Launch shape by batch size: the largest token tile that still gives every
// one of the 256 CUs a tile (two token tiles per wave halve the LDS reads and
// the W staging per token).  Blocks loop over token tiles when the grid is
// capped; the cap is only reached by batches far beyond one resident wave of
// blocks.
struct RouterLaunch {
    int mw, mt;
};
constexpr int64_t kRouterMaxBlocks = 2048;

static RouterLaunch router_launch(int64_t T)
{
    RouterLaunch L{2, 1};
    if (T >= 256 * 256) L = {4, 2};
    else if (T >= 256 * 128) L = {2, 2};
    return L;
}

#define ET_SWITCH_NT(nt, ...)                                                   \
    switch (nt) {                                                               \
        case 1: { constexpr int NT = 1; __VA_ARGS__; } break;                   \
        case 2: { constexpr int NT = 2; __VA_ARGS__; } break;                   \
        case 3: case 4: { constexpr int NT = 4; __VA_ARGS__; } break;           \
        default: { constexpr int NT = 8; __VA_ARGS__; } break;                  \
    }

#define ET_SWITCH_MT(mt, ...)                                                   \
    switch (mt) {                                                               \
        case 2: { constexpr int MT = 2; __VA_ARGS__; } break;                   \
        default: { constexpr int MT = 1; __VA_ARGS__; } break;                  \
    }

#define ET_SWITCH_MW(mw, ...)                                                   \
    switch (mw) {                                                               \
        case 2: { constexpr int MW = 2; __VA_ARGS__; } break;                   \
        default: { constexpr int MW = 4; __VA_ARGS__; } break;                  \
    }

}  // namespace et

using namespace et;

extern "C" int et_router_logits(const void* x, const void* w, int64_t T, int64_t d, int64_t E, float* logits,
                                void* stream)
{
    if (T < 0 || T >= (int64_t(1) << 31)) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_logits: num_tokens out of range");
    if (E < 1 || E > ET_MAX_ROUTER_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_logits: num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_ROUTER_EXPERTS) + "]");
    if (d < 1 || d % 8 != 0 || d >= (int64_t(1) << 22))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_logits: d must be a positive multiple of 8 below 2^22");
    if (T * E >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_logits: num_tokens * num_experts must be < 2^31");
    if (T == 0) return ET_OK;
    if (!x || !w || !logits) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_logits: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_logits: x and w must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int nt = (int)((E + 31) / 32);
    const RouterLaunch L = router_launch(T);
    const int64_t ntiles = (T + 32 * L.mw * L.mt - 1) / (32 * L.mw * L.mt);
    const dim3 grid((unsigned)std::min<int64_t>(ntiles, kRouterMaxBlocks));
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const uint16_t* wp = static_cast<const uint16_t*>(w);
    ET_SWITCH_NT(nt, ET_SWITCH_MW(L.mw, ET_SWITCH_MT(L.mt, launch_router<NT, MW, MT, false>(
                                                               grid, s, xp, wp, T, d, E, logits, RouteEpilogue{}))));
    return check_launch("router_logits_kernel");
}

namespace {

// Workspace of et_router_route: the tokens split into block tiles of
// 32 * mw * mt tokens and route groups of 16.
struct RouterRouteWs {
    uint32_t* masks;           // [T * nwords]
    float* gate_ws;            // [ngroups * 16 * E]
    int32_t* group_counts;     // [ngroups * E]
    int32_t* block_counts;     // [ntiles * E]
    int32_t* block_base;       // [ntiles * E]
    int32_t* group_slots;      // [ngroups]
    int32_t* block_slots;      // [ntiles]
    int32_t* block_slot_base;  // [ntiles]
    int64_t ntiles, gpt;
    size_t bytes;
};

RouterRouteWs router_route_ws(void* base, int64_t T, int64_t E, const RouterLaunch& L)
{
    const int64_t tok = 32 * L.mw * L.mt;
    RouterRouteWs ws{};
    ws.ntiles = (T + tok - 1) / tok;
    ws.gpt = tok / 16;
    const int64_t ngroups = ws.ntiles * ws.gpt;
    const int64_t nwords = (E + 31) / 32;
    size_t off = 0;
    char* b = static_cast<char*>(base);
    auto take = [&](int64_t n) {
        void* q = b + off;
        off += (size_t(n) * 4 + 255) & ~size_t(255);
        return q;
    };
    ws.masks = static_cast<uint32_t*>(take(T * nwords));
    ws.gate_ws = static_cast<float*>(take(ngroups * 16 * E));
    ws.group_counts = static_cast<int32_t*>(take(ngroups * E));
    ws.block_counts = static_cast<int32_t*>(take(ws.ntiles * E));
    ws.block_base = static_cast<int32_t*>(take(ws.ntiles * E));
    ws.group_slots = static_cast<int32_t*>(take(ngroups));
    ws.block_slots = static_cast<int32_t*>(take(ws.ntiles));
    ws.block_slot_base = static_cast<int32_t*>(take(ws.ntiles));
    ws.bytes = off;
    return ws;
}

}  // namespace

extern "C" size_t et_router_route_workspace_bytes(int64_t num_tokens, int64_t num_experts)
{
    if (num_tokens < 0 || num_experts < 1 || num_experts > ET_MAX_ROUTER_EXPERTS) return 0;
    const RouterLaunch L = router_launch(num_tokens);
    return router_route_ws(nullptr, num_tokens, num_experts, L).bytes;
}

extern "C" int et_router_route(const void* x, const void* w, const float* thr, int64_t T, int64_t d, int64_t E,
                               int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                               int32_t* sorted_token, float* slot_gate, int32_t* token_slot, int64_t slot_capacity,
                               float* logits, void* workspace, size_t workspace_bytes, void* stream)
{
    if (T < 0 || T >= (int64_t(1) << 31)) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: num_tokens out of range");
    if (E < 1 || E > ET_MAX_ROUTER_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_ROUTER_EXPERTS) + "]");
    if (d < 1 || d % 8 != 0 || d >= (int64_t(1) << 22))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: d must be a positive multiple of 8 below 2^22");
    if (T * E >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: num_tokens * num_experts must be < 2^31");
    if (slot_capacity < 0) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: slot_capacity < 0");
    if (!thr || !counts || !expert_offsets || !token_offsets || !workspace)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: null thr/counts/offsets/workspace pointer");
    if (T > 0 && (!x || !w)) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: null x or w");
    if (slot_capacity > 0 && (!sorted_token || !slot_gate || !token_slot))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: null slot array with slot_capacity > 0");
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(w) & 15))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_route: x and w must be 16-byte aligned");
    const int nt = (int)((E + 31) / 32);
    const RouterLaunch L = router_launch(T);
    const RouterRouteWs ws = router_route_ws(workspace, T, E, L);
    if (workspace_bytes < ws.bytes)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_router_route: workspace needs " + std::to_string(ws.bytes) +
                                                    " bytes, got " + std::to_string(workspace_bytes));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t ntiles = ws.ntiles;
    if (ntiles > 0) {
        const dim3 grid((unsigned)std::min<int64_t>(ntiles, kRouterMaxBlocks));
        const RouteEpilogue ro{thr, ws.masks, ws.gate_ws, ws.group_counts, ws.block_counts, ws.group_slots,
                               ws.block_slots};
        const uint16_t* xp = static_cast<const uint16_t*>(x);
        const uint16_t* wp = static_cast<const uint16_t*>(w);
        ET_SWITCH_NT(nt, ET_SWITCH_MW(L.mw, ET_SWITCH_MT(L.mt, launch_router<NT, MW, MT, true>(
                                                                   grid, s, xp, wp, T, d, E, logits, ro))));
        if (int rc = check_launch("router_logits_kernel (route)")) return rc;
    }
    if (int rc = launch_route_scan(ws.block_counts, ws.block_slots, (int)ntiles, (int)E, counts, ws.block_base,
                                   ws.block_slot_base, s))
        return rc;
    return launch_route_fill_masks(ws.masks, ws.gate_ws, (int)T, (int)E, (int)ws.gpt, (int)ntiles, counts,
                                   ws.group_counts, ws.block_base, ws.group_slots, ws.block_slot_base,
                                   expert_offsets, token_offsets, sorted_token, slot_gate, token_slot, slot_capacity,
                                   s);
}
