// et_router.hip -- the router producer of the path on gfx950: router logits
// L[T, E] (f32) = X[T, d] (bf16) * W[E, d]^T (bf16), binary32 accumulation on
// the MFMA units (v_mfma_f32_32x32x16_bf16).
//
// The GEMM is skinny (E <= 256 columns) and HBM-bound on X: X is read from HBM
// exactly once, W (E * d * 2 bytes) stays in L2 and is staged through LDS.
//
// Tiling: a block of MW waves owns 32 * MW tokens (32 per wave) and all E
// experts (NT tiles of 32).  The K dimension advances in chunks of KC: the
// block copies W[:, chunk] into LDS (double-buffered, one barrier per chunk)
// while every wave loads its own X fragments straight from global memory,
// several chunks ahead; each k-step of 16 is one MFMA per expert tile.
//
// MFMA 32x32x16 bf16 operand layout (checked on the device): lane l holds
//   A: row l % 32, k = 8 * (l / 32) + i, i < 8     -> 16 contiguous bytes of X
//   B: col l % 32, k = 8 * (l / 32) + i            -> 16 contiguous bytes of W
//   C: col l % 32, acc[j] at row 8 * (j / 4) + 4 * (l / 32) + j % 4
#include <algorithm>

#include "et_common.hpp"

namespace et {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
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
template <int NT, int MW, int MT, int R> struct RtShape {
    static constexpr int THREADS = MW * kWave;
    static constexpr int KC = NT <= 4 ? 64 : 32;
    static constexpr int PITCH = KC + 8;        // bf16 per LDS row
    static constexpr int KSTEPS = KC / 16;
    static constexpr int PF = R - 1;
    static constexpr int TOK = MW * MT * 32;    // tokens per block tile
    static constexpr int SEGS = NT * 32 * KC / 8;  // 16-byte W segments per chunk
    static constexpr int SEGS_PER_THREAD = (SEGS + THREADS - 1) / THREADS;
    static_assert(R % 2 == 0, "the W register double buffer is indexed by ring position");
};

// A block owns TOK tokens at a time and loops over token tiles (the grid is
// capped); wave w owns tokens [t0, t0 + 32 * MT).  Every wave sums k in
// ascending k-steps of 16, one MFMA per step, token tile and expert tile, so
// the bits of a logit depend on d only -- not on T, E or the tiling.
template <int NT, int MW, int MT, int R>
__global__ __launch_bounds__(MW * kWave) void router_logits_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int T, int d, int E,
    float* __restrict__ logits)
{
    using S = RtShape<NT, MW, MT, R>;
    __shared__ uint16_t wl[2][NT * 32 * S::PITCH];
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5;            // which 8 of a k-step's 16
    const int row = lane & 31;
    const int nchunks = (d + S::KC - 1) / S::KC;
    const int ntiles = (int)((T + S::TOK - 1) / S::TOK);
    // Buffer loads with the hardware range check: an offset at or past a
    // descriptor's num_records returns zeros without touching memory.  So
    // rows past T (X) or past E (W) and k past d read as 0 with the choice
    // made on the address -- no select on loaded data, which would make the
    // load wait right away.
    const __amdgpu_buffer_rsrc_t wres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(w), (short)0, (int)((int64_t)E * d * 2), kBufDword3);

    for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t t0 = (int64_t)tile * S::TOK + (int64_t)wave * (32 * MT);
        const int64_t rows_here = max<int64_t>(0, min<int64_t>(32 * MT, (int64_t)T - t0));
        const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x + (t0 < T ? t0 : 0) * (int64_t)d), (short)0, (int)(rows_here * d * 2),
            kBufDword3);

        u32x4_t wreg[2][S::SEGS_PER_THREAD];
        auto load_w = [&](int c, u32x4_t (&wr)[S::SEGS_PER_THREAD]) {
#pragma unroll
            for (int i = 0; i < S::SEGS_PER_THREAD; ++i) {
                const int seg = min(tid + i * S::THREADS, S::SEGS - 1);
                const int e = seg / (S::KC / 8);
                const int k = c * S::KC + (seg % (S::KC / 8)) * 8;
                const uint32_t off = k < d ? ((uint32_t)e * (uint32_t)d + (uint32_t)k) * 2u : kBufOutOfRange;
                wr[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(wres, off, 0, 0));
            }
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
        u32x4_t xr[R][MT][S::KSTEPS];
        auto load_x = [&](int c, u32x4_t (&a)[MT][S::KSTEPS]) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int s = 0; s < S::KSTEPS; ++s) {
                    const int k = c * S::KC + s * 16 + half * 8;
                    const uint32_t off =
                        k < d ? (uint32_t)(m * 32 + row) * (uint32_t)d * 2u + (uint32_t)k * 2u : kBufOutOfRange;
                    a[m][s] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 0, 0));
                }
        };

        f32x16_t acc[MT][NT];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[m][n] = f32x16_t{};

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
            __builtin_amdgcn_sched_barrier(0);
            load_w(c + 2, wreg[r & 1]);
            __builtin_amdgcn_sched_barrier(0);
            load_x(c + S::PF, xr[(r + S::PF) % R]);
            __builtin_amdgcn_sched_barrier(0);
            const uint16_t* wb = wl[r & 1];
#pragma unroll
            for (int s = 0; s < S::KSTEPS; ++s) {
                u32x4_t bf[NT];
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    bf[n] = *reinterpret_cast<const u32x4_t*>(&wb[(n * 32 + row) * S::PITCH + s * 16 + half * 8]);
#pragma unroll
                for (int n = 0; n < NT; ++n)
#pragma unroll
                    for (int m = 0; m < MT; ++m)
                        acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8_t, xr[r][m][s]), __builtin_bit_cast(bf16x8_t, bf[n]), acc[m][n],
                            0, 0, 0);
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

        // epilogue: lane l writes expert n * 32 + l % 32 of 16 token rows per tile
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const int e = n * 32 + row;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int64_t t = t0 + m * 32 + 8 * (j / 4) + 4 * half + (j % 4);
                    if (t < T && e < E) logits[t * E + e] = acc[m][n][j];
                }
            }
    }
}

// X ring length: 12-16 KiB of X in flight per wave.
template <int NT, int MT> constexpr int kRouterRing = (NT <= 4 ? 4 : 8) / MT;

template <int NT, int MW, int MT>
static void launch_router(dim3 grid, hipStream_t s, const uint16_t* x, const uint16_t* w, int64_t T, int64_t d,
                          int64_t E, float* logits)
{
    constexpr int MTE = NT == 8 ? 1 : MT;       // two token tiles of 8 expert tiles do not fit the registers
    router_logits_kernel<NT, MW, MTE, kRouterRing<NT, MTE>>
        <<<grid, dim3(MW * kWave), 0, s>>>(x, w, (int)T, (int)d, (int)E, logits);
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
    if (T >= 256 * 256) return {4, 2};
    if (T >= 256 * 128) return {2, 2};
    return {2, 1};
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
    const int mt = nt == 8 ? 1 : L.mt;
    const int64_t ntiles = (T + 32 * L.mw * mt - 1) / (32 * L.mw * mt);
    const dim3 grid((unsigned)std::min<int64_t>(ntiles, kRouterMaxBlocks));
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const uint16_t* wp = static_cast<const uint16_t*>(w);
    ET_SWITCH_NT(nt, ET_SWITCH_MW(L.mw, ET_SWITCH_MT(L.mt, launch_router<NT, MW, MT>(grid, s, xp, wp, T, d, E, logits))));
    return check_launch("router_logits_kernel");
}
