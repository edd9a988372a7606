// et_router_bwd.hip -- router weight gradient on gfx950:
//     dW[e, c] = sum_t dlogits[t, e] * X[t, c]        (f32 [E, d])
// from the f32 router-logit gradient dlogits [T, E] and the bf16 router input
// X [T, d], on the MFMA units (v_mfma_f32_32x32x16_bf16).
//
// The reduction runs over tokens, which is the outer (row) dimension of both
// operands, so neither loads as an MFMA fragment directly (a fragment lane
// needs 8 consecutive k = tokens).  A block stages 64 tokens x 256 columns of
// X in LDS at a time (row-major, 512-byte rows, a ring of three stages), and
// each wave forms its X fragments with gfx950's transposing LDS read
// ds_read_b64_tr_b16: within each 16-lane group, if lane j points at 4
// consecutive 16-bit elements M[j][0..3], lane i receives M[4 m + i / 4][i % 4]
// for m = 0..3.  With lane j pointing at row r0 + j / 4, columns c0 + 4 (j % 4),
// lane i gets column c0 + i of rows r0..r0+3; two such reads give a fragment
// of 8 consecutive tokens.  Each row stores its 16-byte segment s at slot
// s ^ (4 (row & 3)), which puts the four rows of one read on distinct 64-byte
// bank windows.  dlogits is loaded 8 tokens per lane (one f32 per load, 128
// contiguous bytes per half-wave) and split into hi = bf16(dl) and
// lo = bf16(dl - hi), two MFMAs each, so dW carries ~16 more bits of dl than
// a bf16 GEMM (exact when dl is a bf16 value).
//
// Schedule: a wave runs one MFMA per slot (32 cycles), and every other
// instruction of the stage -- the fragment reads and the hi/lo split of the
// next k-step, the global loads of later stages, the LDS stores of the stage
// after next -- is placed between two MFMAs, in an order pinned with
// scheduling barriers, so it issues while the previous MFMA runs instead of in
// a block of its own.  Stages are separated by a plain s_barrier after the
// wave's LDS operations are done; loads in flight stay in flight across it.
//
// Work split: a block = 4 waves on the same 256 columns and token range.
// With 3 or more expert tiles (32 experts each) a wave takes one expert tile
// and all 8 column tiles (grid z covers tiles past 4; a wave whose tile lies
// past E only stages X); with 2 tiles a wave takes one expert tile and 4
// column tiles, with 1 tile 2 column tiles.  The token range is split over KS
// blocks; each writes its partial dW tile, and a second kernel sums the KS
// partials in order, so the result is deterministic.
#include <algorithm>
#include <type_traits>

#include "et_common.hpp"

namespace et {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

constexpr int kBufDword3 = 0x00020000;           // raw buffer descriptor, word 3 (gfx9)
constexpr uint32_t kOutOfRange = 0x80000000u;    // offset past every num_records: loads return 0
constexpr int kColsPerBlock = 256;               // columns of a block (8 column tiles of 32)
constexpr int kTilesPerBlock = 4;                // expert tiles per block (one per wave) with 8 column tiles a wave
constexpr int kThreads = 4 * kWave;
constexpr int kMaxSplit = 64;
constexpr int kStageTok = 64;                    // tokens per LDS stage (4 k-steps of 16)
constexpr int kRowBytes = kColsPerBlock * 2;     // one token's columns in a stage
constexpr int kStageBytes = kStageTok * kRowBytes;
constexpr int kStages = 3;                       // LDS ring: stage c in buffer c % 3
constexpr int kSegs = kStageBytes / 16 / kThreads;   // 16-byte stage segments per thread (8)
constexpr int kSplitTok = kStageTok;             // a split is a whole number of stages
constexpr int kMemOps = 8 + 2 * kSegs / 4;       // global loads and LDS stores of a wave per k-step

// LDS byte of 16-byte segment s of stage row r.
__host__ __device__ constexpr uint32_t stage_off(int r, int s) { return (uint32_t)(r * kRowBytes + ((s ^ (4 * (r & 3))) << 4)); }

typedef __attribute__((address_space(3))) unsigned char lds_u8_t;

__device__ __forceinline__ uint2 read_tr16(const lds_u8_t* p)
{
    const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
    return __builtin_bit_cast(uint2, v);
}

// dW partial of one (column block, token range).  NC = column tiles per wave
// (8, 4 or 2; see the file comment).
template <int NC>
__global__ __launch_bounds__(kThreads) void router_wgrad_kernel(
    const float* __restrict__ dl, const uint16_t* __restrict__ x, int T, int d, int E, int tok_per_split,
    int ncb, int nsplit, float* __restrict__ part)
{
    __shared__ __attribute__((aligned(16))) unsigned char xs[kStages * kStageBytes];
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = NC == 8 ? (int)blockIdx.z * kTilesPerBlock + wave : NC == 4 ? (wave & 1) : 0;   // expert tile
    const int ct0 = NC == 8 ? 0 : NC == 4 ? 4 * (wave >> 1) : 2 * wave;                            // first column tile
    const int q = lane & 31;
    const int h = lane >> 5;
    // XCD-aware block order: consecutive block ids go to the 8 XCDs in turn,
    // so block id b runs on XCD b % 8.  All column blocks of split ks are put
    // on XCD ks % 8, and the split's dlogits rows are fetched into one L2
    // instead of every XCD's.
    const int b = (int)blockIdx.x;
    const int xcd = b & 7, slot = b >> 3;
    const int cb = slot % ncb;
    const int ks = xcd + 8 * (slot / ncb);
    if (ks >= nsplit) return;                     // whole block: no barrier is skipped by part of it
    const int c0 = cb * kColsPerBlock;
    const int e = n * 32 + q;                     // this lane's expert (A rows)
    const bool active = n * 32 < E;               // wave-uniform
    const int t_begin = ks * tok_per_split;
    const int t_end = min(T, t_begin + tok_per_split);
    const int nstage = (t_end - t_begin + kStageTok - 1) / kStageTok;

    // Per-stage descriptors start at the stage's first token and end at the
    // split's end, so rows past it load as 0 by the range check.  Segment i of
    // this thread is row tid / 32 + 8 i, 16-byte segment tid % 32 (columns
    // past d: out of range); its LDS slot moves by 8 rows (4096 bytes) per i,
    // since (row & 3) does not depend on i.  dlogits: lane (q, h), k-step j,
    // element i is token 16 j + 8 h + i of the stage.
    const int xcol = c0 + 8 * (tid & 31);
    const uint32_t xoff0 = xcol < d ? ((uint32_t)(tid >> 5) * (uint32_t)d + (uint32_t)xcol) * 2u : kOutOfRange;
    const uint32_t xrow8 = (uint32_t)d * 16u;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)xs;
    const uint32_t xlds0 = lds0 + stage_off(tid >> 5, tid & 31);
    const uint32_t doff = e < E ? ((uint32_t)(8 * h) * (uint32_t)E + (uint32_t)e) * 4u : kOutOfRange;
    const uint32_t erow = (uint32_t)E * 4u;
    // Opaque per-stage copies of the lane offsets: the offsets of the
    // individual loads are formed next to each load instead of being kept
    // live across the loop (32 + 8 registers).
    uint32_t xo = xoff0, dof = doff;
    auto refresh = [&]() {
        xo = xoff0;
        dof = doff;
        asm volatile("" : "+v"(xo), "+v"(dof));
    };
    // (read as wave-uniform explicitly: the clamp is formed on the vector unit,
    // and a descriptor field in a vector register costs a loop per load)
    auto nrow_of = [&](int c) {
        return __builtin_amdgcn_readfirstlane(max(0, min(kStageTok, t_end - (t_begin + c * kStageTok))));
    };
    // X fragment of column tile ct0 + cc: lane group gq = lane / 16 reads
    // column 32 (ct0 + cc) + 16 (gq & 1) + lane % 16 of rows
    // 16 j + 8 (gq >> 1) + 0..7 of the k-step.
    const int gq = lane >> 4, i16 = lane & 15;
    const int rrow = 8 * (gq >> 1) + (i16 >> 2);
    uint32_t rb[NC];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
        const int col = 32 * (ct0 + cc) + 16 * (gq & 1) + 4 * (i16 & 3);
        rb[cc] = stage_off(rrow, col >> 3) + (col & 7) * 2;
    }

    f32x16_t acc[NC];
#pragma unroll
    for (int j = 0; j < NC; ++j) acc[j] = f32x16_t{};
    u32x4_t xr[kSegs];        // X of stage c + 2 (to LDS in stage c), then of stage c + 3
    float dv[4][8];           // dlogits of k-step j: stage c until converted (during k-step j - 1), then stage c + 1
    u32x4_t af[2][2];         // A fragments (hi, lo) of k-steps j (af[j & 1]) and j + 1
    u32x4_t bf[2][NC];        // X fragments of k-steps j and j + 1

    auto load_x = [&](int c, u32x4_t (&dst)[kSegs], int i) {
        const __amdgpu_buffer_rsrc_t res = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x + (int64_t)(t_begin + c * kStageTok) * d), (short)0, nrow_of(c) * d * 2, kBufDword3);
        dst[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(res, xo + (uint32_t)i * xrow8, 0, 0));
    };
    auto store_x = [&](int c, const u32x4_t (&src)[kSegs], int i) {
        const uint32_t a = xlds0 + (uint32_t)(c % kStages) * kStageBytes + 4096u * i;
        *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>((uintptr_t)a) = src[i];
    };
    auto load_dl = [&](int c, int j, int i) {
        const __amdgpu_buffer_rsrc_t res = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(dl + (int64_t)(t_begin + c * kStageTok) * E), (short)0, nrow_of(c) * E * 4, kBufDword3);
        dv[j][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(res, dof + (uint32_t)(16 * j + i) * erow, 0, 0));
    };
    // hi/lo split of elements 2 k, 2 k + 1 of a k-step's dlogits
    auto convert = [&](const float (&v)[8], u32x4_t (&a)[2], int k) {
        const uint32_t hw = pack_bf16x2(v[2 * k], v[2 * k + 1]);
        a[0][k] = hw;
        a[1][k] = pack_bf16x2(v[2 * k] - bf16lo(hw), v[2 * k + 1] - bf16hi(hw));
    };
    // Fragment bases of column tile cc in the buffers of stages c and c + 1,
    // formed once a stage; k-step and half are immediate offsets.
    const lds_u8_t* rp[2][NC];
    auto set_bases = [&](int c) {
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
            uint32_t a0 = lds0 + (uint32_t)(c % kStages) * kStageBytes + rb[cc];
            uint32_t a1 = lds0 + (uint32_t)((c + 1) % kStages) * kStageBytes + rb[cc];
            // opaque: keeps the k-step and half offsets in the instructions'
            // offset fields instead of 32 precomputed addresses per stage
            asm volatile("" : "+v"(a0), "+v"(a1));
            rp[0][cc] = (const lds_u8_t*)(uintptr_t)a0;
            rp[1][cc] = (const lds_u8_t*)(uintptr_t)a1;
        }
    };
    // half hf (rows +0 or +4) of the fragment of column tile cc, k-step j of
    // stage c + nx
    auto read_half = [&](int nx, int j, int cc, int hf, u32x4_t& dst) {
        const uint2 v = read_tr16(rp[nx][cc] + 8192 * j + 2048 * hf);
        if (hf == 0) {
            dst[0] = v.x;
            dst[1] = v.y;
        } else {
            dst[2] = v.x;
            dst[3] = v.y;
        }
    };
    auto pin = [&]() { __builtin_amdgcn_sched_barrier(0); };
    auto barrier = [&]() {
        pin();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        pin();
    };
    // memory op m of k-step j of stage c (m < kMemOps): segments 2 j, 2 j + 1
    // of the X of stage c + 2 to its LDS buffer (last read in stage c - 1,
    // before the previous barrier), the same segments of the X of stage c + 3
    // into their registers, then the dlogits of k-step j of stage c + 1 (this
    // k-step's own were split during k-step j - 1)
    auto mem_op = [&](int c, int j, int m, auto act) {
        if (m < 2) store_x(c + 2, xr, 2 * j + m);
        else if (m < 4) load_x(c + 3, xr, 2 * j + m - 2);
        else if (decltype(act)::value) load_dl(c + 1, j, m - 4);
    };

    auto run = [&](auto act) {
        constexpr bool A = decltype(act)::value;
        refresh();
#pragma unroll
        for (int i = 0; i < kSegs; ++i) load_x(0, xr, i);
#pragma unroll
        for (int i = 0; i < kSegs; ++i) store_x(0, xr, i);
#pragma unroll
        for (int i = 0; i < kSegs; ++i) load_x(1, xr, i);
#pragma unroll
        for (int i = 0; i < kSegs; ++i) store_x(1, xr, i);
#pragma unroll
        for (int i = 0; i < kSegs; ++i) load_x(2, xr, i);
        if (A) {
#pragma unroll
            for (int m = 0; m < 32; ++m) load_dl(0, m >> 3, m & 7);
        }
        barrier();
        if (A) {
            set_bases(0);
#pragma unroll
            for (int k = 0; k < 4; ++k) convert(dv[0], af[0], k);
#pragma unroll
            for (int u = 0; u < 2 * NC; ++u) read_half(0, 0, u >> 1, u & 1, bf[0][u >> 1]);
        }
        // stage c: 4 k-steps x 2 NC slots (the parity c & 1, as the second
        // argument's type, gives each parity its own instantiation)
        auto stage = [&](int c, auto /*parity*/) {
            constexpr int S = 8 * NC;
            refresh();
            if (A) set_bases(c);
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int j = s / (2 * NC), u = s % (2 * NC);
                if (A) {
                    const int cc = u % NC;
                    const bf16x8_t av = __builtin_bit_cast(bf16x8_t, af[j & 1][u < NC ? 0 : 1]);
                    acc[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(bf16x8_t, bf[j & 1][cc]),
                                                                      acc[cc], 0, 0, 0);
                    pin();
                    // next k-step: j + 1 of this stage, or k-step 0 of stage c + 1
                    read_half(j == 3 ? 1 : 0, (j + 1) & 3, u >> 1, u & 1, bf[(j + 1) & 1][u >> 1]);
                    if (u % (NC / 2) == 0 && u / (NC / 2) < 4)
                        convert(dv[(j + 1) & 3], af[(j + 1) & 1], u / (NC / 2));
                }
                // memory ops m of this k-step with m * 2 NC / kMemOps == u
#pragma unroll
                for (int m = (u * kMemOps + 2 * NC - 1) / (2 * NC); m < ((u + 1) * kMemOps + 2 * NC - 1) / (2 * NC); ++m)
                    mem_op(c, j, m, act);
                pin();
            }
            barrier();
        };
        for (int c = 0; c < nstage; c += 2) {
            stage(c, std::integral_constant<int, 0>{});
            if (c + 1 < nstage) stage(c + 1, std::integral_constant<int, 1>{});
        }
    };
    if (active) run(std::true_type{});
    else run(std::false_type{});

    // partial tile: lane (q, h) holds column c0 + 32 (ct0 + cc) + q (acc[cc])
    // of expert rows n * 32 + 8 (r / 4) + 4 h + r % 4
    if (!active) return;
    float* pt = part + (int64_t)ks * E * d;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = n * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        if (row < E) {
#pragma unroll
            for (int cc = 0; cc < NC; ++cc) {
                const int col = c0 + 32 * (ct0 + cc) + q;
                if (col < d) pt[(int64_t)row * d + col] = acc[cc][r];
            }
        }
    }
}

__global__ __launch_bounds__(256) void zero_fill_kernel(float* __restrict__ p, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// dW = sum of the KS partials, in split order.
__global__ __launch_bounds__(256) void router_wgrad_reduce_kernel(const float* __restrict__ part, int ks_count,
                                                                  int64_t n4, float* __restrict__ dw)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const f32x4_t* p = reinterpret_cast<const f32x4_t*>(part);
    f32x4_t s = p[i];
    for (int k = 1; k < ks_count; ++k) {
        const f32x4_t v = p[(int64_t)k * n4 + i];
        s[0] += v[0];
        s[1] += v[1];
        s[2] += v[2];
        s[3] += v[3];
    }
    reinterpret_cast<f32x4_t*>(dw)[i] = s;
}

struct WgradPlan {
    int ncb, nt, nz, nc, ks, tok_per_split;
};

// Column tiles per wave (8 from 3 expert tiles up), and splits of the tokens
// so that the grid holds about 256 blocks of 4 waves (one wave per SIMD).
WgradPlan wgrad_plan(int64_t T, int64_t d, int64_t E)
{
    WgradPlan p;
    p.ncb = (int)((d + kColsPerBlock - 1) / kColsPerBlock);
    p.nt = (int)((E + 31) / 32);
    p.nc = p.nt >= 3 ? 8 : p.nt == 2 ? 4 : 2;
    p.nz = p.nc == 8 ? (p.nt + kTilesPerBlock - 1) / kTilesPerBlock : 1;
    const int64_t want = (256 + (int64_t)p.ncb * p.nz - 1) / ((int64_t)p.ncb * p.nz);
    const int64_t max_by_t = std::max<int64_t>(1, (T + kSplitTok - 1) / kSplitTok);
    p.ks = (int)std::max<int64_t>(1, std::min<int64_t>({want, (int64_t)kMaxSplit, max_by_t}));
    const int64_t per = (T + p.ks - 1) / p.ks;
    p.tok_per_split = (int)(((per + kSplitTok - 1) / kSplitTok) * kSplitTok);
    p.ks = (int)std::max<int64_t>(1, (T + p.tok_per_split - 1) / p.tok_per_split);
    return p;
}

}  // namespace

}  // namespace et

using namespace et;

extern "C" size_t et_router_wgrad_workspace_bytes(int64_t num_tokens, int64_t d, int64_t num_experts)
{
    if (num_tokens < 1 || d < 1 || num_experts < 1 || num_experts > ET_MAX_ROUTER_EXPERTS) return 0;
    const WgradPlan p = wgrad_plan(num_tokens, d, num_experts);
    return size_t(p.ks) * size_t(num_experts) * size_t(d) * 4;
}

extern "C" int et_router_wgrad(const float* dlogits, const void* x, int64_t T, int64_t d, int64_t E, float* dw,
                               void* workspace, size_t workspace_bytes, void* stream)
{
    if (T < 0 || T >= (int64_t(1) << 31)) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_wgrad: num_tokens out of range");
    if (E < 1 || E > ET_MAX_ROUTER_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_wgrad: num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_ROUTER_EXPERTS) + "]");
    if (d < 1 || d % 8 != 0 || d >= (int64_t(1) << 22))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_wgrad: d must be a positive multiple of 8 below 2^22");
    if (T * E >= (int64_t(1) << 29) || T * d >= (int64_t(1) << 30))
        return fail(ET_ERR_INVALID_ARGUMENT,
                    "et_router_wgrad: dlogits must be below 2^31 bytes and x below 2^31 bytes");
    if (!dw) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_wgrad: null dw");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t n4 = E * d / 4;
    if (T == 0) {                                // no tokens: dW = 0 (a kernel, so that graph capture can hold it)
        zero_fill_kernel<<<dim3((unsigned)((E * d + 255) / 256)), dim3(256), 0, s>>>(dw, E * d);
        return check_launch("zero_fill_kernel");
    }
    if (!dlogits || !x || !workspace) return fail(ET_ERR_INVALID_ARGUMENT, "et_router_wgrad: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(dw) & 15) ||
        (reinterpret_cast<uintptr_t>(workspace) & 15))
        return fail(ET_ERR_INVALID_ARGUMENT, "et_router_wgrad: x, dw and workspace must be 16-byte aligned");
    const WgradPlan p = wgrad_plan(T, d, E);
    const size_t need = size_t(p.ks) * size_t(E) * size_t(d) * 4;
    if (workspace_bytes < need)
        return fail(ET_ERR_WORKSPACE_TOO_SMALL, "et_router_wgrad: workspace needs " + std::to_string(need) +
                                                    " bytes, got " + std::to_string(workspace_bytes));
    float* part = static_cast<float*>(workspace);
    const unsigned nblk = (unsigned)(p.ncb * ((p.ks + 7) / 8) * 8);   // split groups of 8 (one per XCD)
    const dim3 grid(nblk, 1, (unsigned)p.nz);
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    if (p.nc == 8)
        router_wgrad_kernel<8><<<grid, dim3(kThreads), 0, s>>>(dlogits, xb, (int)T, (int)d, (int)E, p.tok_per_split,
                                                                p.ncb, p.ks, part);
    else if (p.nc == 4)
        router_wgrad_kernel<4><<<grid, dim3(kThreads), 0, s>>>(dlogits, xb, (int)T, (int)d, (int)E, p.tok_per_split,
                                                                p.ncb, p.ks, part);
    else
        router_wgrad_kernel<2><<<grid, dim3(kThreads), 0, s>>>(dlogits, xb, (int)T, (int)d, (int)E, p.tok_per_split,
                                                                p.ncb, p.ks, part);
    if (int rc = check_launch("router_wgrad_kernel")) return rc;
    router_wgrad_reduce_kernel<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s>>>(part, p.ks, n4, dw);
    return check_launch("router_wgrad_reduce_kernel");
}
