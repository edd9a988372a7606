// et_router_bwd.hip -- router weight gradient on gfx950:
//     dW[e, c] = sum_t dlogits[t, e] * X[t, c]        (f32 [E, d])
// from the f32 router-logit gradient dlogits [T, E] and the bf16 router input
// X [T, d], on the MFMA units (v_mfma_f32_32x32x16_bf16).
//
// The reduction runs over tokens, which is the outer (row) dimension of both
// operands, so neither loads as MFMA fragments directly (a fragment lane needs
// 8 consecutive k = tokens).  Each lane therefore loads an 8 x 8 block of X --
// 8 tokens x 8 consecutive columns, eight 16-byte loads -- and transposes it in
// registers (v_perm_b32) into 8 B fragments, one per "virtual column tile" j:
// lane q of tile j is column 8 q + j.  dlogits is loaded 8 tokens per lane
// (one f32 per load, 128 contiguous bytes per half-wave) and split into
// hi = bf16(dl) and lo = bf16(dl - hi), two MFMAs each, so dW carries ~16
// more bits of dl than a bf16 GEMM (exact when dl is a bf16 value).
//
// Work split: a block = one wave per 32-expert tile (up to 4; grid z covers
// more), all waves on the same 256 columns and token range (the X block is
// fetched from HBM once and shared through L1/L2).  The token range is split over KS blocks; each
// writes its partial dW tile, and a second kernel sums the KS partials in
// order, so the result is deterministic.
#include <algorithm>

#include "et_common.hpp"

namespace et {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBufDword3 = 0x00020000;           // raw buffer descriptor, word 3 (gfx9)
constexpr uint32_t kOutOfRange = 0x80000000u;    // offset past every num_records: loads return 0
constexpr int kColsPerBlock = 256;               // 32 lanes x 8 consecutive columns
constexpr int kTilesPerBlock = 4;                // expert tiles (waves) per block; grid z covers the rest
constexpr int kMaxSplit = 64;
constexpr int kRing = 2;                         // k-steps of 16 tokens in the load ring

// The 8 x 8 transpose: xr[i] holds token i's columns 0..7 (2 bf16 per dword);
// bf[j] gets column j's tokens 0..7.
__device__ __forceinline__ void transpose8x8(const u32x4_t (&xr)[8], u32x4_t (&bf)[8])
{
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            bf[j][k] = __builtin_amdgcn_perm(xr[2 * k + 1][j >> 1], xr[2 * k][j >> 1], sel);
    }
}

// dW partial of one (column block, token range): wave = expert tile n.
__global__ __launch_bounds__(kTilesPerBlock * kWave) void router_wgrad_kernel(
    const float* __restrict__ dl, const uint16_t* __restrict__ x, int T, int d, int E, int tok_per_split,
    int ncb, int nsplit, float* __restrict__ part)
{
    const int lane = lane_id();
    const int n = (int)blockIdx.z * kTilesPerBlock + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
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
    if (ks >= nsplit) return;
    const int c0 = cb * kColsPerBlock + 8 * q;      // this lane's 8 columns
    const int e = n * 32 + q;                       // this lane's expert (A rows)
    const int t_begin = ks * tok_per_split;
    const int t_end = min(T, t_begin + tok_per_split);

    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0, (int)((int64_t)T * d * 2), kBufDword3);
    const __amdgpu_buffer_rsrc_t dres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(dl), (short)0, (int)((int64_t)T * E * 4), kBufDword3);

    // loads of one k-step (16 tokens from t): rows t + 8 h + i; rows past the
    // split or past T, columns past d and experts past E read as 0
    auto load = [&](int t, u32x4_t (&xr)[8], float (&dv)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int tt = t + 8 * h + i;
            const bool ok = tt < t_end;
            const uint32_t xo = ok && c0 < d ? ((uint32_t)tt * (uint32_t)d + (uint32_t)c0) * 2u : kOutOfRange;
            const uint32_t dlo = ok && e < E ? ((uint32_t)tt * (uint32_t)E + (uint32_t)e) * 4u : kOutOfRange;
            xr[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xres, xo, 0, 0));
            dv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(dres, dlo, 0, 0));
        }
    };

    f32x16_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x16_t{};

    auto compute = [&](const u32x4_t (&xr)[8], const float (&dv)[8]) {
        u32x4_t bf[8];
        transpose8x8(xr, bf);
        u32x4_t ahi, alo;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ahi[k] = pack_bf16x2(dv[2 * k], dv[2 * k + 1]);
            const float r0 = dv[2 * k] - bf16lo(ahi[k]);
            const float r1 = dv[2 * k + 1] - bf16hi(ahi[k]);
            alo[k] = pack_bf16x2(r0, r1);
        }
        const bf16x8_t ah = __builtin_bit_cast(bf16x8_t, ahi), al = __builtin_bit_cast(bf16x8_t, alo);
        // all hi terms, then all lo terms: the two MFMAs on one accumulator are
        // 8 apart, so none waits for the previous one's result
#pragma unroll
        for (int j = 0; j < 8; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, __builtin_bit_cast(bf16x8_t, bf[j]), acc[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, __builtin_bit_cast(bf16x8_t, bf[j]), acc[j], 0, 0, 0);
    };

    // A ring of kRing k-steps: the loads of step s + kRing - 1 are issued
    // before step s is computed.  The loop runs whole groups of kRing steps
    // over the split (its length is a multiple of 16 kRing tokens) with no
    // exit inside, so the accumulators and the ring keep their registers;
    // steps past t_end load zeros and add nothing.
    u32x4_t xr[kRing][8];
    float dv[kRing][8];
#pragma unroll
    for (int p = 0; p < kRing - 1; ++p) load(t_begin + 16 * p, xr[p], dv[p]);
    for (int t = t_begin; t < t_end; t += 16 * kRing) {
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
            __builtin_amdgcn_sched_barrier(0);
            load(t + 16 * (r + kRing - 1), xr[(r + kRing - 1) % kRing], dv[(r + kRing - 1) % kRing]);
            __builtin_amdgcn_sched_barrier(0);
            compute(xr[r], dv[r]);
        }
    }

    // partial tile: lane (q, h) holds columns c0 .. c0 + 7 (acc[0..7]) of
    // expert rows n * 32 + 8 (r / 4) + 4 h + r % 4
    float* pt = part + (int64_t)ks * E * d;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = n * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        if (row < E && c0 < d) {
            float* dst = pt + (int64_t)row * d + c0;
            *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
            *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
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
    int ncb, nt, ks, tok_per_split;
};

// Splits the tokens so that the grid holds about 1024 waves (one per SIMD):
// columns blocks x expert tiles x splits.
WgradPlan wgrad_plan(int64_t T, int64_t d, int64_t E)
{
    WgradPlan p;
    p.ncb = (int)((d + kColsPerBlock - 1) / kColsPerBlock);
    p.nt = (int)((E + 31) / 32);
    const int64_t want = (1024 + (int64_t)p.ncb * p.nt - 1) / ((int64_t)p.ncb * p.nt);
    const int64_t max_by_t = std::max<int64_t>(1, (T + 63) / 64);
    p.ks = (int)std::max<int64_t>(1, std::min<int64_t>({want, (int64_t)kMaxSplit, max_by_t}));
    const int64_t per = (T + p.ks - 1) / p.ks;
    p.tok_per_split = (int)(((per + 16 * kRing - 1) / (16 * kRing)) * (16 * kRing));
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
    const int nz = (p.nt + kTilesPerBlock - 1) / kTilesPerBlock;
    const unsigned nblk = (unsigned)(p.ncb * ((p.ks + 7) / 8) * 8);   // split groups of 8 (one per XCD)
    router_wgrad_kernel<<<dim3(nblk, 1, nz), dim3(std::min(p.nt, kTilesPerBlock) * kWave), 0, s>>>(
        dlogits, static_cast<const uint16_t*>(x), (int)T, (int)d, (int)E, p.tok_per_split, p.ncb, p.ks, part);
    if (int rc = check_launch("router_wgrad_kernel")) return rc;
    router_wgrad_reduce_kernel<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s>>>(part, p.ks, n4, dw);
    return check_launch("router_wgrad_reduce_kernel");
}
