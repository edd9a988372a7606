// et_common.hpp -- device helpers shared by the routing and row kernels of
// libetmoe.so (gfx950, wave64).  Also the host-side error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "etmoe.h"

namespace et {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// host-side status plumbing
// ---------------------------------------------------------------------------

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Returns ET_OK, or ET_ERR_LAUNCH with the HIP error text recorded.
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// bit casts and bf16
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// bf16 -> f32 is a 16-bit shift of the word.
__device__ __forceinline__ float bf16lo(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return u2f(w & 0xffff0000u); }

// f32 -> bf16, round to nearest even; a NaN keeps its sign and top payload
// bits and is forced quiet (bit 6 of the bf16 word).  gfx950's
// v_cvt_pk_bf16_f32 implements exactly this rule: all 2^32 inputs were checked
// against the integer formulation
//     NaN:  (u >> 16) | 0x40      else:  (u + 0x7fff + ((u >> 16) & 1)) >> 16
// with zero differences (denormals included), so the kernels use the single
// instruction, which converts two values at once.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// ---------------------------------------------------------------------------
// specified exp / sigmoid (bit-exact on any IEEE binary32 machine with fma)
// ---------------------------------------------------------------------------

// exp(x) for x <= 0: Cody-Waite reduction with n = rint(x*log2 e), ln2 split
// into an exact high part and a low part, degree-7 Taylor polynomial of exp(r)
// on |r| <= ln2/2 in Horner form with fma, scaled by 2^n through the exponent
// field.  x < -87 gives 0, so no result is subnormal.  The special cases
// (NaN, x < -87) are selected at the end rather than branched around: inside
// a wave those branches diverge and cost more than the polynomial.
__device__ __forceinline__ float exp_nonpos(float x_in)
{
    const bool nan = x_in != x_in;
    const bool under = x_in < -87.0f;
    const float x = (nan || under) ? 0.0f : x_in;
    const float log2e = 1.4426950216293335f;     // 0x3FB8AA3B
    const float ln2_hi = 0.693145751953125f;     // 0x3F317200
    const float ln2_lo = 1.428606765330187e-6f;  // 0x35BFBE8E
    float n = __builtin_rintf(x * log2e);
    float r = __builtin_fmaf(-n, ln2_hi, x);
    r = __builtin_fmaf(-n, ln2_lo, r);
    float p = 1.9841270113829523e-4f;
    p = __builtin_fmaf(p, r, 1.3888889225199819e-3f);
    p = __builtin_fmaf(p, r, 8.333333767950535e-3f);
    p = __builtin_fmaf(p, r, 4.16666679084301e-2f);
    p = __builtin_fmaf(p, r, 1.666666716337204e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int ni = (int)n;
    const float v = p * u2f((uint32_t)(ni + 127) << 23);
    return nan ? x_in : (under ? 0.0f : v);
}

// sigmoid(l): l >= 0 -> 1/(1+exp(-l)); l < 0 -> exp(l)/(1+exp(l)); NaN stays NaN.
// Both cases share z = exp(-|l|) and one division, (l >= 0 ? 1 : z) / (1 + z),
// so a wave whose lanes straddle 0 evaluates one exp and one division rather
// than both sides of a branch; the bits are those of the two-case form.  The
// division is IEEE correctly rounded (HIP's default for binary32).
__device__ __forceinline__ float sigmoid(float l)
{
    const float z = exp_nonpos(-__builtin_fabsf(l));
    const float num = (l >= 0.0f) ? 1.0f : z;
    const float s = num / (1.0f + z);
    return (l != l) ? l : s;
}

// ---------------------------------------------------------------------------
// wave helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// popcount(mask & lanes-below-me)
__device__ __forceinline__ int rank_below(uint64_t mask)
{
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ int wave_sum_int(int v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// DPP move of a float: lane i takes src from the lane CTRL selects; lanes
// whose source is out of the row, or whose row is not in ROW_MASK, take 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_mov(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the wave's 64 lanes with DPP moves only (no LDS round trips):
// pairs, quads, row_shr 4 and 8 leave each 16-lane row's total in its lane 15;
// row_bcast 15 and 31 then carry row totals up to lane 63.  The order of the
// additions is fixed, so the result is deterministic.  Returned wave-uniform.
__device__ __forceinline__ float wave_sum_dpp(float v)
{
    v += dpp_mov<0xB1>(v);        // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);        // quad_perm [2,3,0,1]
    v += dpp_mov<0x114>(v);       // row_shr:4
    v += dpp_mov<0x118>(v);       // row_shr:8
    v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), kWave - 1));
}

// The same reduction in binary64: each DPP move carries the two 32-bit halves
// of a double.  The order of the additions is that of wave_sum_dpp.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_mov_f64(double x)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xf,
                                                              false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double wave_sum_dpp_f64(double v)
{
    v += dpp_mov_f64<0xB1>(v);
    v += dpp_mov_f64<0x4E>(v);
    v += dpp_mov_f64<0x114>(v);
    v += dpp_mov_f64<0x118>(v);
    v += dpp_mov_f64<0x142, 0xA>(v);
    v += dpp_mov_f64<0x143, 0xC>(v);
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, kWave - 1);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), kWave - 1);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Max over the wave's 64 lanes of an unsigned key, with the DPP moves of
// wave_sum_dpp (lanes outside a move's source row take 0, the identity of an
// unsigned max).  Returned wave-uniform.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_mov_u32(uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xf, false);
}

__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v)
{
    v = max(v, dpp_mov_u32<0xB1>(v));
    v = max(v, dpp_mov_u32<0x4E>(v));
    v = max(v, dpp_mov_u32<0x114>(v));
    v = max(v, dpp_mov_u32<0x118>(v));
    v = max(v, dpp_mov_u32<0x142, 0xA>(v));
    v = max(v, dpp_mov_u32<0x143, 0xC>(v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, kWave - 1);
}

// Inclusive prefix sum across the wave.
__device__ __forceinline__ int wave_incl_scan(int v)
{
    const int lane = lane_id();
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        int o = __shfl_up(v, off, kWave);
        if (lane >= off) v += o;
    }
    return v;
}

}  // namespace et
