// et_swiglu.hip -- the SwiGLU activation of the expert FFN and its backward,
// element-wise over the routed slots (gfx950):
//
//   forward   h[s, j]  = (g * sigmoid(g)) * u,                 g = gu[s, j], u = gu[s, F + j]
//   backward  dgu[s, j]     = (dh * u) * (sigmoid(g) * (1 + g * (1 - sigmoid(g))))
//             dgu[s, F + j] = dh * (g * sigmoid(g)),           dh = dh[s, j]
//
// for s below min(expert_offsets[E], slot_capacity), j < F; bf16 in and out,
// binary32 arithmetic, every operation separately rounded in the order written
// (no contraction), the sigmoid the routing uses.  gu is the gate/up
// projection's output [cap, 2F] (gate rows of the weight first), as the plain
// expert GEMM writes it: a training forward keeps it for the backward, where
// the GEMM's fused SwiGLU epilogue (the inference form) writes h alone.
//
// Both kernels stream HBM once: 6F bytes per slot forward, 10F backward.  A
// thread takes 8 hidden units of one slot (16-byte loads of g, u and dh), a
// grid-stride loop walks slot-major, and the slot count is read on the device,
// so the launch does not depend on the routing (no host synchronisation).
#include <algorithm>

#include "et_common.hpp"

namespace et {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

__device__ __forceinline__ float silu_grad_factor(float g, float s)
{
    // d/dg (g * sigmoid(g)) = sigmoid(g) * (1 + g * (1 - sigmoid(g)))
    const float t = 1.0f - s;
    const float q = g * t;
    const float r = 1.0f + q;
    return s * r;
}

template <bool BWD>
__global__ __launch_bounds__(kThreads) void swiglu_kernel(const uint16_t* __restrict__ gu,
                                                           const uint16_t* __restrict__ dh,
                                                           uint16_t* __restrict__ out,
                                                           const int32_t* __restrict__ expert_offsets, int E,
                                                           int64_t cap, int F)
{
    const int64_t n = min<int64_t>(max<int64_t>(expert_offsets[E], 0), cap);
    const int vpr = F >> 3;                              // 8-unit vectors per slot
    // flat index idx = s * vpr + v, advanced by the grid's thread count: the
    // (s, v) pair is stepped without a division per element
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    const int64_t start = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t ds = stride / vpr;
    const int dv = (int)(stride - ds * vpr);
    int64_t s = start / vpr;
    int v = (int)(start - s * vpr);
    for (; s < n; s += ds, v += dv, s += v >= vpr ? 1 : 0, v -= v >= vpr ? vpr : 0) {
        const int j = v * 8;
        const uint16_t* grow = gu + s * (2 * (int64_t)F);
        const u32x4_t gv = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(grow + j));
        const u32x4_t uv = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(grow + F + j));
        if constexpr (!BWD) {
            u32x4_t hv;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float g0 = bf16lo(gv[w]), g1 = bf16hi(gv[w]);
                const float h0 = (g0 * sigmoid(g0)) * bf16lo(uv[w]);
                const float h1 = (g1 * sigmoid(g1)) * bf16hi(uv[w]);
                hv[w] = pack_bf16x2(h0, h1);
            }
            __builtin_nontemporal_store(hv, reinterpret_cast<u32x4_t*>(out + s * (int64_t)F + j));
        } else {
            const u32x4_t dv = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(dh + s * (int64_t)F + j));
            u32x4_t dg, du;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                float r[2][2];
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const float g = p ? bf16hi(gv[w]) : bf16lo(gv[w]);
                    const float u = p ? bf16hi(uv[w]) : bf16lo(uv[w]);
                    const float d = p ? bf16hi(dv[w]) : bf16lo(dv[w]);
                    const float sg = sigmoid(g);
                    r[0][p] = (d * u) * silu_grad_factor(g, sg);
                    r[1][p] = d * (g * sg);
                }
                dg[w] = pack_bf16x2(r[0][0], r[0][1]);
                du[w] = pack_bf16x2(r[1][0], r[1][1]);
            }
            uint16_t* orow = out + s * (2 * (int64_t)F);
            __builtin_nontemporal_store(dg, reinterpret_cast<u32x4_t*>(orow + j));
            __builtin_nontemporal_store(du, reinterpret_cast<u32x4_t*>(orow + F + j));
        }
    }
}

int launch_swiglu(const char* fn, bool bwd, const void* gu, const void* dh, int64_t F,
                  const int32_t* expert_offsets, int64_t E, int64_t slot_capacity, void* out, void* stream)
{
    if (E < 1 || E > ET_MAX_EXPERTS)
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": num_experts must be in [1, " +
                                                 std::to_string(ET_MAX_EXPERTS) + "]");
    if (F < 8 || F % 8 != 0 || F >= (int64_t(1) << 28))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": F must be a positive multiple of 8 below 2^28");
    if (slot_capacity < 0 || slot_capacity >= (int64_t(1) << 31))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": slot_capacity out of range");
    if (slot_capacity == 0) return ET_OK;
    if (!gu || !expert_offsets || !out || (bwd && !dh))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": null pointer");
    if ((reinterpret_cast<uintptr_t>(gu) & 15) || (reinterpret_cast<uintptr_t>(out) & 15) ||
        (reinterpret_cast<uintptr_t>(dh) & 15))
        return fail(ET_ERR_INVALID_ARGUMENT, std::string(fn) + ": gu, dh and the output must be 16-byte aligned");
    const int64_t vecs = slot_capacity * (F / 8);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    const int64_t blocks = std::min<int64_t>((vecs + kThreads - 1) / kThreads, (int64_t)cus * 8);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (bwd)
        swiglu_kernel<true><<<dim3((unsigned)blocks), dim3(kThreads), 0, s>>>(
            static_cast<const uint16_t*>(gu), static_cast<const uint16_t*>(dh), static_cast<uint16_t*>(out),
            expert_offsets, (int)E, slot_capacity, (int)F);
    else
        swiglu_kernel<false><<<dim3((unsigned)blocks), dim3(kThreads), 0, s>>>(
            static_cast<const uint16_t*>(gu), nullptr, static_cast<uint16_t*>(out), expert_offsets, (int)E,
            slot_capacity, (int)F);
    return check_launch(fn);
}

}  // namespace
}  // namespace et

using namespace et;

extern "C" int et_swiglu_fwd(const void* gu, int64_t F, const int32_t* expert_offsets, int64_t num_experts,
                             int64_t slot_capacity, void* h, void* stream)
{
    return launch_swiglu("et_swiglu_fwd", false, gu, nullptr, F, expert_offsets, num_experts, slot_capacity, h,
                         stream);
}

extern "C" int et_swiglu_bwd(const void* gu, const void* dh, int64_t F, const int32_t* expert_offsets,
                             int64_t num_experts, int64_t slot_capacity, void* dgu, void* stream)
{
    return launch_swiglu("et_swiglu_bwd", true, gu, dh, F, expert_offsets, num_experts, slot_capacity, dgu,
                         stream);
}
