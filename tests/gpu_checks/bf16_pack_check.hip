// bf16_pack_check.hip -- TEST INFRASTRUCTURE (built into libbf16check.so by
// __graft_entry__.build(); loaded only by tests/test_gpu_bf16_pack.py).
//
// Exhaustive check that the product's f32 -> bf16 packing (et::pack_bf16x2 in
// peer-review-agents_amd/csrc/et_common.hpp, gfx950's v_cvt_pk_bf16_f32) equals
// the specified rounding rule for every one of the 2^32 binary32 inputs.  The
// rule is written here with integer operations only, on the input's bits:
//     NaN:       (u >> 16) | 0x0040          (sign and top payload kept, quiet)
//     otherwise: (u + 0x7fff + ((u >> 16) & 1)) >> 16   (round to nearest even)
#include "../../peer-review-agents_amd/csrc/et_common.hpp"

namespace {

__device__ __forceinline__ uint32_t rule_bf16(uint32_t u)
{
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x0040u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Each thread checks the pair of inputs (2i, 2i + 1) of its launch's range.
__global__ __launch_bounds__(256) void pack_check_kernel(uint64_t base, unsigned long long* mismatches,
                                                         unsigned int* first_bad)
{
    const uint64_t i = base + ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 2;
    const uint32_t u0 = (uint32_t)i, u1 = (uint32_t)(i + 1);
    const uint32_t got = et::pack_bf16x2(__uint_as_float(u0), __uint_as_float(u1));
    const uint32_t want = rule_bf16(u0) | (rule_bf16(u1) << 16);
    if (got != want) {
        atomicAdd(mismatches, 1ull);
        atomicMin(first_bad, u0);
    }
}

}  // namespace

// Runs the check over all 2^32 inputs on the current device and stream 0.
// Returns 0 and fills *mismatches (pairs that differ) and *first_bad (lowest
// differing input of a pair, 0xffffffff if none); a negative value on a HIP error
// (-1000 - hipError_t for a failed allocation).
extern "C" int bf16_pack_check(unsigned long long* mismatches, unsigned int* first_bad)
{
    unsigned long long* d_mis = nullptr;
    unsigned int* d_first = nullptr;
    hipError_t e = hipMalloc(&d_mis, sizeof(*d_mis));
    if (e != hipSuccess) return -1000 - (int)e;
    e = hipMalloc(&d_first, sizeof(*d_first));
    if (e != hipSuccess) { (void)hipFree(d_mis); return -1000 - (int)e; }
    const unsigned long long zero = 0;
    const unsigned int none = 0xffffffffu;
    int rc = 0;
    if (hipMemcpy(d_mis, &zero, sizeof(zero), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d_first, &none, sizeof(none), hipMemcpyHostToDevice) != hipSuccess)
        rc = -2;
    const uint64_t per_launch = uint64_t(1) << 30;   // inputs per launch: 2^29 threads
    for (uint64_t base = 0; rc == 0 && base < (uint64_t(1) << 32); base += per_launch) {
        pack_check_kernel<<<dim3((unsigned)(per_launch / 2 / 256)), dim3(256)>>>(base, d_mis, d_first);
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = -3;
    }
    if (rc == 0 && (hipMemcpy(mismatches, d_mis, sizeof(*mismatches), hipMemcpyDeviceToHost) != hipSuccess ||
                    hipMemcpy(first_bad, d_first, sizeof(*first_bad), hipMemcpyDeviceToHost) != hipSuccess))
        rc = -4;
    (void)hipFree(d_mis);
    (void)hipFree(d_first);
    return rc;
}
