// rcp_check.hip - exhaustive check behind q8_1_rcp (tinystrata_amd/csrc/tsx_device.hpp), run on the GPU by
// tests/test_numerics.py through tinystrata_amd/libtsx_numerics_check.so: for every float d in [2^-100, 2^100], the
// hardware reciprocal with one fma Newton step, fma(fma(-d, r0, 1), r0, r0), equals the IEEE quotient 1 / d.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {
__global__ void rcp_newton_kernel(unsigned long long* bad) {
    const uint32_t lo = 0x0D800000u, hi = 0x71800000u;  // the bit patterns of 2^-100 and 2^100
    unsigned int mine = 0;
    for (uint64_t b = lo + (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; b <= hi; b += (uint64_t) gridDim.x * blockDim.x) {
        const float d = __uint_as_float((uint32_t) b);
        const float r0 = __builtin_amdgcn_rcpf(d);
        const float r1 = __builtin_fmaf(__builtin_fmaf(-d, r0, 1.0f), r0, r0);
        mine += __float_as_uint(r1) != __float_as_uint(1.0f / d) ? 1u : 0u;
    }
    if (mine) atomicAdd(bad, (unsigned long long) mine);
}
}  // namespace

extern "C" int tsx_check_rcp_newton(unsigned long long* mismatches) {
    unsigned long long* d = nullptr;
    if (hipMalloc(&d, sizeof(*d)) != hipSuccess) return 1;
    int rc = hipMemset(d, 0, sizeof(*d)) != hipSuccess;
    if (!rc) {
        rcp_newton_kernel<<<2048, 256>>>(d);
        rc = hipGetLastError() != hipSuccess;
    }
    if (!rc) rc = hipMemcpy(mismatches, d, sizeof(*d), hipMemcpyDeviceToHost) != hipSuccess;
    (void) hipFree(d);
    return rc;
}
