// GPU check behind the actor entry's inverse-range channel
// (turbinator_c_amd/csrc/recip_range.h): on gfx950, recip_range(y) equals the
// IEEE quotient 1.0f / y (this file is built with correctly rounded division)
// and the double quotient rounded once, (float)(1.0 / (double)y), for every
// float y in [0.2, 30].  Prints "<n> checked, <a> differ from the IEEE
// quotient, <b> differ from the double quotient" and exits 0 when the run
// itself succeeded.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../turbinator_c_amd/csrc/recip_range.h"

__global__ void compare_range(unsigned lo, unsigned hi, unsigned long long *counts) {
    for (unsigned i = lo + blockIdx.x * blockDim.x + threadIdx.x; i <= hi;
         i += gridDim.x * blockDim.x) {
        const float y = __uint_as_float(i);
        const unsigned got = __float_as_uint(recip_range(y));
        atomicAdd(&counts[0], 1ull);
        if (got != __float_as_uint(1.0f / y)) atomicAdd(&counts[1], 1ull);
        if (got != __float_as_uint((float)(1.0 / (double)y))) atomicAdd(&counts[2], 1ull);
    }
}

#define CHECK(call)                                                                 \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            printf("%s failed: %s\n", #call, hipGetErrorString(e_));                \
            return 1;                                                               \
        }                                                                           \
    } while (0)

int main(void) {
    // 0x3e4ccccd is 0.2f and 0x41f00000 is 30.0f; the grid stride (2^21)
    // keeps i + stride below 2^32, so the loop ends at hi.
    const unsigned lo = 0x3e4ccccdu, hi = 0x41f00000u;
    unsigned long long *counts = NULL, h[3] = {0, 0, 0};
    CHECK(hipMalloc((void **)&counts, sizeof(h)));
    CHECK(hipMemset(counts, 0, sizeof(h)));
    hipLaunchKernelGGL(compare_range, dim3(8192), dim3(256), 0, 0, lo, hi, counts);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(h, counts, sizeof(h), hipMemcpyDeviceToHost));
    printf("%llu checked, %llu differ from the IEEE quotient, %llu differ from the double "
           "quotient\n", h[0], h[1], h[2]);
    CHECK(hipFree(counts));
    return 0;
}
