// GPU check behind the controller's use of sincosf (turbinator_c_amd/csrc/
// onboard.hip, sin_cos): on gfx950, sincosf(x) returns the same bits as
// sinf(x) and cosf(x) for every float x (all 2^32 bit patterns; NaN results
// compare equal whatever their payload).  Prints "<n> mismatches" and exits
// 0 when the run itself succeeded.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

__global__ void compare_all(unsigned long long *mismatches, unsigned *first) {
    const uint64_t n = 1ull << 32;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float x = __uint_as_float((unsigned)i);
        const float s1 = sinf(x), c1 = cosf(x);
        float s2, c2;
        sincosf(x, &s2, &c2);
        const bool ds = __float_as_uint(s1) != __float_as_uint(s2) && !(s1 != s1 && s2 != s2);
        const bool dc = __float_as_uint(c1) != __float_as_uint(c2) && !(c1 != c1 && c2 != c2);
        if (ds || dc) {
            atomicAdd(mismatches, 1ull);
            atomicMin(first, (unsigned)i);
        }
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
    unsigned long long *mismatches = NULL, count = 0;
    unsigned *first = NULL, first_bits = 0;
    CHECK(hipMalloc((void **)&mismatches, sizeof(*mismatches)));
    CHECK(hipMalloc((void **)&first, sizeof(*first)));
    CHECK(hipMemset(mismatches, 0, sizeof(*mismatches)));
    CHECK(hipMemset(first, 0xff, sizeof(*first)));
    hipLaunchKernelGGL(compare_all, dim3(8192), dim3(256), 0, 0, mismatches, first);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(&count, mismatches, sizeof(count), hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(&first_bits, first, sizeof(first_bits), hipMemcpyDeviceToHost));
    printf("%llu mismatches (first input bits 0x%08x)\n", count, first_bits);
    CHECK(hipFree(mismatches));
    CHECK(hipFree(first));
    return 0;
}
