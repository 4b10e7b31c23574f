// GPU check behind ob_atan2 (turbinator_c_amd/csrc/onboard.hip): on gfx950,
// (float)atan2((double)y, (double)x) is the correctly rounded atan2 (equal to
// the host's double atan2 rounded once) on 8.4e6 arguments, and it equals the
// host libm's atan2f, the function the onboard oracle calls, on the
// arguments that reach the controller's angle-wrap discontinuity exactly:
// equal and opposite components (+-pi/4, +-3pi/4), zero components (0,
// +-pi/2, +-pi) and results within a few ulps of +-pi.  Elsewhere (near
// +-pi/2 with a nonzero x, random pairs) the host atan2f is itself often an
// ulp from the correctly rounded value; those differences are counted but
// move the angles continuously.
// Prints "<n> checked, <a> differ from double atan2, <m> exact-angle
// arguments, <b> differ from atan2f, <c> other arguments differ from atan2f"
// and exits 0 when the run itself succeeded.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

__global__ void eval(const float *y, const float *x, float *out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = (float)atan2((double)y[i], (double)x[i]);
}

#define CHECK(call)                                                                 \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            printf("%s failed: %s\n", #call, hipGetErrorString(e_));                \
            return 1;                                                               \
        }                                                                           \
    } while (0)

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static uint32_t next32(void) {  // xorshift64*
    rng ^= rng >> 12;
    rng ^= rng << 25;
    rng ^= rng >> 27;
    return (uint32_t)((rng * 2685821657736338717ull) >> 32);
}
static float float_of(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

int main(void) {
    const size_t cap = 1u << 23;
    float *hy = (float *)malloc(cap * sizeof(float)), *hx = (float *)malloc(cap * sizeof(float));
    float *hr = (float *)malloc(cap * sizeof(float));
    size_t n = 0, exact_lo = 0, exact_hi = 0;
#define PUSH(Y, X)                     \
    do {                               \
        if (n < cap) {                 \
            hy[n] = (Y);               \
            hx[n] = (X);               \
            ++n;                       \
        }                              \
    } while (0)
    const float mags[] = {0.0f, 1e-30f, 1e-7f, 0.5f, 1.0f, 2.0f, 7.5f, 1000.0f, 3e38f};
    const int nm = (int)(sizeof mags / sizeof mags[0]);
    for (int i = 0; i < nm; ++i)
        for (int j = 0; j < nm; ++j)
            for (int s = 0; s < 4; ++s) PUSH((s & 1 ? -1.0f : 1.0f) * mags[i], (s & 2 ? -1.0f : 1.0f) * mags[j]);
    exact_lo = n;
    for (int k = 0; k < 200000; ++k) {  // equal and opposite magnitudes
        const float a = float_of(0x00800000u + next32() % 0x7e800000u);
        for (int s = 0; s < 4; ++s) PUSH((s & 1 ? -a : a), (s & 2 ? -a : a));
        PUSH(0.0f, -a);
        PUSH(-0.0f, -a);
        PUSH(a, 0.0f);
        PUSH(-a, -0.0f);
    }
    for (int k = 0; k < 1000000; ++k) {  // near +-pi
        const float x = float_of(0x3b800000u + next32() % 0x05800000u);  // [2^-8, 8)
        const float t = ldexpf(1.0f + (float)(next32() & 0xffff) / 65536.0f, -(int)(next32() % 40) - 18);
        PUSH((next32() & 1 ? -t : t) * x, -x);
    }
    exact_hi = n;
    for (int k = 0; k < 1000000; ++k) {  // near 0 and near +-pi/2
        const float x = float_of(0x3b800000u + next32() % 0x05800000u);
        const float t = ldexpf(1.0f + (float)(next32() & 0xffff) / 65536.0f, -(int)(next32() % 40) - 18);
        const float y = (next32() & 1 ? -t : t) * x;
        PUSH(y, x);
        PUSH(-x, y);
    }
    while (n < cap) {  // random finite pairs
        const uint32_t a = next32(), b = next32();
        if ((a & 0x7f800000u) == 0x7f800000u || (b & 0x7f800000u) == 0x7f800000u) continue;
        PUSH(float_of(a), float_of(b));
    }
    float *dy = NULL, *dx = NULL, *dr = NULL;
    CHECK(hipMalloc((void **)&dy, n * sizeof(float)));
    CHECK(hipMalloc((void **)&dx, n * sizeof(float)));
    CHECK(hipMalloc((void **)&dr, n * sizeof(float)));
    CHECK(hipMemcpy(dy, hy, n * sizeof(float), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dx, hx, n * sizeof(float), hipMemcpyHostToDevice));
    hipLaunchKernelGGL(eval, dim3(4096), dim3(256), 0, 0, dy, dx, dr, n);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(hr, dr, n * sizeof(float), hipMemcpyDeviceToHost));
    size_t vs_d = 0, exact_f = 0, other_f = 0;
    for (size_t i = 0; i < n; ++i) {
        const float f = atan2f(hy[i], hx[i]), d = (float)atan2((double)hy[i], (double)hx[i]);
        uint32_t ub, uf, ud;
        memcpy(&ub, &hr[i], 4);
        memcpy(&uf, &f, 4);
        memcpy(&ud, &d, 4);
        const bool exact = i >= exact_lo && i < exact_hi;
        if (ub != ud && vs_d < 3) printf("y %a x %a device %a double %a\n", hy[i], hx[i], hr[i], d);
        if (ub != uf && exact && exact_f < 3)
            printf("y %a x %a device %a atan2f %a\n", hy[i], hx[i], hr[i], f);
        vs_d += ub != ud;
        exact_f += ub != uf && exact;
        other_f += ub != uf && !exact;
    }
    printf("%zu checked, %zu differ from double atan2, %zu exact-angle arguments, %zu differ "
           "from atan2f, %zu other arguments differ from atan2f\n",
           n, vs_d, exact_hi - exact_lo, exact_f, other_f);
    CHECK(hipFree(dy));
    CHECK(hipFree(dx));
    CHECK(hipFree(dr));
    free(hy);
    free(hx);
    free(hr);
    return 0;
}
