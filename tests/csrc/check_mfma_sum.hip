// GPU check behind the compact actor's error analysis (turbinator_c_amd/csrc/
// sac_actor.hip): how one v_mfma_f32_16x16x32_f16 instruction sums its 32
// products and the accumulator on gfx950.
//
// Deterministic blocks (one product term set per output row i):
//   same group   +2^20, 2^(8-i), -2^20 at k = 0, 1, 2 (one lane's 8 k values)
//   across       +2^20 at k = 0, -2^20 at k = 8, 2^(8-i) at k = 16
//   second half  +2^20 at k = 0, -2^20 at k = 1, 2^(8-i) at k = 5 (the same
//                eight k values, another group of four)
//   rounding     2^20 + (i+1) 2^-6 + j 2^-10 at k = 0, 1, 2
// Random blocks: fp16 operands of either sign in [2^-6, 2^6], fp32
// accumulators in [2^-6, 2^12].  Every product and accumulator is then a
// multiple of 2^-32 of at most 2^12, so every partial sum of an output (32
// products and the accumulator) is a multiple of 2^-32 below 2^18: exact in
// double.
//
// Prints one line
//   "<k> smallest-kept-exponent-same-group <a> kept-across <h> kept-half
//    <t> truncated <b> above-exact <n> random max <m> mean <q> toward-zero <z>"
// where k is the smallest e for which 2^e survived beside the cancelling
// 2^20 pair in one group, a and h the number of across-group and
// second-half rows that kept their small product (of 16 each), t the rounding outputs (of 256) below the
// nearest-even float of the exact sum, b those above the exact sum, m and q
// the maximum and mean |error| / (u sum|p|) over the random outputs
// (u = 2^-24, the sum over the products and the accumulator), and z the
// fraction of nonzero errors that point toward zero.  Exits 0 when the run
// itself succeeded.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Block e: A[e] 16x32, B[e] 32x16, C[e] and D[e] 16x16, row-major.  One wave
// per block; lane l holds A row l%16 and B column l%16 at k = 8(l/16)..+7,
// and D rows 4(l/16)..+3 of column l%16.
__global__ __launch_bounds__(64) void mfma_blocks(const _Float16 *A, const _Float16 *B,
                                                  const float *C, float *D, int blocks) {
    const int e = blockIdx.x, l = threadIdx.x, r = l % 16, g = l / 16;
    if (e >= blocks) return;
    f16x8 a, b;
    for (int t = 0; t < 8; ++t) {
        a[t] = A[e * 512 + r * 32 + 8 * g + t];
        b[t] = B[e * 512 + (8 * g + t) * 16 + r];
    }
    f32x4 c;
    for (int v = 0; v < 4; ++v) c[v] = C[e * 256 + (4 * g + v) * 16 + r];
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    for (int v = 0; v < 4; ++v) D[e * 256 + (4 * g + v) * 16 + r] = c[v];
}

#define CHECK(call)                                                                 \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));       \
            return 1;                                                               \
        }                                                                           \
    } while (0)

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static double uniform01(void) {  // splitmix64
    uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (double)(z >> 11) * 0x1p-53;
}
static double signed_log_uniform(double lo, double hi) {
    const double m = exp2(lo + (hi - lo) * uniform01());
    return uniform01() < 0.5 ? -m : m;
}

enum { kFixed = 4, kRandom = 1024, kBlocks = kFixed + kRandom };

int main(void) {
    const size_t na = (size_t)kBlocks * 512, nc = (size_t)kBlocks * 256;
    _Float16 *A = (_Float16 *)calloc(na, sizeof(_Float16));
    _Float16 *B = (_Float16 *)calloc(na, sizeof(_Float16));
    float *C = (float *)calloc(nc, sizeof(float));
    float *D = (float *)calloc(nc, sizeof(float));
    if (!A || !B || !C || !D) return 1;
    const float big = 1024.0f;  // big * big = 2^20
    // Blocks 0, 1, 3: +2^20, 2^(8-i), -2^20 in one group / across groups /
    // in the other half of one lane's eight k values.
    for (int e : {0, 1, 3}) {
        const int kb = 0, ks = e == 0 ? 1 : e == 1 ? 16 : 5, kn = e == 0 ? 2 : e == 1 ? 8 : 1;
        for (int i = 0; i < 16; ++i) {
            A[e * 512 + i * 32 + kb] = (_Float16)big;
            A[e * 512 + i * 32 + ks] = (_Float16)ldexpf(1.0f, 8 - i);
            A[e * 512 + i * 32 + kn] = (_Float16)(-big);
        }
        for (int j = 0; j < 16; ++j) {
            B[e * 512 + kb * 16 + j] = (_Float16)big;
            B[e * 512 + ks * 16 + j] = (_Float16)1.0f;
            B[e * 512 + kn * 16 + j] = (_Float16)big;
        }
    }
    // Block 2: 2^20 + (i+1) 2^-6 + j 2^-10 (the sum's ulp is 2^-3).
    for (int i = 0; i < 16; ++i) {
        A[2 * 512 + i * 32 + 0] = (_Float16)big;
        A[2 * 512 + i * 32 + 1] = (_Float16)((float)(i + 1) * 0x1p-6f);
        A[2 * 512 + i * 32 + 2] = (_Float16)0x1p-10f;
    }
    for (int j = 0; j < 16; ++j) {
        B[2 * 512 + 0 * 16 + j] = (_Float16)big;
        B[2 * 512 + 1 * 16 + j] = (_Float16)1.0f;
        B[2 * 512 + 2 * 16 + j] = (_Float16)(float)j;
    }
    for (int e = kFixed; e < kBlocks; ++e) {
        for (int k = 0; k < 512; ++k) {
            A[e * 512 + k] = (_Float16)signed_log_uniform(-6.0, 6.0);
            B[e * 512 + k] = (_Float16)signed_log_uniform(-6.0, 6.0);
        }
        for (int k = 0; k < 256; ++k) C[e * 256 + k] = (float)signed_log_uniform(-6.0, 12.0);
    }

    _Float16 *dA, *dB;
    float *dC, *dD;
    CHECK(hipMalloc(&dA, na * sizeof(_Float16)));
    CHECK(hipMalloc(&dB, na * sizeof(_Float16)));
    CHECK(hipMalloc(&dC, nc * sizeof(float)));
    CHECK(hipMalloc(&dD, nc * sizeof(float)));
    CHECK(hipMemcpy(dA, A, na * sizeof(_Float16), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dB, B, na * sizeof(_Float16), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dC, C, nc * sizeof(float), hipMemcpyHostToDevice));
    mfma_blocks<<<kBlocks, 64>>>(dA, dB, dC, dD, kBlocks);
    CHECK(hipGetLastError());
    CHECK(hipMemcpy(D, dD, nc * sizeof(float), hipMemcpyDeviceToHost));

    // Exact sums in double (exact for every block here, see the header).
    #define EXACT(e, i, j, out)                                                          \
        do {                                                                             \
            double s_ = C[(e) * 256 + (i) * 16 + (j)], m_ = fabs(s_);                    \
            for (int k_ = 0; k_ < 32; ++k_) {                                            \
                const double p_ = (double)(float)A[(e) * 512 + (i) * 32 + k_] *          \
                                  (double)(float)B[(e) * 512 + k_ * 16 + (j)];           \
                s_ += p_;                                                                \
                m_ += fabs(p_);                                                          \
            }                                                                            \
            (out)[0] = s_;                                                               \
            (out)[1] = m_;                                                               \
        } while (0)

    int smallest_kept = 99;
    for (int i = 0; i < 16; ++i)
        if (D[0 * 256 + i * 16 + 0] == ldexpf(1.0f, 8 - i)) smallest_kept = 8 - i;
    int kept_across = 0, kept_half = 0;
    for (int i = 0; i < 16; ++i) {
        kept_across += D[1 * 256 + i * 16 + 0] == ldexpf(1.0f, 8 - i);
        kept_half += D[3 * 256 + i * 16 + 0] == ldexpf(1.0f, 8 - i);
    }
    int truncated = 0, above = 0;
    for (int i = 0; i < 16; ++i)
        for (int j = 0; j < 16; ++j) {
            double x[2];
            EXACT(2, i, j, x);
            const float got = D[2 * 256 + i * 16 + j];
            truncated += got < (float)x[0];
            above += (double)got > x[0];
        }
    double worst = 0.0, total = 0.0;
    long nonzero = 0, toward_zero = 0, outputs = 0;
    for (int e = kFixed; e < kBlocks; ++e)
        for (int i = 0; i < 16; ++i)
            for (int j = 0; j < 16; ++j) {
                double x[2];
                EXACT(e, i, j, x);
                const double err = (double)D[e * 256 + i * 16 + j] - x[0];
                const double rel = fabs(err) / (0x1p-24 * x[1]);
                worst = rel > worst ? rel : worst;
                total += rel;
                ++outputs;
                if (err != 0.0) {
                    ++nonzero;
                    toward_zero += (err < 0.0) == (x[0] > 0.0);
                }
            }
    printf("%d smallest-kept-exponent-same-group %d kept-across %d kept-half %d truncated "
           "%d above-exact %ld random max %.3f mean %.3f toward-zero %.3f\n",
           smallest_kept, kept_across, kept_half, truncated, above, outputs, worst, total / outputs,
           nonzero ? (double)toward_zero / nonzero : 0.0);
    return 0;
}
