/* The onboard kernels' atan2 near +-pi: for x < 0 and |y| <= 1e-6 |x| whose
 * atan2f lies within the kernels' threshold (|result| >= 3.1415920f),
 * sign(y) (pi - |y / x|) formed in double and rounded once must equal the
 * correctly rounded atan2 ((float)atan2 in double) and the host libm's
 * atan2f.  x runs over [-8, -2^-8] (every 4,099th float), y over every binade
 * down to the smallest subnormal with 31 mantissas each, both signs.
 * Prints "<count> checked, <n> differ from double atan2, <m> from atan2f". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float float_of(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static float near_pi(float y, float x) {
    const double t = fabs((double)y / (double)x);
    return copysignf((float)(3.14159265358979323846 - t), y);
}

int main(void) {
    long checked = 0, vs_double = 0, vs_libm = 0;
    for (uint32_t xb = 0xbb800000u; xb <= 0xc1000000u; xb += 4099) {
        const float x = float_of(xb);
        for (int e = -149; e <= -1; ++e) {
            for (int k = 0; k < 31; ++k) {
                const float ay = ldexpf(1.0f + (float)k / 31.0f, e);
                if (ay > 1e-6f * fabsf(x)) break;
                for (int s = 0; s < 2; ++s) {
                    const float y = s ? -ay : ay;
                    const float libm = atan2f(y, x);
                    if (!(fabsf(libm) >= 3.1415920f)) continue;
                    const float mine = near_pi(y, x);
                    ++checked;
                    vs_double += mine != (float)atan2((double)y, (double)x);
                    vs_libm += mine != libm;
                }
            }
        }
    }
    printf("%ld checked, %ld differ from double atan2, %ld from atan2f\n", checked, vs_double,
           vs_libm);
    return vs_double != 0;
}
