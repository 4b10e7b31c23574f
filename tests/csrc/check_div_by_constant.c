/* Exhaustive check that the depth camera kernel's quotient
 *   q = (float)((double)x * RN_double(1/200))
 * equals the IEEE single-precision quotient x / 200.0f for every float x in
 * [0, 200] (and -0.0).  Why it can hold: x/200 = (x/8)/25 and 1/25 has a
 * binary period of 20, so a non-representable quotient never lies within
 * ~2^-45 (relative) of a float rounding midpoint, while the double product
 * is within ~2^-52 of the exact quotient.  Prints the mismatch count; exits
 * non-zero on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const double inv = 1.0 / 200.0;
    const uint32_t top = 0x43480000u; /* 200.0f */
    unsigned long long bad = 0, n = 0;
    for (uint32_t bits = 0; bits <= top; ++bits) {
        float x;
        memcpy(&x, &bits, 4);
        const volatile float xv = x;
        const float want = xv / 200.0f;
        const float got = (float)((double)xv * inv);
        uint32_t a, b;
        memcpy(&a, &want, 4);
        memcpy(&b, &got, 4);
        bad += a != b;
        ++n;
    }
    const float nz = -0.0f;
    bad += signbit((float)((double)nz * inv)) != signbit(nz / 200.0f);
    printf("%llu values, %llu mismatches\n", n, bad);
    return bad != 0;
}
