/* Exhaustive checks that a quotient by a constant formed as one double
 * product equals the IEEE single-precision quotient over the inputs a
 * kernel gives it:
 *   - the depth camera map:  (float)((double)x * RN_double(1/200)) == x / 200.0f
 *     for every float x in [0, 200] (and -0.0).  Why it can hold: x/200 =
 *     (x/8)/25 and 1/25 has a binary period of 20, so a non-representable
 *     quotient never lies within ~2^-45 (relative) of a float rounding
 *     midpoint, while the double product is within ~2^-52 of the exact
 *     quotient;
 *   - the actor's symlog scaling: (float)((double)x * RN_double(1/c)) == x / c
 *     with c = sqrtf(1.0001f), for every float x in [0, 8] (|symlog| is at
 *     most log1p(1000) < 7; rounding to nearest is symmetric in the sign).
 *   - the onboard controller's and plane kernel's constant divisors (10, 20,
 *     30, 45, pi/6, pi/4 and the thrust span 294.2*0.85*(1 - 0.08), each as
 *     the float the device code forms): every finite float x, visited with
 *     the stride given as the first argument (default 61; a stride of 1 is
 *     the full 4.28e9-value check, about 30 CPU-minutes).
 * Prints one "<n> values, <m> mismatches" line per check; exits non-zero on
 * any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static unsigned long long check(float c, double inv, uint32_t top, const char *name) {
    unsigned long long bad = 0, n = 0;
    for (uint32_t bits = 0; bits <= top; ++bits) {
        float x;
        memcpy(&x, &bits, 4);
        const volatile float xv = x;
        const float want = xv / c;
        const float got = (float)((double)xv * inv);
        uint32_t a, b;
        memcpy(&a, &want, 4);
        memcpy(&b, &got, 4);
        bad += a != b;
        ++n;
    }
    const float nz = -0.0f;
    bad += signbit((float)((double)nz * inv)) != signbit(nz / c);
    printf("%s: %llu values, %llu mismatches\n", name, n, bad);
    return bad;
}

static unsigned long long check_all(float c, uint32_t stride, const char *name) {
    const double inv = 1.0 / (double)c;
    unsigned long long bad = 0, n = 0;
    for (uint64_t b = 0; b < (1ull << 32); b += stride) {
        const uint32_t bits = (uint32_t)b;
        if ((bits & 0x7f800000u) == 0x7f800000u) continue; /* inf, NaN */
        float x;
        memcpy(&x, &bits, 4);
        const volatile float xv = x;
        const float want = xv / c;
        const float got = (float)((double)xv * inv);
        uint32_t a, g;
        memcpy(&a, &want, 4);
        memcpy(&g, &got, 4);
        bad += a != g;
        ++n;
    }
    printf("%s: %llu values, %llu mismatches\n", name, n, bad);
    return bad;
}

int main(int argc, char **argv) {
    const uint32_t stride = argc > 1 ? (uint32_t)strtoul(argv[1], NULL, 10) : 61u;
    const volatile float c_sym = 1.0001f, pi = 3.14159265358979323846f, installed = 294.2f;
    const float c = sqrtf(c_sym);
    unsigned long long bad = check(200.0f, 1.0 / 200.0, 0x43480000u /* 200.0f */, "x / 200");
    bad += check(c, 1.0 / (double)c, 0x41000000u /* 8.0f */, "x / sqrtf(1.0001f)");
    const float max_installed = installed * 0.85f, min_thrust = max_installed * 0.08f;
    const float span = max_installed - min_thrust;
    bad += check_all(10.0f, stride, "all x / 10");
    bad += check_all(20.0f, stride, "all x / 20");
    bad += check_all(30.0f, stride, "all x / 30");
    bad += check_all(45.0f, stride, "all x / 45");
    bad += check_all(pi / 6.0f, stride, "all x / (pi/6)");
    bad += check_all(pi / 4.0f, stride, "all x / (pi/4)");
    bad += check_all(span, stride, "all x / thrust span");
    return bad != 0;
}
