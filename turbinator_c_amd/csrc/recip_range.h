// 1 / y for y in [0.2, 30], correctly rounded: the hardware reciprocal
// (about 1 ulp) refined by one Newton step in fused multiply-adds.  On
// gfx950 it equals the IEEE quotient 1.0f / y for every float in that range
// (tests/csrc/check_recip.hip checks all 61,027,124 of them); the IEEE
// division is a ten-instruction sequence with a scale and a fix-up.
#pragma once

__device__ __forceinline__ float recip_range(float y) {
    const float r = __builtin_amdgcn_rcpf(y);
    return __builtin_fmaf(__builtin_fmaf(-y, r, 1.0f), r, r);
}
