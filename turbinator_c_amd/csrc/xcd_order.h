// Workgroup-to-environment order shared by the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

// MI355X dispatches workgroups to its 8 XCDs round-robin by id, and each XCD
// has its own L2.  This bijection of [0, g) gives XCD x the contiguous
// environments [x n8, (x+1) n8) (n8 = g / 8; ids past 8 n8 map to
// themselves), so neighbouring environments meet in the same L2: rows that
// share cache lines at their ends are read once, and each XCD's writes are
// contiguous.
__device__ __forceinline__ size_t xcd_contiguous(size_t b, size_t g) {
    const size_t n8 = g / 8;
    return b < 8 * n8 ? (b % 8) * n8 + b / 8 : b;
}
