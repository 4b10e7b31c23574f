// gfx950 kernels of the 142-feature sensor path and their C entry points.
//
// Semantics follow the reference CPU twin tb_train_extract_features_cpu
// (src/training/training.c:57-142); the reference CUDA kernel it replaces is
// src/cuda/features.cu:90-169.  The path is an HBM-bound streaming reduction
// (33,584 algorithmic bytes and ~4,100 log evaluations per environment), so
// the design is about coalescing and bytes in flight, not MFMA:
//
//   * one 256-thread workgroup (4 wave64) per environment, grid-stride over
//     environments; each wave issues 8 fully coalesced 1 KiB loads (4 LiDAR,
//     4 camera), so a workgroup holds the environment's 32 KiB in flight;
//   * wave w reads LiDAR floats [1024w, 1024w+1024) as float4 per lane,
//     evaluates the bin transform in registers and writes the values into an
//     LDS stage laid out sector-major: chunk c (row el = c/4, bins 4(c%4)..+3)
//     of sector s at 16-byte unit c*68 + s.  The pitch of 68 units makes the
//     stage writes conflict-free over 64 banks and the reads (lane s walks
//     c = 0..15) conflict-free on any bank count;
//   * after one barrier wave 0 sums its sector's 64 values sequentially in
//     the reference order (row outer, bin inner), so the LiDAR means differ
//     from the CPU only by the per-bin log1p, never by summation order;
//   * wave w also owns camera w: v_dot4_u32_u8 byte sums and a cross-lane
//     integer reduction make the 16 quadrant means bit-exact;
//   * wave 1 produces the 62 clamp and mission features (bit-exact) from
//     values it loads together with its LiDAR and camera loads.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

#include "turbinator/training/cuda_features.h"
#include "turbinator/training/hip_features.h"
#include "xcd_order.h"

namespace {

constexpr int kObsDim = 4148;
constexpr int kFeatureDim = 142;
constexpr int kLidarOffset = 48;
constexpr int kBlockThreads = 256;
constexpr int kStagePitch = 68;  // 16-byte units per LDS stage chunk row
constexpr unsigned kMaxBlocks = 1u << 20;
constexpr size_t kMaxBatch = 0x7fffffffu;
// Diagnostics row (bytes): sector minimum as float [0, 256), per sector a
// 16-bit word (first-minimum position inside the sector | valid count << 8)
// [256, 384), camera quadrant minimum byte [384, 400), camera quadrant
// nonzero count as 16 bits [400, 432).
constexpr int kDiagBytes = TB_HIP_DIAG_BYTES;
constexpr int kDiagArgCount = 256, kDiagCamMin = 384, kDiagCamOcc = 400;

// L = log1pf(120.0f) = 0x1.32ee3cp+2 as the reference evaluates it (glibc
// and GCC's constant folding agree; it is the correctly rounded float of
// ln 121).  ln2 / L split into two floats, and 1 / L:
constexpr float kLn2OverLHi = 0x1.28009cp-3f;
constexpr float kLn2OverLLo = -0x1.9578d6p-29f;
constexpr float kInvL = 0x1.ab0a8ap-3f;
constexpr float kPi = 3.14159265358979323846f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

struct Rows {
    const unsigned char *obs;
    size_t obs_stride;
    const unsigned char *mission;
    size_t mission_stride;
    const unsigned char *cameras;
    size_t camera_stride;
    const float *depth;  // fp32 depth cameras [batch, 16384] metres (DEPTH kernels)
    size_t depth_stride;
    float *out;
    unsigned char *diag;  // optional [batch, kDiagBytes] diagnostics rows (DIAG kernels)
    const uint32_t *index;  // optional: output row e reads input row index[e]
    size_t capacity;        // input rows available when index is set
    size_t batch;
};

// f(r) of training.c:65-68 without a libm call.  For valid r the argument
// x = min(r, 120) is split exactly as 1 + x = u + c (Fast2Sum with the larger
// operand first), so log1p(x) = log(u) + log1p(c/u) ~= log2(u)*ln2 + c/u with
// |c/u| <= 2^-24.  The hardware log2 and the c/u term are combined with the
// 1/log1pf(120) scaling in one FMA chain (ln2/L kept as a hi+lo pair).
__device__ __forceinline__ float lidar_bin_feature(float r) {
    const bool valid = (r >= 0.0f) && (r < __builtin_huge_valf());
    const float x = __builtin_fminf(r, 120.0f);
    const float a = __builtin_fmaxf(x, 1.0f);
    const float b = __builtin_fminf(x, 1.0f);
    const float u = a + b;
    const float c = b - (u - a);
    const float l2 = __builtin_amdgcn_logf(u);
    const float t = c * __builtin_amdgcn_rcpf(u);
    float f = __builtin_fmaf(l2, kLn2OverLHi, __builtin_fmaf(l2, kLn2OverLLo, t * kInvL));
    f = (x == 0.0f) ? x : f;  // log1p(+-0) = +-0
    return valid ? f : -1.0f;
}

// The same value inside the sector sums, minus the signed-zero select: the
// sums start at +0.0f and adding +-0 to +-0 or to a nonzero sum gives what
// adding the exact +-0 would, so the select cannot change a sum.
__device__ __forceinline__ float lidar_bin_term(float r) {
    const bool valid = (r >= 0.0f) && (r < __builtin_huge_valf());
    const float x = __builtin_fminf(r, 120.0f);
    const float a = __builtin_fmaxf(x, 1.0f);
    const float b = __builtin_fminf(x, 1.0f);
    const float u = a + b;
    const float c = b - (u - a);
    const float l2 = __builtin_amdgcn_logf(u);
    const float t = c * __builtin_amdgcn_rcpf(u);
    const float f = __builtin_fmaf(l2, kLn2OverLHi, __builtin_fmaf(l2, kLn2OverLLo, t * kInvL));
    return valid ? f : -1.0f;
}

__device__ __forceinline__ float clamp_ref(float x, float lo, float hi) {
    return x < lo ? lo : (x > hi ? hi : x);  // training.c:57-59
}

__device__ __forceinline__ float finite_or_zero(float x) {
    return __builtin_isfinite(x) ? x : 0.0f;  // training.c:61-63
}

__device__ __forceinline__ float scalar_scale(int i) {  // training.c:70-81
    float s = 1.0f;
    if (i < 2) s = 300.0f;
    else if (i == 2) s = 100.0f;
    else if (i < 6) s = 50.0f;
    else if (i >= 10 && i < 13) s = 5.0f;
    else if (i >= 13 && i < 16) s = 30.0f;
    else if (i >= 28 && i < 32) s = kPi / 4.0f;
    else if (i >= 32 && i < 40) s = 5.0f;
    else if (i == 44 || i == 45) s = kPi / 2.0f;
    return s;
}

// Four consecutive floats; LV is the widest load the row alignment allows.
template <int LV>
__device__ __forceinline__ f32x4 load_lidar4(const float *p) {
    if constexpr (LV == 4) {
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
    } else if constexpr (LV == 2) {
        const f32x2 lo = __builtin_nontemporal_load(reinterpret_cast<const f32x2 *>(p));
        const f32x2 hi = __builtin_nontemporal_load(reinterpret_cast<const f32x2 *>(p + 2));
        return f32x4{lo.x, lo.y, hi.x, hi.y};
    } else {
        return f32x4{__builtin_nontemporal_load(p), __builtin_nontemporal_load(p + 1),
                     __builtin_nontemporal_load(p + 2), __builtin_nontemporal_load(p + 3)};
    }
}

// Sixteen consecutive camera bytes; CV is the widest load the alignment allows.
template <int CV>
__device__ __forceinline__ u32x4 load_camera16(const unsigned char *p) {
    if constexpr (CV == 16) {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    } else if constexpr (CV == 8) {
        const u32x2 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
        const u32x2 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p + 8));
        return u32x4{lo.x, lo.y, hi.x, hi.y};
    } else if constexpr (CV == 4) {
        const unsigned *q = reinterpret_cast<const unsigned *>(p);
        return u32x4{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1),
                     __builtin_nontemporal_load(q + 2), __builtin_nontemporal_load(q + 3)};
    } else {
        unsigned w[4];
        for (int k = 0; k < 4; ++k)
            w[k] = (unsigned)p[4 * k] | ((unsigned)p[4 * k + 1] << 8) |
                   ((unsigned)p[4 * k + 2] << 16) | ((unsigned)p[4 * k + 3] << 24);
        return u32x4{w[0], w[1], w[2], w[3]};
    }
}

__device__ __forceinline__ unsigned byte_sum(u32x4 w, unsigned acc) {
    acc = __builtin_amdgcn_udot4(w.x, 0x01010101u, acc, false);
    acc = __builtin_amdgcn_udot4(w.y, 0x01010101u, acc, false);
    acc = __builtin_amdgcn_udot4(w.z, 0x01010101u, acc, false);
    return __builtin_amdgcn_udot4(w.w, 0x01010101u, acc, false);
}

// Sum over the 32 lanes that share lane bit 1 (the camera column half qx).
__device__ __forceinline__ unsigned sum_same_qx(unsigned v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// Depth (metres) -> luma byte: 255 * (1 - clamp(d, 0, 200) / 200), rounded
// half to even; non-finite depth counts as 0 m.  The quotient is formed as
// (float)((double)x * RN(1/200)), which equals the IEEE quotient x / 200.0f
// for every float x in [0, 200] (checked exhaustively by
// tests/csrc/check_div_by_constant.c), so the bytes are bit-exact.
__device__ __forceinline__ unsigned depth_luma(float depth_m) {
    // clamp_ref(finite_or_zero(x), 0, 200) as one median-of-three after the
    // finiteness select: equal for every finite x (a -0.0 that may come out
    // as +0.0 gives the same byte).
    const float d = __builtin_amdgcn_fmed3f(finite_or_zero(depth_m), 0.0f, 200.0f);
    const float q = (float)((double)d * (1.0 / 200.0));
    return (unsigned)__builtin_rintf(255.0f * (1.0f - q));
}

// Sum over the 32 lanes that share lane bit 3 (column half of a 64-float
// depth row read as 16 lanes x float4).
__device__ __forceinline__ unsigned sum_same_bit3(unsigned v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ unsigned bytes_min(u32x4 w, unsigned m) {
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int b = 0; b < 4; ++b) m = min(m, (w[d] >> (8 * b)) & 0xffu);
    return m;
}

// Bytes != 0: the high bit of each byte of ((x & 0x7f..) + 0x7f..) | x is set
// exactly when that byte is nonzero (no carry crosses a byte).
__device__ __forceinline__ unsigned bytes_nonzero(u32x4 w, unsigned n) {
#pragma unroll
    for (int d = 0; d < 4; ++d)
        n += __builtin_popcount((((w[d] & 0x7f7f7f7fu) + 0x7f7f7f7fu) | w[d]) & 0x80808080u);
    return n;
}

__device__ __forceinline__ unsigned min_same_qx(unsigned v) {
    v = min(v, __shfl_xor(v, 1));
    v = min(v, __shfl_xor(v, 4));
    v = min(v, __shfl_xor(v, 8));
    v = min(v, __shfl_xor(v, 16));
    v = min(v, __shfl_xor(v, 32));
    return v;
}

// LV: floats per LiDAR load (4, 2 or 1 from the row alignment).
// CV: bytes per camera load (16, 8, 4 or 1 from the row alignment).
// DIAG: also write the per-environment diagnostics (no reference
// counterpart): LiDAR sector minimum / first argmin / valid count and camera
// quadrant minimum byte / nonzero count, from the same loads.
// DEPTH: cameras arrive as fp32 depth and are quantised to luma bytes in
// registers (the configurations' 4x64x64 fp32 cameras).
template <int LV, int CV, bool DIAG, bool DEPTH = false>
__global__ __launch_bounds__(kBlockThreads) void features_kernel(Rows rows) {
    __shared__ f32x4 stage[16 * kStagePitch];
    // DIAG partials per (chunk, sector): minimum valid range and
    // (position of its first occurrence among the chunk's 4 bins, 1-based,
    // 0 if none) | (valid count << 16).  One 8-byte slot per (chunk, sector),
    // so that wave 0 reads them at 16-bit immediate offsets from one address
    // register; wave 0 turns positions into bin indices.
    __shared__ u32x2 dpart[DIAG ? 16 * kStagePitch : 1];
    // DIAG: the environment's 432-byte diagnostics row, assembled here and
    // written by wave 1 as 27 lane-consecutive 16-byte stores.
    __shared__ u32x4 drow[DIAG ? kDiagBytes / 16 : 1];
    // DIAG: the 16 camera quadrant means, written after the barrier by wave 3
    // in one store (94.1 -> 91.9 us for the diagnostics entry); the plain
    // kernel stores them from the four waves directly (gathering measured
    // 0.4 us slower there).
    __shared__ float quads[DIAG ? 16 : 1];
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool has_cameras = DEPTH || rows.cameras != nullptr;

    for (size_t env = xcd_contiguous(blockIdx.x, gridDim.x); env < rows.batch;
         env += gridDim.x) {
        // With DIAG the lane index passes through an empty asm once per
        // environment, so the values derived from it (addresses, stage
        // positions, bin offsets) are formed per environment instead of
        // being hoisted out of this loop, which nearly always runs once,
        // into registers held across it: 64 instead of 100 VGPRs, 6 instead
        // of 4 waves per SIMD.  The other variants keep the hoisted form
        // (7 waves per SIMD measured faster than 8 there).
        int lane = threadIdx.x & 63;
        if constexpr (DIAG) asm volatile("" : "+v"(lane));
        // Stage position of this lane's float4 for each of the wave's 4
        // loads: LiDAR float4 index i*64 + lane (i = 4w + k) is row
        // (i%8)*2 + lane/32 of head i/8, azimuth sector (lane%32)/4, bins
        // 4*(lane%4)..+3.
        int unit[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * w + k, head = i >> 3, row = ((i & 7) << 1) + (lane >> 5);
            const int sector = head * 32 + (row >> 2) * 8 + ((lane & 31) >> 2);
            const int chunk = (row & 3) * 4 + (lane & 3);
            unit[k] = chunk * kStagePitch + sector;
        }
        float *out = rows.out + env * kFeatureDim;
        size_t src = env;
        if (rows.index) {
            src = rows.index[env];
            if (src >= rows.capacity) {  // reads nothing; marks the row
                if (threadIdx.x < kFeatureDim) out[threadIdx.x] = __builtin_nanf("");
                continue;
            }
        }
        const float *obs = reinterpret_cast<const float *>(rows.obs + src * rows.obs_stride);
        const float *lidar = obs + kLidarOffset;
        const float *mission =
            reinterpret_cast<const float *>(rows.mission + src * rows.mission_stride);
        // Issue every load of this wave before using any of them; wave 1
        // lanes 0..61 also fetch their proprio / scan / mission value now so
        // no load waits behind the barrier.
        float sv = 0.0f, m6 = 0.0f;
        if (w == 1 && lane < 62) {
            sv = lane < 48 ? obs[lane] : (lane < 52 ? obs[4144 + lane - 48] : mission[lane - 52]);
            m6 = mission[6];
        }
        f32x4 v[4];
        u32x4 px[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = load_lidar4<LV>(lidar + (4 * w + k) * 256 + 4 * lane);
        if (!DEPTH && has_cameras) {
            // Camera w, rows 16k + lane/4, bytes 16*(lane%4)..+15.
            const unsigned char *cam = rows.cameras + src * rows.camera_stride + w * 4096;
#pragma unroll
            for (int k = 0; k < 4; ++k) px[k] = load_camera16<CV>(cam + (k * 64 + lane) * 16);
        }

#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f32x4 f;
            f.x = lidar_bin_term(v[k].x);
            f.y = lidar_bin_term(v[k].y);
            f.z = lidar_bin_term(v[k].z);
            f.w = lidar_bin_term(v[k].w);
            stage[unit[k]] = f;
            if constexpr (DIAG) {
                // Bins in increasing order, so a strict < keeps the first
                // minimum; selects rather than branches.
                float best = 0.0f;
                unsigned first = 0u, count = 0u;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float r = v[k][e];
                    const bool valid = (int)(r >= 0.0f) & (int)(r < __builtin_huge_valf());
                    const bool take = (int)valid & ((int)(first == 0u) | (int)(r < best));
                    count += valid ? 1u : 0u;
                    best = take ? r : best;
                    first = take ? (unsigned)(e + 1) : first;
                }
                dpart[unit[k]] = u32x2{__float_as_uint(best), first | (count << 16)};
            }
        }

        // Quadrant (cam w, qy, qx = lane bit 1): loads k = 0,1 cover rows
        // 0..31 (qy 0), k = 2,3 rows 32..63 (qy 1).  training.c:128-141.
        float *const qrow = DIAG ? quads : out + 126;
        if constexpr (DEPTH) {
            // Camera w as 4096 floats: load k covers rows 4k + lane/16,
            // columns 4*(lane%16)..+3, so qy = k/8 and qx = lane bit 3.
            const float *cam = reinterpret_cast<const float *>(
                reinterpret_cast<const unsigned char *>(rows.depth) + src * rows.depth_stride) +
                w * 4096;
            unsigned top = 0u, bottom = 0u;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const f32x4 d = __builtin_nontemporal_load(
                    reinterpret_cast<const f32x4 *>(cam + k * 256 + 4 * lane));
                const unsigned s4 =
                    depth_luma(d.x) + depth_luma(d.y) + depth_luma(d.z) + depth_luma(d.w);
                if (k < 8) top += s4;
                else bottom += s4;
            }
            top = sum_same_bit3(top);
            bottom = sum_same_bit3(bottom);
            if (lane == 0 || lane == 8) {
                const int qx = lane >> 3;
                qrow[w * 4 + qx] = (float)top / (1024.0f * 255.0f);
                qrow[w * 4 + 2 + qx] = (float)bottom / (1024.0f * 255.0f);
            }
        } else if (has_cameras) {
            const unsigned top = sum_same_qx(byte_sum(px[1], byte_sum(px[0], 0u)));
            const unsigned bottom = sum_same_qx(byte_sum(px[3], byte_sum(px[2], 0u)));
            if (lane == 0 || lane == 2) {
                const int qx = lane >> 1;
                qrow[w * 4 + qx] = (float)top / (1024.0f * 255.0f);
                qrow[w * 4 + 2 + qx] = (float)bottom / (1024.0f * 255.0f);
            }
        } else if (lane < 4) {
            qrow[w * 4 + lane] = 0.0f;
        }
        if constexpr (DIAG) {  // camera words are dead after this
            unsigned char *diag = reinterpret_cast<unsigned char *>(drow);
            unsigned short *occ = reinterpret_cast<unsigned short *>(diag + kDiagCamOcc);
            if (has_cameras) {
                const unsigned top_min = min_same_qx(bytes_min(px[1], bytes_min(px[0], 255u)));
                const unsigned bot_min = min_same_qx(bytes_min(px[3], bytes_min(px[2], 255u)));
                const unsigned top_occ = sum_same_qx(bytes_nonzero(px[1], bytes_nonzero(px[0], 0u)));
                const unsigned bot_occ = sum_same_qx(bytes_nonzero(px[3], bytes_nonzero(px[2], 0u)));
                if (lane == 0 || lane == 2) {
                    const int q = w * 4 + (lane >> 1);
                    diag[kDiagCamMin + q] = (unsigned char)top_min;
                    diag[kDiagCamMin + q + 2] = (unsigned char)bot_min;
                    occ[q] = (unsigned short)top_occ;
                    occ[q + 2] = (unsigned short)bot_occ;
                }
            } else if (lane < 4) {
                diag[kDiagCamMin + w * 4 + lane] = 0u;
                occ[w * 4 + lane] = 0u;
            }
        }

        if (w == 1 && lane < 62) {
            // training.c:107-112.
            float scalar;
            if (lane < 48) {
                scalar = clamp_ref(finite_or_zero(sv) / scalar_scale(lane), -1.0f, 1.0f);
            } else if (lane < 52) {
                scalar = clamp_ref(finite_or_zero(sv), 0.0f, 1.0f);
            } else {
                const int i = lane - 52;
                const bool arena = finite_or_zero(m6) > 0.5f;
                const float m = (i >= 7 && arena) ? 0.0f : sv;
                scalar = clamp_ref(finite_or_zero(m), -1.0f, 1.0f);
            }
            out[lane] = scalar;
        }
        __syncthreads();
        if (w == 0) {
            // training.c:113-127: sequential sum, row outer, bin inner.
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const f32x4 f = stage[c * kStagePitch + lane];
                sum += f.x;
                sum += f.y;
                sum += f.z;
                sum += f.w;
            }
            out[62 + lane] = sum / 64.0f;
        }
        if (DIAG && w == 3 && lane < 16) out[126 + lane] = quads[lane];
        if (DIAG && w == 1) {
            // The diagnostics reduction runs on wave 1, beside wave 0's sums.
                // Chunks in increasing c are in scan order (row outer, bin
                // inner), so a strict < keeps the first minimum.  Chunk c of
                // sector `lane` holds its elevation row c / 4 (within the
                // sector), bins 4 (c % 4) .. + 3 of the azimuth sector, so
                // the position of chunk bin pos (1-based) inside the
                // sector's 64 bins, row-major, is 4 c + pos - 1.
                float best = 0.0f;
                unsigned first = 0u, count = 0u;
#pragma unroll
                for (int c = 0; c < 16; ++c) {
                    const u32x2 part = dpart[c * kStagePitch + lane];
                    const unsigned pos = part.y & 0xffffu;
                    const float m = __uint_as_float(part.x);
                    count += part.y >> 16;
                    const bool take = (int)(pos != 0u) & ((int)(first == 0u) | (int)(m < best));
                    best = take ? m : best;
                    first = take ? 4 * c + pos : first;
                }
                unsigned char *diag = reinterpret_cast<unsigned char *>(drow);
                reinterpret_cast<float *>(diag)[lane] = first == 0u ? -1.0f : best;
                const unsigned word = ((first - 1u) & 0xffu) | (count << 8);
                reinterpret_cast<unsigned short *>(diag + kDiagArgCount)[lane] = (unsigned short)word;
                // The row is written by this wave only from here on.
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (lane < kDiagBytes / 16)
                    reinterpret_cast<u32x4 *>(rows.diag + env * kDiagBytes)[lane] = drow[lane];
            }
        // The stage is reused by this block's next environment, if any.
        if (env + gridDim.x < rows.batch) __syncthreads();
    }
}

__global__ __launch_bounds__(256) void lidar_transform_kernel(const float *in, float *out,
                                                              size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = lidar_bin_feature(in[i]);
}

int vector_bytes(const void *base, size_t stride, int widest) {
    const uintptr_t bits = reinterpret_cast<uintptr_t>(base) | (uintptr_t)stride;
    for (int v = widest; v > 1; v >>= 1)
        if ((bits & (uintptr_t)(v - 1)) == 0) return v;
    return 1;
}

template <int LV, bool DIAG>
void launch_lv(const Rows &rows, int cv, unsigned blocks, unsigned lds, hipStream_t stream) {
    switch (cv) {
    case 16: features_kernel<LV, 16, DIAG><<<blocks, kBlockThreads, lds, stream>>>(rows); break;
    case 8: features_kernel<LV, 8, DIAG><<<blocks, kBlockThreads, lds, stream>>>(rows); break;
    case 4: features_kernel<LV, 4, DIAG><<<blocks, kBlockThreads, lds, stream>>>(rows); break;
    default: features_kernel<LV, 1, DIAG><<<blocks, kBlockThreads, lds, stream>>>(rows); break;
    }
}

template <bool DIAG>
void launch_diag(const Rows &rows, int lv, int cv, unsigned blocks, unsigned lds,
                 hipStream_t stream) {
    if (lv == 4) launch_lv<4, DIAG>(rows, cv, blocks, lds, stream);
    else if (lv == 2) launch_lv<2, DIAG>(rows, cv, blocks, lds, stream);
    else launch_lv<1, DIAG>(rows, cv, blocks, lds, stream);
}

// Workgroups in flight per CU.  Its registers let the plain kernel hold 7
// per CU; on the streaming layouts fewer keep HBM busier (16,384
// environments, identical outputs): rows laid out as the reference's batch
// 4 per CU (85.76 -> 83.99 us; 3 per CU 91.9 us), strided replay records 5
// per CU (353.9 -> 348.1 us for 65,536 records).  Indexed gathers, fp32
// depth cameras and the diagnostics variant keep their resource limit
// (4 per CU measured 91.9 -> 94.8, 208.0 -> 210.3 and 94.2 -> 116.2 us).
// The cap is dynamic LDS the kernel does not use: a workgroup then takes
// more than 1 / (n + 1) of the CU's LDS, so n fit.
constexpr unsigned kLdsPerCu = 160 * 1024;
constexpr unsigned kStageLds = 16 * kStagePitch * sizeof(f32x4);

unsigned occupancy_lds(const Rows &rows) {
    if (rows.depth || rows.diag || rows.index) return 0;
    const bool batch_rows = rows.obs_stride == kObsDim * sizeof(float) &&
                            rows.mission_stride == 10 * sizeof(float) &&
                            rows.camera_stride == 16384;
    const unsigned per_cu = batch_rows ? 4 : 5;
    const unsigned total = (kLdsPerCu / (per_cu + 1) + 1 + 1023) / 1024 * 1024;
    return total - kStageLds;
}

template <int LV>
void launch_depth(const Rows &rows, unsigned blocks, hipStream_t stream) {
    features_kernel<LV, 16, false, true><<<blocks, kBlockThreads, 0, stream>>>(rows);
}

int launch_features(const Rows &rows, hipStream_t stream) {
    // Float rows are 4-byte aligned (checked by the callers); the LiDAR block
    // starts 192 bytes into the row.
    const int lv = vector_bytes(rows.obs + kLidarOffset * sizeof(float), rows.obs_stride, 16) / 4;
    const int cv = rows.cameras ? vector_bytes(rows.cameras, rows.camera_stride, 16) : 16;
    const unsigned blocks = rows.batch > kMaxBlocks ? kMaxBlocks : (unsigned)rows.batch;
    // Report errors of this launch only: a failure left on the thread by an
    // unrelated earlier runtime call (e.g. selecting a missing device) is
    // not a launch failure.
    (void)hipGetLastError();
    if (rows.depth) {
        if (lv == 4) launch_depth<4>(rows, blocks, stream);
        else if (lv == 2) launch_depth<2>(rows, blocks, stream);
        else launch_depth<1>(rows, blocks, stream);
    } else if (rows.diag) launch_diag<true>(rows, lv, cv, blocks, 0, stream);
    else launch_diag<false>(rows, lv, cv, blocks, occupancy_lds(rows), stream);
    return hipGetLastError() == hipSuccess;
}

}  // namespace

extern "C" int tb_cuda_extract_features_device(const float *device_obs,
                                               const float *device_mission,
                                               const unsigned char *device_cameras,
                                               float *device_features, size_t batch_size,
                                               void *stream) {
    if (!device_obs || !device_mission || !device_features || batch_size == 0 ||
        batch_size > kMaxBatch)
        return 0;
    Rows rows;
    rows.obs = reinterpret_cast<const unsigned char *>(device_obs);
    rows.obs_stride = kObsDim * sizeof(float);
    rows.mission = reinterpret_cast<const unsigned char *>(device_mission);
    rows.mission_stride = 10 * sizeof(float);
    rows.cameras = device_cameras;
    rows.camera_stride = 16384;
    rows.depth = nullptr;
    rows.depth_stride = 0;
    rows.out = device_features;
    rows.diag = nullptr;
    rows.index = nullptr;
    rows.capacity = 0;
    rows.batch = batch_size;
    return launch_features(rows, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int tb_hip_extract_features_diagnostics_device(const float *obs, const float *mission,
                                                          const unsigned char *cameras,
                                                          float *features, void *diagnostics,
                                                          size_t batch_size, void *stream) {
    if (!obs || !mission || !features || !diagnostics || batch_size == 0 ||
        batch_size > kMaxBatch || (reinterpret_cast<uintptr_t>(diagnostics) & 15u) != 0)
        return 0;  // the rows are written with 16-byte stores
    Rows rows;
    rows.obs = reinterpret_cast<const unsigned char *>(obs);
    rows.obs_stride = kObsDim * sizeof(float);
    rows.mission = reinterpret_cast<const unsigned char *>(mission);
    rows.mission_stride = 10 * sizeof(float);
    rows.cameras = cameras;
    rows.camera_stride = 16384;
    rows.depth = nullptr;
    rows.depth_stride = 0;
    rows.out = features;
    rows.diag = static_cast<unsigned char *>(diagnostics);
    rows.index = nullptr;
    rows.capacity = 0;
    rows.batch = batch_size;
    return launch_features(rows, reinterpret_cast<hipStream_t>(stream));
}

namespace {

int strided_entry(const void *obs, size_t obs_stride, const void *mission, size_t mission_stride,
                  const void *cameras, size_t camera_stride, const uint32_t *index,
                  size_t capacity, float *features, size_t batch_size, void *stream) {
    if (!obs || !mission || !features || batch_size == 0 || batch_size > kMaxBatch) return 0;
    if (((reinterpret_cast<uintptr_t>(obs) | obs_stride) & 3u) != 0 ||
        ((reinterpret_cast<uintptr_t>(mission) | mission_stride) & 3u) != 0 ||
        (reinterpret_cast<uintptr_t>(features) & 3u) != 0)
        return 0;
    Rows rows;
    rows.obs = static_cast<const unsigned char *>(obs);
    rows.obs_stride = obs_stride;
    rows.mission = static_cast<const unsigned char *>(mission);
    rows.mission_stride = mission_stride;
    rows.cameras = static_cast<const unsigned char *>(cameras);
    rows.camera_stride = camera_stride;
    rows.depth = nullptr;
    rows.depth_stride = 0;
    rows.out = features;
    rows.diag = nullptr;
    rows.index = index;
    rows.capacity = capacity;
    rows.batch = batch_size;
    return launch_features(rows, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" int tb_hip_extract_features_strided_device(const void *obs, size_t obs_stride,
                                                      const void *mission,
                                                      size_t mission_stride,
                                                      const void *cameras,
                                                      size_t camera_stride, float *features,
                                                      size_t batch_size, void *stream) {
    return strided_entry(obs, obs_stride, mission, mission_stride, cameras, camera_stride,
                         nullptr, 0, features, batch_size, stream);
}

extern "C" int tb_hip_extract_features_indexed_device(
    const void *obs, size_t obs_stride, const void *mission, size_t mission_stride,
    const void *cameras, size_t camera_stride, size_t capacity, const unsigned int *indices,
    float *features, size_t batch_size, void *stream) {
    if (!indices || capacity == 0) return 0;
    return strided_entry(obs, obs_stride, mission, mission_stride, cameras, camera_stride,
                         indices, capacity, features, batch_size, stream);
}

extern "C" int tb_hip_extract_features_depth_device(const float *obs, const float *mission,
                                                    const float *depth, float *features,
                                                    size_t batch_size, void *stream) {
    if (!obs || !mission || !depth || !features || batch_size == 0 || batch_size > kMaxBatch ||
        (reinterpret_cast<uintptr_t>(depth) & 15u) != 0)
        return 0;
    Rows rows;
    rows.obs = reinterpret_cast<const unsigned char *>(obs);
    rows.obs_stride = kObsDim * sizeof(float);
    rows.mission = reinterpret_cast<const unsigned char *>(mission);
    rows.mission_stride = 10 * sizeof(float);
    rows.cameras = nullptr;
    rows.camera_stride = 0;
    rows.depth = depth;
    rows.depth_stride = 16384 * sizeof(float);
    rows.out = features;
    rows.diag = nullptr;
    rows.index = nullptr;
    rows.capacity = 0;
    rows.batch = batch_size;
    return launch_features(rows, reinterpret_cast<hipStream_t>(stream));
}

// Staging of tb_hip_extract_features_host_static: the inputs and features of
// up to TB_HIP_STATIC_MAX_BATCH environments, one array per GPU (every GPU
// the library runs on holds its own copy), sections on 256 bytes.  Host code
// never passes `scratch` itself to a kernel or copy: its name there stands
// for the host-side shadow, not a device address.  The device address comes
// from hipGetSymbolAddress, once per device, with that device current.
namespace {
constexpr size_t kStaticMax = TB_HIP_STATIC_MAX_BATCH;
constexpr size_t align_section(size_t x) { return (x + 255) & ~(size_t)255; }
constexpr size_t kStaticObs = 0;
constexpr size_t kStaticMission = align_section(kStaticObs + kStaticMax * kObsDim * sizeof(float));
constexpr size_t kStaticCameras = align_section(kStaticMission + kStaticMax * 10 * sizeof(float));
constexpr size_t kStaticFeatures = align_section(kStaticCameras + kStaticMax * 16384);
constexpr size_t kStaticBytes = align_section(kStaticFeatures + kStaticMax * kFeatureDim * sizeof(float));
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

namespace {
// scratch's device address per device, 0 until first looked up.
std::atomic<unsigned char *> scratch_address[kMaxDevices];

unsigned char *static_staging() {
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)
        return nullptr;
    unsigned char *address = scratch_address[device].load(std::memory_order_acquire);
    if (address) return address;
    void *found = nullptr;
    if (hipGetSymbolAddress(&found, HIP_SYMBOL(scratch)) != hipSuccess || !found) return nullptr;
    address = static_cast<unsigned char *>(found);
    scratch_address[device].store(address, std::memory_order_release);
    return address;
}
}  // namespace

// tb_cuda_extract_features_host (src/cuda/features.cu:62-88) with the staging
// above instead of a handle's buffers: the same copies in, the device entry,
// the copy out and the wait, on the caller's stream.  No allocation: the
// only runtime calls are hipGetDevice, hipGetSymbolAddress (first call on a
// device), hipStreamIsCapturing, hipMemcpyAsync, the launch and
// hipStreamSynchronize.  Nothing in the staging has to start at zero: each
// call writes the rows it reads.
//
// The call is synchronous and copies pageable host memory, neither of which
// a stream under graph capture accepts (a refused call would also end the
// caller's capture), so a capturing stream gets 0 with nothing enqueued.  A
// failure after the first copy was queued waits for the queued work before
// returning 0, so the caller may reuse its host arrays at once.
extern "C" int tb_hip_extract_features_host_static(const float *obs, const float *mission,
                                                   const unsigned char *cameras, size_t count,
                                                   float *out_features, void *stream) {
    if (!obs || !mission || !cameras || !out_features || count == 0 || count > kStaticMax)
        return 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &capture) != hipSuccess ||
        capture != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return 0;
    }
    unsigned char *staging = static_staging();
    if (!staging) return 0;
    float *d_obs = reinterpret_cast<float *>(staging + kStaticObs);
    float *d_mission = reinterpret_cast<float *>(staging + kStaticMission);
    unsigned char *d_cameras = staging + kStaticCameras;
    float *d_features = reinterpret_cast<float *>(staging + kStaticFeatures);
    const bool ok =
        hipMemcpyAsync(d_obs, obs, count * kObsDim * sizeof(float), hipMemcpyHostToDevice, s) ==
            hipSuccess &&
        hipMemcpyAsync(d_mission, mission, count * 10 * sizeof(float), hipMemcpyHostToDevice,
                       s) == hipSuccess &&
        hipMemcpyAsync(d_cameras, cameras, count * 16384, hipMemcpyHostToDevice, s) ==
            hipSuccess &&
        tb_cuda_extract_features_device(d_obs, d_mission, d_cameras, d_features, count,
                                        stream) &&
        hipMemcpyAsync(out_features, d_features, count * kFeatureDim * sizeof(float),
                       hipMemcpyDeviceToHost, s) == hipSuccess;
    const bool done = hipStreamSynchronize(s) == hipSuccess;
    if (!ok) (void)hipGetLastError();
    return ok && done;
}

extern "C" int tb_hip_lidar_transform_device(const float *ranges, float *out, size_t count,
                                             void *stream) {
    if (!ranges || !out || count == 0) return 0;
    size_t want = (count + 255) / 256;
    const unsigned blocks = want > kMaxBlocks ? kMaxBlocks : (unsigned)want;
    (void)hipGetLastError();
    lidar_transform_kernel<<<blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(ranges, out,
                                                                                      count);
    return hipGetLastError() == hipSuccess;
}

extern "C" int tb_cuda_synchronize(void *stream) {
    return hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)) == hipSuccess;
}
