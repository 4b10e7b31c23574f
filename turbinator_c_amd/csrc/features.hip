// gfx950 kernels of the 142-feature sensor path and their C entry points.
//
// Semantics follow the reference CPU twin tb_train_extract_features_cpu
// (src/training/training.c:57-142); the reference CUDA kernel it replaces is
// src/cuda/features.cu:90-169.  Design (HBM-bound streaming reduction, no
// MFMA):
//   * one wavefront (64 lanes) per environment, four environments per
//     256-thread workgroup, grid-stride over environments;
//   * lane s owns LiDAR sector s (head = s/32, elevation sector = (s/8)%4,
//     azimuth sector = s%8) and reads its four 64-byte row runs with 128-bit
//     loads, summing the 64 bins in the reference order (row outer, bin
//     inner), so the only difference from the CPU is the per-bin log1p;
//   * cameras stream as 16 fully coalesced 1 KiB wave loads per environment;
//     byte sums use v_dot4_u32_u8 and a cross-lane integer reduction, so the
//     16 quadrant means are bit-exact;
//   * lanes 0..61 produce the clamp and mission features (bit-exact).

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "turbinator/training/cuda_features.h"
#include "turbinator/training/hip_features.h"

namespace {

constexpr int kObsDim = 4148;
constexpr int kFeatureDim = 142;
constexpr int kLidarOffset = 48;
constexpr int kWave = 64;
constexpr int kEnvsPerBlock = 4;
constexpr int kBlockThreads = kWave * kEnvsPerBlock;
constexpr unsigned kMaxBlocks = 1u << 20;
constexpr size_t kMaxBatch = 0x7fffffffu;

// log1pf(120.0f) as the reference evaluates it (glibc and GCC's folding
// agree; it is the correctly rounded float of ln 121).
constexpr float kLog1p120 = 0x1.32ee3cp+2f;
// ln2 / kLog1p120 split into two floats, and 1 / kLog1p120.
constexpr float kLn2OverLHi = 0x1.28009cp-3f;
constexpr float kLn2OverLLo = -0x1.9578d6p-29f;
constexpr float kInvL = 0x1.ab0a8ap-3f;
constexpr float kPi = 3.14159265358979323846f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

struct Rows {
    const unsigned char *obs;
    size_t obs_stride;
    const unsigned char *mission;
    size_t mission_stride;
    const unsigned char *cameras;
    size_t camera_stride;
    float *out;
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

template <int CV>
__device__ __forceinline__ u32x4 load_camera_chunk(const unsigned char *p) {
    if constexpr (CV == 16) {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    } else if constexpr (CV == 8) {
        const u32x2 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
        const u32x2 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p + 8));
        return u32x4{lo.x, lo.y, hi.x, hi.y};
    } else if constexpr (CV == 4) {
        const unsigned *q = reinterpret_cast<const unsigned *>(p);
        return u32x4{q[0], q[1], q[2], q[3]};
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

// LV: floats per LiDAR load (4 when every row run is 16-byte aligned, else 1).
// CV: bytes per camera load unit (16, 8, 4 or 1, from the row alignment).
template <int LV, int CV>
__global__ __launch_bounds__(kBlockThreads) void features_kernel(Rows rows) {
    const int lane = threadIdx.x & (kWave - 1);
    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const size_t first = (size_t)blockIdx.x * kEnvsPerBlock + wave;
    const size_t step = (size_t)gridDim.x * kEnvsPerBlock;

    // LiDAR sector of this lane.
    const int head = lane >> 5, es = (lane >> 3) & 3, as = lane & 7;
    const int sector_off = kLidarOffset + head * 2048 + es * 512 + as * 16;

    for (size_t env = first; env < rows.batch; env += step) {
        const float *obs = reinterpret_cast<const float *>(rows.obs + env * rows.obs_stride);
        const float *mission =
            reinterpret_cast<const float *>(rows.mission + env * rows.mission_stride);
        float *out = rows.out + env * kFeatureDim;

        // ---- LiDAR sector sum, reference order: row el outer, bin az inner.
        const float *sec = obs + sector_off;
        float sum = 0.0f;
        if constexpr (LV == 4) {
            f32x4 v[16];
#pragma unroll
            for (int el = 0; el < 4; ++el)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    v[el * 4 + j] = __builtin_nontemporal_load(
                        reinterpret_cast<const f32x4 *>(sec + el * 128 + 4 * j));
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                sum += lidar_bin_feature(v[k].x);
                sum += lidar_bin_feature(v[k].y);
                sum += lidar_bin_feature(v[k].z);
                sum += lidar_bin_feature(v[k].w);
            }
        } else {
#pragma unroll
            for (int el = 0; el < 4; ++el) {
                float v[16];
#pragma unroll
                for (int az = 0; az < 16; ++az) v[az] = sec[el * 128 + az];
#pragma unroll
                for (int az = 0; az < 16; ++az) sum += lidar_bin_feature(v[az]);
            }
        }

        // ---- Camera quadrant byte sums.  Chunk k = it*64 + lane of the
        // environment's 1024 16-byte chunks lies in camera it/4, row
        // (it%4)*16 + lane/4, columns 16*(lane%4)..+15, i.e. quadrant
        // (cam = it/4, qy = (it%4)/2, qx = (lane>>1)&1); accumulator it/2.
        float cam_mean = 0.0f;
        if (rows.cameras) {
            const unsigned char *cam = rows.cameras + env * rows.camera_stride;
            unsigned acc[8];
#pragma unroll
            for (int a = 0; a < 8; ++a) acc[a] = 0u;
#pragma unroll
            for (int it = 0; it < 16; ++it) {
                const u32x4 w = load_camera_chunk<CV>(cam + (size_t)(it * 64 + lane) * 16);
                acc[it >> 1] = byte_sum(w, acc[it >> 1]);
            }
            // Sum over the 32 lanes sharing qx (lane bit 1 untouched).
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                unsigned v = acc[a];
                v += __shfl_xor(v, 1);
                v += __shfl_xor(v, 4);
                v += __shfl_xor(v, 8);
                v += __shfl_xor(v, 16);
                v += __shfl_xor(v, 32);
                acc[a] = v;
            }
            // Output lane q < 16 wants accumulator q/2 of qx = q&1, held by
            // lane 2*(q&1).
            const int src = (lane & 1) << 1;
            unsigned pick = 0u;
#pragma unroll
            for (int a = 0; a < 8; ++a) {
                const unsigned v = __shfl(acc[a], src);
                pick = ((lane >> 1) == a) ? v : pick;
            }
            cam_mean = (float)pick / (1024.0f * 255.0f);  // training.c:138
        }

        // ---- Proprioception, scan statistics and mission (training.c:107-112).
        float scalar = 0.0f;
        if (lane < 48) {
            scalar = clamp_ref(finite_or_zero(obs[lane]) / scalar_scale(lane), -1.0f, 1.0f);
        } else if (lane < 52) {
            scalar = clamp_ref(finite_or_zero(obs[4144 + lane - 48]), 0.0f, 1.0f);
        } else if (lane < 62) {
            const int i = lane - 52;
            const bool arena = finite_or_zero(mission[6]) > 0.5f;
            const float v = (i >= 7 && arena) ? 0.0f : mission[i];
            scalar = clamp_ref(finite_or_zero(v), -1.0f, 1.0f);
        }

        if (lane < 62) out[lane] = scalar;
        out[62 + lane] = sum / 64.0f;
        if (lane < 16) out[126 + lane] = cam_mean;
    }
}

__global__ __launch_bounds__(256) void lidar_transform_kernel(const float *in, float *out,
                                                              size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = lidar_bin_feature(in[i]);
}

int camera_vector_bytes(const void *cameras, size_t stride) {
    const uintptr_t bits = reinterpret_cast<uintptr_t>(cameras) | (uintptr_t)stride;
    if ((bits & 15u) == 0) return 16;
    if ((bits & 7u) == 0) return 8;
    if ((bits & 3u) == 0) return 4;
    return 1;
}

template <int LV>
void launch_lv(const Rows &rows, int cv, unsigned blocks, hipStream_t stream) {
    switch (cv) {
    case 16: features_kernel<LV, 16><<<blocks, kBlockThreads, 0, stream>>>(rows); break;
    case 8: features_kernel<LV, 8><<<blocks, kBlockThreads, 0, stream>>>(rows); break;
    case 4: features_kernel<LV, 4><<<blocks, kBlockThreads, 0, stream>>>(rows); break;
    default: features_kernel<LV, 1><<<blocks, kBlockThreads, 0, stream>>>(rows); break;
    }
}

int launch_features(const Rows &rows, hipStream_t stream) {
    const uintptr_t lidar_bits =
        (reinterpret_cast<uintptr_t>(rows.obs) + kLidarOffset * sizeof(float)) |
        (uintptr_t)rows.obs_stride;
    const int lv = (lidar_bits & 15u) == 0 ? 4 : 1;
    const int cv = rows.cameras ? camera_vector_bytes(rows.cameras, rows.camera_stride) : 16;
    size_t want = (rows.batch + kEnvsPerBlock - 1) / kEnvsPerBlock;
    const unsigned blocks = want > kMaxBlocks ? kMaxBlocks : (unsigned)want;
    if (lv == 4) launch_lv<4>(rows, cv, blocks, stream);
    else launch_lv<1>(rows, cv, blocks, stream);
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
    rows.out = device_features;
    rows.batch = batch_size;
    return launch_features(rows, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int tb_hip_extract_features_strided_device(const void *obs, size_t obs_stride,
                                                      const void *mission,
                                                      size_t mission_stride,
                                                      const void *cameras,
                                                      size_t camera_stride, float *features,
                                                      size_t batch_size, void *stream) {
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
    rows.out = features;
    rows.batch = batch_size;
    return launch_features(rows, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int tb_hip_lidar_transform_device(const float *ranges, float *out, size_t count,
                                             void *stream) {
    if (!ranges || !out || count == 0) return 0;
    size_t want = (count + 255) / 256;
    const unsigned blocks = want > kMaxBlocks ? kMaxBlocks : (unsigned)want;
    lidar_transform_kernel<<<blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(ranges, out,
                                                                                      count);
    return hipGetLastError() == hipSuccess;
}

extern "C" int tb_cuda_synchronize(void *stream) {
    return hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)) == hipSuccess;
}
