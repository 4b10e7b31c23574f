// gfx950 kernel of the onboard tactical (24) and physics-prior (15) features.
//
// Semantics follow the reference device code
// src/network/onboard_features.cuh:6-519 (tb_onboard_tactical,
// tb_onboard_prior, tb_onboard_tactical_prior), which the reference runs as
// one thread per environment inside its actor input kernel
// (src/network/network_gpu.cu:274-304).  Here the two halves of the work get
// the execution shape that suits them:
//
//   * the LiDAR scan (two passes over 1,536 rays: closest return, corridor
//     minimum, cluster membership and y sum) runs one wave per environment,
//     24 rays per lane, so each load instruction reads 256 contiguous LiDAR
//     bytes and no workgroup barrier is needed.  The wave lists its
//     in-window rays in ray order (ballot + lane prefix) and runs both
//     passes over the list; above kListCap in-window rays it sweeps every
//     slot, branch-free, with the two heads' rays at the same azimuth and
//     elevation sharing the first two products of each rotated component.
//     The closest return is a 32-bit wave minimum of the range bits followed
//     by a lane-mask search for its first slot and lane (the first minimum
//     in the reference scan order); the corridor minimum is a DPP / permlane
//     fminf reduction, with a +0 / -0 tie settled as the reference's strict
//     < settles it (the first in ray order); the cluster count comes from
//     lane masks, and the cluster's y centres are added in float in ray
//     order, as the reference does, because the sign of that sum picks the
//     slalom lane.  The controller uses the closest return for dodge
//     missions only and the corridor and cluster for slalom missions only
//     (onboard_features.cuh:208-244), so unless the caller asks for the
//     scan's diagnostics each environment gets only the part its mission
//     uses, and the next environment's ranges are requested only as far as
//     it needs them.  In the onboard entry the environments whose mission
//     uses the scan are shared out over the 16 waves of a CU from a pool in
//     LDS, so the waves that would have drawn several slalom missions do
//     not set the kernel's time; the actor entry's scan, which also writes
//     the LiDAR channels of every environment, keeps a static share;
//   * the tactical features and the controller (mission decode, targets,
//     landing / standard / inversion / BWB laws, cannon) run in a second
//     kernel from the parked scan results, both on one quad of lanes per
//     environment (lane a evaluates arm a and a quarter of the independent
//     transcendental calls).  The controller's long register-heavy chain is
//     kept apart from the scan so both keep their occupancy, except where
//     the batch is one round of 64-environment workgroups over most CUs
//     (the onboard entry from 10,240 to 16,384 environments): there one
//     kernel does both, each workgroup scanning its own environments into
//     LDS before their controller runs, which saves the second launch and
//     the parked results' round trip.  The angles
//     that reach its angle wraps use a correctly rounded atan2: exact angles
//     (from equal or zero components) reach a wrap's discontinuity, where
//     one ulp flips the wrapped error's sign.
//
// Ray directions come from a table generated at build time with the host
// libm (gen_ray_table.c), and the scan arithmetic is evaluated without FMA
// contraction in the reference's operation order, so the per-ray world
// vectors, and with them the closest return, its ray index, the corridor
// minimum, the cluster count and the cluster y sum, are reproducible
// bit-for-bit against the unfused C restatement.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "turbinator/training/hip_features.h"
#include "recip_range.h"
#include "xcd_order.h"

#include "onboard_rays.inc"

namespace {

constexpr int kBlockThreads = 256;
constexpr int kWavesPerBlock = kBlockThreads / 64;
constexpr int kControlWaves = 4;  // control workgroup: waves 0..3 controller, 4..7 tactical
constexpr int kControlThreads = 2 * kControlWaves * 64;
constexpr int kScanRays = 1536 / 64;  // rays per lane: one wave scans one environment
// In-window rays a wave lists for the compact pass; with more, every slot is
// swept instead.
constexpr int kListCap = 512;
constexpr int kListRounds = kListCap / 64;
constexpr unsigned kMaxBlocks = 1u << 20;
constexpr int kStreamThreads = 1024;  // actor plane kernel: one workgroup per environment
constexpr unsigned kScanBlocks = 256 * 4;   // persistent scan grid: 4 per CU
// Controller grid cap: 4,096 workgroups of 64 environments.  One workgroup is
// resident per CU (205 VGPRs), so the cap is 16 full rounds of the chip and
// larger batches stride; a 16,384-environment call launches 256.
constexpr unsigned kControlBlocks = 4096;
constexpr size_t kMaxBatch = 0x7fffffffu;
constexpr float kPi = 3.14159265358979323846f;

struct ScanResult {
    float min_r, min_r_dx, min_r_dy, min_dx_c, cluster_y_sum;
    int min_ray, cluster_count, pad;
};

// x / c for a constant float c, as one double product.  For each constant
// this file divides by (10, 20, 30, 45, pi/6, pi/4 and the thrust span) the
// result equals the IEEE quotient for every finite float x
// (tests/csrc/check_div_by_constant.c, run over all 4.28e9 finite floats);
// the IEEE division is a ten-instruction dependent sequence.
__device__ __forceinline__ float div_const(float x, float c) {
    return (float)((double)x * (1.0 / (double)c));
}

// onboard_features.cuh:6-22
__device__ __forceinline__ float ob_clamp(float x, float lo, float hi) {
    if (__builtin_isnan(x)) return x;
    return fminf(hi, fmaxf(lo, x));
}
__device__ __forceinline__ float ob_obs(float x) {
    return __builtin_isnan(x) ? 0.0f : (__builtin_isinf(x) ? copysignf(1000.0f, x) : x);
}
__device__ __forceinline__ float ob_mission(float x) {
    return __builtin_isnan(x) ? 0.0f : (__builtin_isinf(x) ? copysignf(1.0f, x) : x);
}
// sinf and cosf of one argument through sincosf: one argument reduction
// instead of two, and the same bits as the separate calls for every float
// (checked over all 2^32 inputs on gfx950 by tests/csrc/check_sincos.hip).
struct SinCos {
    float s, c;
};
__device__ __forceinline__ SinCos sin_cos(float x) {
    SinCos r;
    sincosf(x, &r.s, &r.c);
    return r;
}
// atan2 rounded correctly, for the angles that reach an angle wrap (yaw,
// the goal and course bearings, the cannon azimuths, the outer gimbals).
// ob_wrap is discontinuous where its two angles differ by pi, and that is
// reached exactly by angles such as -3pi/4 and pi/4 (from equal or zero
// components), or pi and a yaw of +-0: there one ulp of either angle flips
// the wrapped error between about -pi and +pi and the controller's torques
// with it.  The single-precision atan2f can be an ulp from the correctly
// rounded value on such arguments; the host libm's atan2f, which the oracle
// calls, is correctly rounded on them (equal, opposite and zero components,
// results near +-pi: tests/csrc/check_atan2.hip), and so is the double
// evaluation rounded once.  Elsewhere either libm may be an ulp off, which
// moves the angles continuously.  The tactical terms and the wrap's own
// atan2 depend on their angles continuously and keep atan2f.
__device__ __forceinline__ float ob_atan2(float y, float x) {
    return (float)atan2((double)y, (double)x);
}
__device__ __forceinline__ float ob_wrap(float target, float current) {
    const SinCos d = sin_cos(target - current);
    return atan2f(d.s, d.c);
}
__device__ __forceinline__ float ob_norm3(float x, float y, float z) {
    return sqrtf(x * x + y * y + z * z);
}

// Normalised, sign-fixed attitude quaternion (onboard_features.cuh:105-109)
// and its rotation matrix rows (:137-145).
struct Attitude {
    float qw, qx, qy, qz;
    float r[9];
};

__device__ __forceinline__ Attitude attitude_of(float o6, float o7, float o8, float o9) {
    Attitude a;
    float qnorm = fmaxf(ob_norm3(o6, o7, o8), 0.0f);
    qnorm = fmaxf(sqrtf(qnorm * qnorm + o9 * o9), 1.0e-8f);
    const float sign = o6 < 0.0f ? -1.0f : 1.0f;
    a.qw = sign * o6 / qnorm;
    a.qx = sign * o7 / qnorm;
    a.qy = sign * o8 / qnorm;
    a.qz = sign * o9 / qnorm;
    const float qw = a.qw, qx = a.qx, qy = a.qy, qz = a.qz;
    a.r[0] = 1.0f - 2.0f * (qy * qy + qz * qz);
    a.r[1] = 2.0f * (qx * qy - qw * qz);
    a.r[2] = 2.0f * (qx * qz + qw * qy);
    a.r[3] = 2.0f * (qx * qy + qw * qz);
    a.r[4] = 1.0f - 2.0f * (qx * qx + qz * qz);
    a.r[5] = 2.0f * (qy * qz - qw * qx);
    a.r[6] = 2.0f * (qx * qz - qw * qy);
    a.r[7] = 2.0f * (qy * qz + qw * qx);
    a.r[8] = 1.0f - 2.0f * (qx * qx + qy * qy);
    return a;
}

// Wave-wide reductions without the LDS crossbar: DPP exchanges inside each
// row of 16 lanes (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror) and the gfx950 permlane swaps across rows (partner l^16, then
// l^32).  Each step hands every lane the pair {own value, partner value};
// the combining operations below are symmetric, so every lane ends with the
// whole-wave result.
template <int CTRL>
__device__ __forceinline__ int dpp_partner(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

template <bool SWAP32>
__device__ __forceinline__ int swap_pair(int v, int &other) {
    const auto s = SWAP32 ? __builtin_amdgcn_permlane32_swap(v, v, false, false)
                          : __builtin_amdgcn_permlane16_swap(v, v, false, false);
    other = s[1];
    return s[0];
}

__device__ __forceinline__ float wave_min(float v) {
    v = fminf(v, __int_as_float(dpp_partner<0xB1>(__float_as_int(v))));
    v = fminf(v, __int_as_float(dpp_partner<0x4E>(__float_as_int(v))));
    v = fminf(v, __int_as_float(dpp_partner<0x141>(__float_as_int(v))));
    v = fminf(v, __int_as_float(dpp_partner<0x140>(__float_as_int(v))));
    int o;
    float a = __int_as_float(swap_pair<false>(__float_as_int(v), o));
    v = fminf(a, __int_as_float(o));
    a = __int_as_float(swap_pair<true>(__float_as_int(v), o));
    return fminf(a, __int_as_float(o));
}

// Ray directions as three planes (x, y, z) of 1,536 floats in LDS.
struct RayPlanes {
    float d[3][1536];
};

__device__ __forceinline__ unsigned wave_min_u32(unsigned v) {
    v = min(v, (unsigned)dpp_partner<0xB1>((int)v));
    v = min(v, (unsigned)dpp_partner<0x4E>((int)v));
    v = min(v, (unsigned)dpp_partner<0x141>((int)v));
    v = min(v, (unsigned)dpp_partner<0x140>((int)v));
    int o;
    v = min((unsigned)swap_pair<false>((int)v, o), (unsigned)o);
    return min((unsigned)swap_pair<true>((int)v, o), (unsigned)o);
}

// Buffer resources (gfx9 word 3): loads read zero past num_records instead
// of faulting, so a resource of 0 bytes turns a prefetch into zeros (ranges
// outside the scan window) without a branch.  A branch-free prefetch also
// keeps the load counter exact: a load issued on one path only would make
// the compiler wait for every load at the join.
constexpr int kBufferWord3 = 0x00020000;
constexpr unsigned kObsRowBytes = 4148 * sizeof(float);
constexpr int kNontemporal = 2;  // cache policy bit 1 (nt)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t obs_rsrc(const float *obs, bool valid) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(obs), (short)0,
                                             valid ? (int)kObsRowBytes : 0, kBufferWord3);
}

// The 24 ranges lane l of an environment's wave owns: slot u = 2 row + half
// is ray 128 row + 64 half + l (row = 6 head + el), so slots run in ray
// order and each load instruction reads 256 contiguous LiDAR bytes.
// Elevation rows 4..5 are read through `upper`, which a caller that needs
// only the closest return (rows 0..3) gives 0 bytes: they then read zeros,
// outside the scan window.
__device__ __forceinline__ void load_ranges(__amdgpu_buffer_rsrc_t obs,
                                            __amdgpu_buffer_rsrc_t upper, int lane,
                                            float (&rg)[kScanRays]) {
#pragma unroll
    for (int u = 0; u < kScanRays; ++u) {
        const int row = u / 2, head = row / 6, el = row % 6;
        rg[u] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(
                       el < 4 ? obs : upper, 4 * (48 + lane),
                       4 * ((16 * head + el) * 128 + 64 * (u % 2)), kNontemporal));
    }
}

// onboard_features.cuh:105-109,137-145 (attitude rows) and :183 (py) of one
// environment: the frame of its scan.
struct ScanFrame {
    float r[9], py;
};

struct FrameObs {
    float o1, o6, o7, o8, o9, m4, m5;  // and the two mission values scan_need reads
};

__device__ __forceinline__ FrameObs load_frame_obs(const float *obs, const float *mission) {
    return FrameObs{obs[1], obs[6], obs[7], obs[8], obs[9], mission[4], mission[5]};
}

__device__ __forceinline__ ScanFrame scan_frame(FrameObs &v) {
    // An empty asm that takes the seven values waits for their loads once,
    // here, instead of letting each load sink to its use inside the branchy
    // non-finite mapping (one memory round trip each).
    asm volatile("" : "+v"(v.o1), "+v"(v.o6), "+v"(v.o7), "+v"(v.o8), "+v"(v.o9), "+v"(v.m4),
                 "+v"(v.m5));
    const Attitude att = attitude_of(ob_obs(v.o6), ob_obs(v.o7), ob_obs(v.o8), ob_obs(v.o9));
    ScanFrame f;
#pragma unroll
    for (int k = 0; k < 9; ++k) f.r[k] = att.r[k];
    f.py = ob_obs(v.o1);
    return f;
}

// One listed in-window ray: its range (bits) and ray index.
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ bool in_window(float range) {
    return (int)(range > 0.35f) & (int)(range < 11.5f);
}

// in_window as one unsigned compare of the bits: 0x3eb33334 is the least
// float above 0.35f and 0x41380000 is 11.5f; negative values, zeros, NaN
// and infinities all fall outside [0x3eb33334, 0x41380000).  The listed
// pass stores the difference `bits - kWindowLo` itself: it orders in-window
// ranges like the ranges, and kWindowSpan marks "none".
constexpr unsigned kWindowLo = 0x3eb33334u;             // least float above 0.35f
constexpr unsigned kWindowSpan = 0x41380000u - kWindowLo;  // 11.5f - kWindowLo
__device__ __forceinline__ unsigned window_offset(float range) {
    return __float_as_uint(range) - kWindowLo;
}

// The 618M actor's three LiDAR channels of one range (network_gpu.cu:
// 467-479): inverse range, range / 30 and validity.  Both the plane kernel
// and the scan kernel of the actor entry form them here.  The divisor of the
// inverse range lies in [0.2, 30] for every input (non-finite ranges clamp
// to 0.05 or 30), where recip_range is the IEEE quotient; it is formed on
// every lane and selected, without a branch.
__device__ __forceinline__ float lidar_channel(float range, int kind) {
    const bool valid = range > 0.0f && __builtin_isfinite(range);
    const float clamped = fmaxf(0.05f, fminf(30.0f, range));
    if (kind == 0) return valid ? recip_range(fmaxf(0.2f, clamped)) : 0.0f;
    if (kind == 1) return valid ? div_const(clamped, 30.0f) : 1.0f;
    return valid ? 1.0f : 0.0f;
}

// Buffer cache-policy bits of the actor entry's plane stores: nt (1) and
// sc1 (4).
constexpr int kStorePolicy = 2 | 16;

// onboard_features.cuh:199-207 for one ray with rotated direction rw:
// returns the corridor centre x (+inf when the ray is outside the window or
// the corridor) and sets y_center.  Bitwise, so the compares stay one
// straight-line block.
__device__ __forceinline__ float corridor_centre(float rwx, float rwy, float rwz, float range,
                                                 float py, float &y_center) {
    const float wx = rwx * range, wy = rwy * range, wz = rwz * range;
    const float x_center = wx + rwx * 1.10f;
    y_center = py + wy + rwy * 1.10f;
    const bool corridor = (int)in_window(range) & (int)(fabsf(wz) <= 2.1f) &
                          (int)(x_center >= -0.35f) & (int)(x_center <= 10.5f) &
                          (int)(fabsf(y_center) <= 3.5f);
    return corridor ? x_center : __builtin_huge_valf();
}

// sum + v[l0] + v[l1] + ... in float, one rounding per term, over the lanes
// of `members` in ascending order (onboard_features.cuh:231-234 adds each
// cluster ray's y_center in scan order; the sign of the sum decides the
// slalom lane at :238, so the reference's rounding sequence is kept).  The
// loop runs on the scalar unit, one v_readlane and one add per member.
__device__ __forceinline__ float add_in_lane_order(float sum, float v, uint64_t members) {
    while (members) {
        const int l = (int)__builtin_ctzll(members);
        sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
        members &= members - 1;
    }
    return sum;
}

// The 618M actor's three LiDAR channel planes of the wave's 1,536 rays,
// written into `planes`, the environment's [6][16][128] channel block: these
// rays are in the wave's registers already, so the actor entry reads them
// from HBM once, and its plane kernel writes only the other elevation rows.
// Slot u holds row 6 head + el, azimuths 64 (u % 2) + lane: channel kind k
// of head h is plane h + 2k, so each store writes 256 consecutive bytes of
// one plane row.
__device__ __forceinline__ void write_channel_planes(const float (&rg)[kScanRays],
                                                     __amdgpu_buffer_rsrc_t planes, int lane) {
#pragma unroll
    for (int u = 0; u < kScanRays; ++u) {
        const int row = u / 2, head = row / 6, el = row % 6;
#pragma unroll
        for (int kind = 0; kind < 3; ++kind)
            __builtin_amdgcn_raw_buffer_store_b32(
                __builtin_bit_cast(unsigned, lidar_channel(rg[u], kind)), planes, 4 * lane,
                4 * ((head + 2 * kind) * 2048 + el * 128 + 64 * (u % 2)), kStorePolicy);
    }
}

// What the controller uses of an environment's scan (onboard_features.cuh:
// 107-109 for the mission flags, :208-244 for the uses): a dodge mission
// uses the closest return (min_r and its world offset), a slalom mission the
// corridor minimum and the cluster, and every other mission none of it.
// The two flags exclude each other (dodge needs m5 > 0.75, slalom m5 <= 0.25).
constexpr int kNeedNone = 0, kNeedClosest = 1, kNeedCorridor = 2, kNeedAll = 3;

__device__ __forceinline__ int scan_need(float raw_m4, float raw_m5) {
    const float m4 = ob_mission(raw_m4), m5 = ob_mission(raw_m5);
    const bool lateral = m4 > 0.75f && m5 > 0.25f;
    const bool slalom = m4 > 0.75f && !lateral;
    const bool dodge = m5 > 0.75f;
    return slalom ? kNeedCorridor : (dodge ? kNeedClosest : kNeedNone);
}

// Lane 0's closest-return fields of `out` from the winning ray and range
// bits (onboard_features.cuh:202, the world offset in the reference's
// operation order).
__device__ __forceinline__ void closest_fields(int ray, unsigned min_bits, const RayPlanes &rays,
                                               const ScanFrame &f, ScanResult &out) {
    const float range = ray >= 0 ? __uint_as_float(min_bits) : 30.0f;
    out.min_r = range;
    out.min_r_dx = 0.0f;
    out.min_r_dy = 0.0f;
    out.min_ray = -1;
    if (ray >= 0) {
        const float dx = rays.d[0][ray], dy = rays.d[1][ray], dz = rays.d[2][ray];
        const float rwx = f.r[0] * dx + f.r[1] * dy + f.r[2] * dz;
        const float rwy = f.r[3] * dx + f.r[4] * dy + f.r[5] * dz;
        out.min_r_dx = rwx * range;
        out.min_r_dy = rwy * range;
        out.min_ray = ray;
    }
}

// onboard_features.cuh:184-234 for one environment, on one wave (24 rays per
// lane, no workgroup barrier).
//   * The reference maps non-finite ranges to 0 / +-1000 first; both fail
//     the 0.35 < r < 11.5 window, as NaN does, so the raw value is tested.
//     The reference skips rays outside the window (:193, :218), and so does
//     the common path here: the in-window rays are listed in the wave's
//     `list` (ballot + lane prefix count) and passes 1 and 2 run over the
//     list, 64 rays per instruction.  When more than kListCap rays are in
//     the window, every slot is swept instead (the same per-ray arithmetic).
//   * The closest return over elevation rows 0..3 is found straight from
//     the ranges, before any list, in two steps: the wave's minimum
//     in-window range (as bits: positive floats order like their bit
//     patterns), then the first slot in ray order and the first lane holding
//     exactly that range, from lane masks on the scalar unit.  That is the
//     reference's first minimum in scan order.  Lane 0 computes the winner's
//     world offset with the reference's expression.
//   * Pass 1 keeps each ray's corridor centre (x = +inf outside the window or
//     the corridor), so pass 2 is a compare-and-add.  The reference's
//     strict-< update over corridor rays is the minimum of their centres,
//     except that of a +0 and a -0 it keeps the first in ray order, which a
//     search over the zero centres restores when the minimum is zero.
//   * Once the ranges are consumed (listed, or swept by pass 1), the
//     registers take the next environment's (`next`, a 0-byte resource when
//     there is none): they have the rest of this environment to arrive.
//   * `f` and `need` are wave-uniform.  Only the corridor and cluster use
//     the list: with kNeedClosest only (a dodge mission) nothing is listed
//     and the corridor work is skipped; with kNeedCorridor only (slalom) the
//     closest-return search is skipped; with kNeedNone nothing is done.  The
//     fields skipped keep their empty values.
__device__ __forceinline__ void scan_env(float (&rg)[kScanRays], const RayPlanes &rays,
                                         const ScanFrame &f, __amdgpu_buffer_rsrc_t next,
                                         __amdgpu_buffer_rsrc_t next_upper, int lane,
                                         u32x2 *list, ScanResult &out, int need) {
    // Closest return, straight from the ranges: each lane's minimum over its
    // 16 slots of elevation rows 0..3 as bits (positive floats order like
    // their bits; a ray outside the window counts as 11.5, the window's
    // exclusive upper bound, so it never wins), the wave's minimum, then the
    // first slot (slots are in ray order) and its first lane holding exactly
    // that range: the reference's first minimum in scan order.
    constexpr unsigned kWindowTop = 0x41380000u;  // 11.5f
    unsigned min_bits = kWindowTop;
    int min_ray = -1;
    if (need & kNeedClosest) {
        unsigned lane_min = kWindowTop;
#pragma unroll
        for (int u = 0; u < kScanRays; ++u) {
            if ((u / 2) % 6 >= 4) continue;
            lane_min = min(lane_min, rg[u] > 0.35f ? __float_as_uint(rg[u]) : kWindowTop);
        }
        min_bits = wave_min_u32(lane_min);
        if (min_bits != kWindowTop) {
            // Visiting slots from the last to the first leaves the first slot
            // (in ray order) that holds the range, at its first lane.
#pragma unroll
            for (int u = kScanRays - 1; u >= 0; --u) {
                if ((u / 2) % 6 >= 4) continue;
                const uint64_t hit =
                    __builtin_amdgcn_ballot_w64(__float_as_uint(rg[u]) == min_bits);
                if (hit) min_ray = 64 * u + (int)__builtin_ctzll(hit);
            }
        }
    }

    // List the in-window rays in slot order while counting them: entry =
    // (range bits - kWindowLo, ray).  The slot's first entry address is
    // uniform (scalar), so each lane's address is one shift-add of its lane
    // prefix.  Once a slot's rays would overflow the list, counting stops:
    // n then exceeds kListCap and the list is not used.
    int n = 0;
#pragma unroll
    for (int u = 0; u < kScanRays; ++u) {
        // Only the corridor and cluster use the list.
        if (!(need & kNeedCorridor)) break;
        // A slot adds at most 64 entries, so the list can be full only from
        // slot kListCap / 64 + 1 on.
        if (64 * u > kListCap && n > kListCap) break;
        const unsigned off = window_offset(rg[u]);
        const bool in = off < kWindowSpan;
        const uint64_t m = __builtin_amdgcn_ballot_w64(in);
        // The lane's list position: the running count plus the in-window
        // lanes below it (mbcnt adds its second operand).  With n <= kListCap
        // every position is below kListCap + 64, inside the list and its
        // spare entries; a slot that takes the count past kListCap abandons
        // the list, so what it wrote there is never read.  Lanes outside the
        // window write to their own spare entry, so the store needs no
        // branch.
        unsigned pos = __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo((unsigned)m, (unsigned)n));
        asm volatile("" : "+v"(pos));  // formed on every lane, then selected
        *(list + (in ? pos : (unsigned)(kListCap + lane))) = u32x2{off, (unsigned)(64 * u + lane)};
        n += (int)__builtin_popcountll(m);
    }

    float min_dx_c = 30.0f;
    int count = 0;
    float y_sum = 0.0f;
    if (n <= kListCap) {
        // The list is written and read by this wave only.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        load_ranges(next, next_upper, lane, rg);
        // Round r's values exist only when 64 r < n, and every later loop
        // stops at the same bound (initialising the unused rounds cost
        // about 35 moves per environment).
        float xl[kListRounds], yl[kListRounds];
#pragma unroll
        for (int r = 0; r < kListRounds; ++r) {
            if (64 * r < n) {
                const int e = 64 * r + lane;
                const u32x2 entry = list[e];
                const bool valid = e < n;
                // Entries past n are left from earlier environments: they
                // read as 11.5 (kWindowSpan + kWindowLo), outside the window.
                const unsigned off = valid ? entry.x : kWindowSpan;
                const float range = __uint_as_float(off + kWindowLo);
                const int ray = valid ? (int)entry.y : 0;
                const float dx = rays.d[0][ray], dy = rays.d[1][ray], dz = rays.d[2][ray];
                const float rwx = f.r[0] * dx + f.r[1] * dy + f.r[2] * dz;
                const float rwy = f.r[3] * dx + f.r[4] * dy + f.r[5] * dz;
                const float rwz = f.r[6] * dx + f.r[7] * dy + f.r[8] * dz;
                xl[r] = corridor_centre(rwx, rwy, rwz, range, f.py, yl[r]);
                min_dx_c = fminf(min_dx_c, xl[r]);
            }
        }
        if (need & kNeedCorridor) {
            min_dx_c = wave_min(min_dx_c);
            if (min_dx_c == 0.0f) {
                // +0 and -0 tie; the reference keeps the first in ray order.
#pragma unroll
                for (int r = 0; r < kListRounds; ++r) {
                    if (64 * r >= n) break;
                    const uint64_t zero = __builtin_amdgcn_ballot_w64(xl[r] == 0.0f);
                    if (zero) {
                        min_dx_c = __int_as_float(__builtin_amdgcn_readlane(
                            __float_as_int(xl[r]), (int)__builtin_ctzll(zero)));
                        break;
                    }
                }
            }
            const float limit = min_dx_c + 1.4f;
#pragma unroll
            for (int r = 0; r < kListRounds; ++r) {
                if (64 * r >= n) break;
                const uint64_t members = __builtin_amdgcn_ballot_w64(xl[r] <= limit);
                count += __builtin_popcountll(members);
                y_sum = add_in_lane_order(y_sum, yl[r], members);
            }
        }
    } else {
        // Every slot.  The rays of rows el and el + 6 (heads 0 and 1) at the
        // same azimuth have the same table x, y and the negated z, bit for
        // bit.  With the reference's order (R0 d.x + R1 d.y) + R2 d.z the
        // head-1 sum is therefore P - Q where the head-0 sum is P + Q,
        // exactly (a + (-b) and a - b are the same IEEE operation), so each
        // pair reads one direction and forms P and Q once.
        float xc[kScanRays], yc[kScanRays];
        int min_slot = kScanRays;
#pragma unroll
        for (int el = 0; el < 6; ++el) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int ray = 128 * el + 64 * half + lane;
                const float dx = rays.d[0][ray], dy = rays.d[1][ray], dz = rays.d[2][ray];
                const float p0 = f.r[0] * dx + f.r[1] * dy, q0 = f.r[2] * dz;
                const float p1 = f.r[3] * dx + f.r[4] * dy, q1 = f.r[5] * dz;
                const float p2 = f.r[6] * dx + f.r[7] * dy, q2 = f.r[8] * dz;
#pragma unroll
                for (int head = 0; head < 2; ++head) {
                    const int u = 2 * (6 * head + el) + half;
                    xc[u] = corridor_centre(head ? p0 - q0 : p0 + q0, head ? p1 - q1 : p1 + q1,
                                            head ? p2 - q2 : p2 + q2, rg[u], f.py, yc[u]);
                    // The reference's strict < in ray order: the lane keeps
                    // its minimum at the lowest slot (slots are visited head
                    // innermost, not in ray order; equal values differ only
                    // as +0 / -0, which is settled across lanes below).
                    const bool lower = (int)(xc[u] < min_dx_c) |
                                       ((int)(xc[u] == min_dx_c) & (int)(u < min_slot));
                    min_dx_c = lower ? xc[u] : min_dx_c;
                    min_slot = lower ? u : min_slot;
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_ranges(next, next_upper, lane, rg);
        {
            // +0 and -0 tie; the reference keeps the first in ray order
            // (slot u holds rays 64 u .. 64 u + 63): the lowest ray among the
            // lanes' first zeros.  Formed on every environment and selected:
            // a branch here cost the kernel 50 VGPRs.
            const float lane_min = min_dx_c;
            min_dx_c = wave_min(lane_min);
            const unsigned key =
                lane_min == 0.0f ? 64u * (unsigned)min_slot + (unsigned)lane : ~0u;
            const float first_zero = __int_as_float(__builtin_amdgcn_readlane(
                __float_as_int(lane_min), (int)(wave_min_u32(key) & 63u)));
            min_dx_c = min_dx_c == 0.0f ? first_zero : min_dx_c;
        }
        // Pass 2: the cluster is counted from the lane masks (scalar unit)
        // and its y values summed in ray order (slot outer, lane inner).
        // All 24 masks are formed before the first sum: interleaving the
        // mask compares with the member loops took the kernel from 119 to
        // 182 VGPRs (2 waves per SIMD instead of 4).
        const float limit = min_dx_c + 1.4f;
        uint64_t members[kScanRays];
#pragma unroll
        for (int u = 0; u < kScanRays; ++u) {
            members[u] = __builtin_amdgcn_ballot_w64(xc[u] <= limit);
            count += __builtin_popcountll(members[u]);
        }
#pragma unroll
        for (int u = 0; u < kScanRays; ++u) y_sum = add_in_lane_order(y_sum, yc[u], members[u]);
    }
    if (lane == 0) {
        closest_fields(min_ray, min_bits, rays, f, out);
        out.min_dx_c = min_dx_c;
        out.cluster_count = count;
        out.cluster_y_sum = y_sum;
    }
}

// Lane k of every group of four (a quad) reads quad lane K's value.
template <int K>
__device__ __forceinline__ float quad_lane(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), K * 0x55, 0xF, 0xF, false));
}

// The four lanes' values of v, in every lane of the quad.
struct Quad4 {
    float v[4];
};
__device__ __forceinline__ Quad4 quad_all(float v) {
    return Quad4{{quad_lane<0>(v), quad_lane<1>(v), quad_lane<2>(v), quad_lane<3>(v)}};
}

// Quad lane a's choice among four values.
__device__ __forceinline__ float quad_pick(int a, float v0, float v1, float v2, float v3) {
    return a == 0 ? v0 : (a == 1 ? v1 : (a == 2 ? v2 : v3));
}

// onboard_features.cuh:25-86 on the four lanes of a quad: lane a evaluates
// arm a's thrust terms, and the independent calls of one function are spread
// over the quad and broadcast (the three atanhf of the mission offsets; yaw
// and the target bearing; the two hypotf and the two atan2f of the aim;
// eight tanhf in two calls), so a lane makes 11 library calls instead of
// the 25 of the per-environment chain.  Every call takes the arguments the
// reference's code gives it, and the arm sums are formed in its order from
// the broadcasts, so each feature is the value that code forms.  Lane a
// returns features 6a .. 6a + 5 in t, mapped as the reference maps them
// (NaN -> 0, +-inf -> +-1).
__device__ void tactical_quad(const float *o, const float *m, int a, float (&t)[6]) {
    const float pi = kPi;
    const float spool_a = ob_clamp(o[16 + a], 0.0f, 1.0f);
    const float thrust_a = 0.036f + 0.964f * spool_a;
    const float ci_a = cosf(o[28 + a]);
    const Quad4 spool = quad_all(spool_a);
    const Quad4 fz = quad_all(thrust_a * o[24 + a] * ci_a);
    const Quad4 tz = quad_all(thrust_a * o[20 + a] * ci_a);
    float tau_z = 0.0f, spool_mean = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        tau_z += tz.v[i];
        spool_mean += spool.v[i];
    }
    spool_mean *= 0.25f;
    float v[24];
    v[0] = fz.v[1] - fz.v[3];
    v[1] = fz.v[2] - fz.v[0];
    v[2] = 0.5f * tau_z;
    v[3] = 0.25f * (fz.v[0] + fz.v[1] + fz.v[2] + fz.v[3]) - 0.5f;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[4 + i] = 2.0f * (spool.v[i] - spool_mean);
    const float qw = o[6], qx = o[7], qy = o[8], qz = o[9];
    const float bz_x = 2.0f * (qx * qz + qw * qy);
    const float bz_y = 2.0f * (qy * qz - qw * qx);
    const float ct = ob_clamp(1.0f - 2.0f * (qx * qx + qy * qy), -1.0f, 1.0f);
    const float bx_x = 1.0f - 2.0f * (qy * qy + qz * qz);
    const float bx_y = 2.0f * (qx * qy + qw * qz);
    // rx, ry, rz on lanes 0, 1, 2 (lane 3 repeats rz).
    const float r_a = atanhf(ob_clamp(m[7 + (a < 2 ? a : 2)], -0.995f, 0.995f)) * 20.0f;
    const float rx = quad_lane<0>(r_a), ry = quad_lane<1>(r_a), rz = quad_lane<2>(r_a);
    // yaw on lane 0, the target bearing atan2f(ry, rx) on the others.
    const float at_a = atan2f(a == 0 ? bx_y : ry, a == 0 ? bx_x : rx);
    const float yaw = quad_lane<0>(at_a), bearing = quad_lane<1>(at_a);
    const SinCos yaw_sc = sin_cos(yaw);
    const float cy = yaw_sc.c, sy = yaw_sc.s;
    v[8] = cy * bz_y - sy * bz_x;
    v[9] = -sy * bz_y - cy * bz_x;
    v[10] = ct;
    v[11] = ct < 0.20f ? 1.0f : 0.0f;
    const float dist = fmaxf(ob_norm3(rx, ry, rz), 1.0f);
    const float flight = div_const(dist, 20.0f);
    const float wx = rx - o[3] * 0.5f * flight;
    const float wy = ry - o[4] * 0.5f * flight;
    const float wz = rz - o[5] * 0.5f * flight + 0.5f * 9.80665f * flight * flight;
    const float ux = -qx, uy = -qy, uz = -qz;
    const float cx = uy * wz - uz * wy + qw * wx;
    const float cyq = uz * wx - ux * wz + qw * wy;
    const float cz = ux * wy - uy * wx + qw * wz;
    const float bx = wx + 2.0f * (uy * cz - uz * cyq);
    const float by = wy + 2.0f * (uz * cx - ux * cz);
    const float bz = wz + 2.0f * (ux * cyq - uy * cx);
    // hypotf(rx, ry) on lane 0, hypotf(bx, by) on the others; then the aim's
    // azimuth on lane 0 and elevation on the others.
    const float hy_a = hypotf(a == 0 ? rx : bx, a == 0 ? ry : by);
    const float h_rxy = quad_lane<0>(hy_a), h_bxy = quad_lane<1>(hy_a);
    const float aim_a = atan2f(a == 0 ? by : bz, a == 0 ? bx : fmaxf(h_bxy, 0.2f));
    const float az = ob_clamp(quad_lane<0>(aim_a), pi / 12.0f, pi * 5.0f / 12.0f);
    const float el = ob_clamp(quad_lane<1>(aim_a), -pi / 6.0f, pi / 6.0f);
    const float err = hypotf(az - o[44], el - o[45]);
    const float th1 = tanhf(quad_pick(a, (cy * rx + sy * ry) * 0.08f, (-sy * rx + cy * ry) * 0.08f,
                                      rz * 0.12f, h_rxy * 0.05f));
    const float th2 = tanhf(quad_pick(a, (cy * o[3] + sy * o[4]) * 0.15f,
                                      (-sy * o[3] + cy * o[4]) * 0.15f, err * 2.0f, 0.0f));
    v[12] = quad_lane<0>(th1);
    v[13] = quad_lane<1>(th1);
    v[14] = quad_lane<2>(th1);
    v[15] = quad_lane<3>(th1);
    v[16] = quad_lane<0>(th2);
    v[17] = quad_lane<1>(th2);
    v[21] = quad_lane<2>(th2);
    v[18] = expf(-fmaxf(o[2] - 0.62f, 0.0f));
    v[19] = div_const(az - pi * 0.25f, pi / 6.0f);
    v[20] = div_const(el, pi / 6.0f);
    v[22] = (o[46] <= 0.02f && o[47] > 0.01f && err < 0.26f && dist < 34.0f) ? 1.0f : -1.0f;
    v[23] = sinf(bearing - pi * 0.25f - yaw);
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const float x = quad_pick(a, v[k], v[6 + k], v[12 + k], v[18 + k]);
        t[k] = __builtin_isnan(x) ? 0.0f : (__builtin_isinf(x) ? copysignf(1.0f, x) : x);
    }
}

// One lane's share of the prior features: its arm's throttle, outer and
// inner commands, and (identical in the four lanes) cannon azimuth,
// elevation and fire.
struct ArmOutputs {
    float throttle, outer, inner, az, el, fire;
};

// onboard_features.cuh:88-513 with the LiDAR passes replaced by `scan`, on
// the four lanes of a quad: lane a evaluates arm a's terms (the two per-arm
// loops, :114-125 and :376-391) and the four lanes repeat the shared chain,
// except that independent calls of one function are spread over the quad
// (four atan2, four atanh, four sine/cosine pairs, four angle wraps) and
// their results broadcast.  The arm sums and the running maximum are formed
// in the reference's order from quad broadcasts, so every value is the one
// the per-environment code forms.  The statements are reordered only where
// a value is needed earlier for such a group.
__device__ ArmOutputs prior_features(const float *input_obs, const float *input_mission,
                                     const ScanResult &scan, int a) {
    const float pi = kPi;
    const float max_installed = 294.2f * 0.85f;
    const float idle_frac = 0.08f;
    const float min_thrust = max_installed * idle_frac;
    const float gravity = 9.80665f;
    const float outer_limit = 2.0f;
    const float inner_limit = pi / 4.0f;
    const float cannon_az_ctr = pi / 4.0f;
    const float cannon_az_half = pi / 6.0f;
    const float cannon_el_lim = pi / 6.0f;
    float o[48], m[10];
#pragma unroll
    for (int i = 0; i < 48; ++i) o[i] = input_obs[i];
#pragma unroll
    for (int i = 0; i < 10; ++i) m[i] = input_mission[i];
    // The staged inputs the chain reads are all taken from LDS here, at
    // once: an empty asm on each value keeps the compiler from sinking its
    // read to the first use, where every read cost the chain its own LDS
    // round trip (51 waits on LDS in the kernel before, 29 after).
    float arm_in[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) arm_in[k] = input_obs[16 + 4 * k + a];
    {
        constexpr int kUsed[] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 40, 41, 44, 45, 46, 47};
#pragma unroll
        for (int i : kUsed) asm volatile("" : "+v"(o[i]));
#pragma unroll
        for (int i = 0; i < 10; ++i) asm volatile("" : "+v"(m[i]));
#pragma unroll
        for (int k = 0; k < 4; ++k) asm volatile("" : "+v"(arm_in[k]));
    }
#pragma unroll
    for (int i = 0; i < 48; ++i) o[i] = ob_obs(o[i]);
#pragma unroll
    for (int i = 0; i < 10; ++i) m[i] = ob_mission(m[i]);
    const float px = o[0], py = o[1], pz = o[2], vx = o[3], vy = o[4], vz = o[5];
    const Attitude att = attitude_of(o[6], o[7], o[8], o[9]);
    const float qw = att.qw, qx = att.qx, qy = att.qy, qz = att.qz;
    const float ux = -qx, uy = -qy, uz = -qz;
    const float r00 = att.r[0], r01 = att.r[1], r02 = att.r[2];
    const float r10 = att.r[3], r11 = att.r[4], r12 = att.r[5];
    const float r20 = att.r[6], r21 = att.r[7], r22 = att.r[8];
    const float ox = o[10], oy = o[11], oz = o[12];
    const float omega_norm = ob_norm3(ox, oy, oz);

    // Arm a of the four (this lane's); the quad exchanges the arm forces.
    const float spool = ob_clamp(ob_obs(arm_in[0]), 0.0f, 1.0f);
    const float thrust = max_installed * (idle_frac + (1.0f - idle_frac) * spool);
    const float outer = ob_atan2(ob_obs(arm_in[1]), ob_obs(arm_in[2]));
    const SinCos o_sc = sin_cos(outer);
    const float c_inner = cosf(ob_obs(arm_in[3]));
    const float fz_a = thrust * o_sc.c * c_inner;
    const float ft_a = thrust * o_sc.s * c_inner;
    const Quad4 fz = quad_all(fz_a), ft = quad_all(ft_a);
    float total_fz = 0.0f, jammed_yaw_ft = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        total_fz += fz.v[i];
        jammed_yaw_ft += ft.v[i];
    }
    const bool landing = m[1] > 0.75f;
    const bool cargo = m[2] > 0.75f;
    const bool inversion = m[3] > 0.75f && m[0] < -0.25f;
    const bool turbine_out = m[3] > 0.75f && m[2] < -0.25f;
    const bool lateral = m[4] > 0.75f && m[5] > 0.25f;
    const bool slalom = m[4] > 0.75f && !lateral;
    const bool dodge = m[5] > 0.75f;
    const bool arena = m[6] > 0.75f;
    const bool bwb_arena = m[6] > 0.75f && m[4] < -0.25f;
    const bool bwb_cruise = m[4] > 0.75f && m[2] > 0.25f;
    const bool bwb_intercept = m[6] > 0.75f && m[5] > 0.60f;
    const bool bwb_endurance = bwb_cruise && m[0] > 0.25f;
    const bool bwb = bwb_arena || bwb_cruise || bwb_intercept;
    const float fuel = ob_clamp(o[40], 0.0f, 1.0f) * 9.0f;
    const float ammo_mass = ob_clamp(o[47], 0.0f, 4.0f) * 6.0f;
    const bool payload = o[41] > 0.5f;
    const float mass = (arena ? 40.0f : 43.0f) + fuel + ammo_mass + (payload ? 30.0f : 0.0f);
    const float weight = mass * gravity;
    const float body_z_x = 2.0f * (qx * qz + qw * qy);
    const float body_z_y = 2.0f * (qy * qz - qw * qx);
    const float ct = ob_clamp(r22, -1.0f, 1.0f);
    const float tau_x_actual = fz.v[1] - fz.v[3];
    const float tau_y_actual = fz.v[2] - fz.v[0];
    const float az_actual = (total_fz * ct - weight) / mass;
    const bool heavy_cargo = cargo && payload;
    const bool landing_like = landing || heavy_cargo;

    // Independent calls of one function, one per lane of the quad: yaw, the
    // opponent bearing, the BWB roll and ground-track angles; the mission
    // offsets (atanh at the standard clamp, and the first at the BWB clamp).
    const Quad4 angles = quad_all(ob_atan2(quad_pick(a, r10, m[1], r21, vy),
                                         quad_pick(a, r00, m[2], r22, vx)));
    const float yaw = angles.v[0], opp_bearing = angles.v[1];
    const float roll_right = angles.v[2], track_yaw = angles.v[3];
    const Quad4 offsets = quad_all(atanhf(quad_pick(
        a, ob_clamp(m[7], -0.9995f, 0.9995f), ob_clamp(m[8], -0.9995f, 0.9995f),
        ob_clamp(m[9], -0.9995f, 0.9995f), ob_clamp(m[7], -0.9999f, 0.9999f))));

    const float relx = offsets.v[0] * 20.0f;
    const float rely = offsets.v[1] * 20.0f;
    const float relz = offsets.v[2] * 20.0f;
    float tx = (arena || lateral) ? px + relx : 0.0f;
    if (cargo) tx = 15.0f;
    if (slalom) tx = 36.0f;
    const float ty = (arena || lateral) ? py + rely : 0.0f;
    float tz = 8.0f;
    if (landing) tz = 0.60f;
    if (inversion) tz = 14.0f;
    if (cargo || arena) tz = pz + relz;
    float ex = tx, ey = ty, ez = tz;
    const float dx_opp = tx - px, dy_opp = ty - py;
    const float dxy = hypotf(dx_opp, dy_opp);
    const bool valid_d = dxy > 1.0e-3f;
    const float safe_d = valid_d ? dxy : 1.0f;
    const bool intercept = arena && m[0] > 0.75f && m[5] < -0.25f;
    const float desired_range = intercept ? 8.5f : 12.5f;
    float ax = valid_d ? tx - (dx_opp / safe_d) * desired_range : tx;
    float ay = valid_d ? ty - (dy_opp / safe_d) * desired_range : ty;
    const float scale = fminf(16.0f / fmaxf(hypotf(ax, ay), 1.0e-3f), 1.0f);
    ax *= scale;
    ay *= scale;
    const float pull = ob_clamp(div_const(hypotf(px, py) - 21.0f, 10.0f), 0.0f, 1.0f);
    ax *= 1.0f - pull;
    ay *= 1.0f - pull;
    const float az_t = pz < 8.0f || vz < -1.0f ? 12.2f : ob_clamp(tz, 8.5f, 12.2f);
    if (arena) { ex = ax; ey = ay; ez = az_t; }
    const float errx = ex - px, erry = ey - py;
    const float horiz_dist = hypotf(errx, erry);

    // Cannon aim point in the body frame (formed here so that its two
    // angles join the quad's next atan2 round).
    const float to_x = tx - px, to_y = ty - py, to_z = tz - pz;
    const float dist = fmaxf(ob_norm3(to_x, to_y, to_z), 1.0f);
    const float flight = div_const(dist, 20.0f);
    const float aim_x = to_x - vx * (0.65f * flight);
    const float aim_y = to_y - vy * (0.65f * flight);
    const float aim_z = to_z - vz * (0.65f * flight) + 0.53f * gravity * flight * flight;
    const float cx = uy * aim_z - uz * aim_y + qw * aim_x;
    const float cyq = uz * aim_x - ux * aim_z + qw * aim_y;
    const float cz = ux * aim_y - uy * aim_x + qw * aim_z;
    const float aim_bx = aim_x + 2.0f * (uy * cz - uz * cyq);
    const float aim_by = aim_y + 2.0f * (uz * cx - ux * cz);
    const float aim_bz = aim_z + 2.0f * (ux * cyq - uy * cx);
    const Quad4 bearings = quad_all(ob_atan2(
        quad_pick(a, ty - py, scan.min_r_dy, aim_by, aim_bz),
        quad_pick(a, tx - px, scan.min_r_dx, aim_bx, fmaxf(hypotf(aim_bx, aim_by), 0.2f))));
    const float raw_bearing = bearings.v[0], min_az = bearings.v[1];
    const float des_cannon_az =
        ob_clamp(bearings.v[2], cannon_az_ctr - cannon_az_half, cannon_az_ctr + cannon_az_half);
    const float des_cannon_el = ob_clamp(bearings.v[3], -cannon_el_lim, cannon_el_lim);

    // Sine and cosine of yaw, of the closest return's bearing, of the BWB
    // roll, and of the slalom hill phase.
    const float hill = ob_clamp(div_const(px - 6.0f, 30.0f), 0.0f, 1.0f);
    const SinCos sc = sin_cos(quad_pick(a, yaw, min_az, roll_right, pi * hill));
    const Quad4 sines = quad_all(sc.s), cosines = quad_all(sc.c);
    const float cyaw = cosines.v[0], syaw = sines.v[0];

    float avoid_x = 0.0f, avoid_y = 0.0f, slalom_speed = 3.8f, nearest_dx = 30.0f;
    if (dodge && scan.min_r < 7.5f) {
        avoid_x = -sines.v[1] * 2.2f;
        avoid_y = cosines.v[1] * 2.2f;
    }
    const float min_dx_c = scan.min_dx_c;
    const int cluster_count = scan.cluster_count;
    const float cluster_y = scan.cluster_y_sum / fmaxf((float)cluster_count, 1.0f);
    const bool has_slalom_obs = slalom && horiz_dist > 2.5f && min_dx_c < 10.2f &&
                                cluster_count > 0;
    if (has_slalom_obs) {
        nearest_dx = min_dx_c;
        ey = cluster_y >= 0.0f ? -1.85f : 1.85f;
    }
    const float lane_err = fabsf(py - ey);
    float speed_limit = lane_err > 0.55f ? 2.75f : 4.10f;
    if (lane_err > 1.05f) speed_limit = 1.55f;
    if (min_dx_c >= 6.6f && px > 4.0f) speed_limit = 3.10f;
    if (has_slalom_obs) slalom_speed = speed_limit;
    if (slalom && horiz_dist > 3.5f) ez = 2.5f * sines.v[3] + 8.0f;
    const float upx = ex - px, upy = ey - py, upz = ez - pz;
    const float up_horiz = hypotf(upx, upy);
    const bool active_slalom = slalom && nearest_dx < 10.2f && horiz_dist > 3.0f;

    const float pad_z = fmaxf(ez, 0.60f), above_pad = pz - pad_z;
    const float horiz_speed = hypotf(vx, vy);
    const float transit_cap = heavy_cargo ? 2.65f : 3.4f;
    const float low_cap = above_pad < 1.2f ? 0.55f : (heavy_cargo ? 1.25f : 1.6f);
    const float max_vxy_land = up_horiz > 1.8f ? transit_cap : low_cap;
    const float kp_land = heavy_cargo ? 0.75f : 1.05f;
    const float des_vx_land = ob_clamp(kp_land * upx, -max_vxy_land, max_vxy_land);
    const float des_vy_land = ob_clamp(kp_land * upy, -max_vxy_land, max_vxy_land);
    const float vz_land_touch = pz > 0.635f ? -0.16f : 0.0f;
    const float vz_land_cargo = ob_clamp(1.6f * (0.64f - pz), -0.30f, 0.18f);
    const float vz_land_low = cargo ? vz_land_cargo : vz_land_touch;
    const float max_desc = cargo ? -0.82f : -1.4f;
    const float vz_land_mid = ob_clamp(-0.70f * above_pad, max_desc, -0.25f);
    const float vz_land_align = ob_clamp(1.2f * (pad_z + 0.90f - pz), -0.30f, 0.60f);
    const float transit_z = heavy_cargo ? fmaxf(1.2f + 0.28f * up_horiz, 2.0f) : 2.0f;
    const float max_desc_trans = heavy_cargo ? -1.05f : -1.6f;
    const float vz_land_trans = ob_clamp(1.3f * (transit_z - pz), max_desc_trans, 1.4f);
    float des_vz_land = above_pad > 1.05f ? vz_land_mid : vz_land_low;
    if ((up_horiz > 0.85f || horiz_speed > 0.65f) && above_pad < 0.95f)
        des_vz_land = vz_land_align;
    if (up_horiz > 1.8f) des_vz_land = vz_land_trans;
    const float max_axy_land = heavy_cargo ? 2.2f : 2.6f;
    const float des_ax_land = ob_clamp(2.4f * (des_vx_land - vx), -max_axy_land, max_axy_land);
    const float des_ay_land = ob_clamp(2.4f * (des_vy_land - vy), -max_axy_land, max_axy_land);
    const float kp_az_land = heavy_cargo ? 5.0f : 4.5f;
    const float kd_az_land = heavy_cargo ? 1.0f : 0.80f;
    const float min_az_land = heavy_cargo ? -1.8f : -2.8f;
    const float des_az_land = ob_clamp(kp_az_land * (des_vz_land - vz) - kd_az_land * az_actual,
                                       min_az_land, 5.5f);

    const float inv_max_v = up_horiz > 9.0f && fabsf(upz) < 2.5f && ct > 0.90f ? 6.2f : 4.2f;
    const float lat_vx = fabsf(upy) > 1.35f ? 1.45f : 3.8f;
    float max_vx = arena ? 3.2f : 3.0f;
    if (inversion) max_vx = inv_max_v;
    float max_vy = max_vx;
    if (lateral) { max_vx = lat_vx; max_vy = 3.4f; }
    if (slalom) max_vx = 3.5f;
    if (active_slalom) { max_vx = slalom_speed; max_vy = 3.2f; }
    const float max_vz = vz < -2.0f || inversion ? 6.5f : 2.6f;
    const float kp_xy = inversion ? 0.85f : (lateral ? 0.95f : 0.90f);
    const float kp_vx = active_slalom ? 1.25f : kp_xy;
    const float kp_vy = active_slalom ? 1.45f : (lateral ? 1.05f : kp_xy);
    const float des_vx = ob_clamp(kp_vx * upx + avoid_x, -max_vx, max_vx);
    const float des_vy = ob_clamp(kp_vy * upy + avoid_y, -max_vy, max_vy);
    float des_vz = ob_clamp(1.25f * upz, -2.6f, max_vz);
    if ((inversion || arena) && vz < -1.0f) des_vz = fmaxf(des_vz, 0.8f);
    const float kp_ax = active_slalom ? 3.0f : 2.4f;
    const float kp_ay = active_slalom ? 3.0f : 2.6f;
    const float des_ax_std = ob_clamp(kp_ax * (des_vx - vx), -3.8f, 3.8f);
    const float des_ay_std = ob_clamp(kp_ay * (des_vy - vy), -3.8f, 3.8f);
    const float max_az = vz < -1.8f || inversion ? 14.0f : 6.5f;
    const float des_az_std = ob_clamp(3.8f * (des_vz - vz) - 0.80f * az_actual, -4.0f, max_az);
    const float des_ax = landing_like ? des_ax_land : des_ax_std;
    const float des_ay = landing_like ? des_ay_land : des_ay_std;
    const float des_az = landing_like ? des_az_land : des_az_std;

    const float tilt = acosf(ct);
    const bool need_headroom = inversion || arena || ct < 0.88f;
    const bool urgent_climb = arena && (pz < 8.5f || vz < -1.2f) && ct > 0.58f;
    const float max_coll =
        urgent_climb ? 3.95f
                     : (need_headroom
                            ? ob_clamp(3.95f - 0.90f * omega_norm - 1.30f * tilt, 2.55f, 3.95f)
                            : 3.95f);
    const float fz_des = ob_clamp((weight + mass * des_az) / fmaxf(ct, 0.45f), 0.10f * weight,
                                  max_coll * max_installed);
    const float horiz_scale =
        urgent_climb ? 0.0f
                     : (need_headroom
                            ? ob_clamp(1.0f - 1.5f * fmaxf(tilt - 0.15f, 0.0f), 0.0f, 1.0f)
                            : 1.0f);
    const float tilt_comp = turbine_out ? 0.65f : 0.0f;
    const float damp_v = active_slalom ? 0.8f : 0.4f;
    const float fx_world =
        (mass * des_ax + damp_v * vx - tilt_comp * total_fz * body_z_x) * horiz_scale;
    const float fy_world =
        (mass * des_ay + damp_v * vy - tilt_comp * total_fz * body_z_y) * horiz_scale;
    const float max_fh =
        active_slalom ? 105.0f : (lateral ? 125.0f : (heavy_cargo ? 52.0f : 80.0f));
    const float fx_body = ob_clamp(cyaw * fx_world + syaw * fy_world, -max_fh, max_fh);
    const float fy_body = ob_clamp(-syaw * fx_world + cyaw * fy_world, -max_fh, max_fh);

    const float cw_x = body_z_y, cw_y = -body_z_x;
    const float tt_x = 2.0f * (-uz * cw_y), tt_y = 2.0f * (uz * cw_x);
    const float tt_z = 2.0f * (ux * cw_y - uy * cw_x);
    const float te_x = cw_x + qw * tt_x + (uy * tt_z - uz * tt_y);
    const float te_y = cw_y + qw * tt_y + (uz * tt_x - ux * tt_z);
    const float te_z = qw * tt_z + (ux * tt_y - uy * tt_x);
    const float te_norm = ob_norm3(te_x, te_y, te_z);
    const float tilt_scale = te_norm > 1.0e-5f ? tilt / fmaxf(te_norm, 1.0e-5f) : 0.0f;
    const float e_rx = te_x * tilt_scale, e_ry = te_y * tilt_scale;

    const bool inv_hold_yaw = (inversion || arena) && (pz < 6.0f || vz < -0.5f || ct < 0.88f);
    const bool opp_bearing_valid = arena && fabsf(m[1]) + fabsf(m[2]) > 0.1f;
    const float target_bearing = opp_bearing_valid ? opp_bearing : raw_bearing;
    const float desired_yaw = arena && horiz_dist > 1.0f && !inv_hold_yaw
                                  ? target_bearing - cannon_az_ctr
                                  : (inv_hold_yaw ? yaw : 0.0f);

    // BWB geometry (onboard_features.cuh:437-510), up to the angles its two
    // wraps need; the control law follows after the shared part.
    float vb_x = 0.0f, vb_y = 0.0f, brx = 0.0f, bry = 0.0f, btx = 0.0f, bty = 0.0f, gz = 0.0f;
    float gdist = 0.0f, gamma_des = 0.0f, bdist = 0.0f, bbx = 0.0f;
    float desired_yaw_b = 0.0f, course_yaw = 0.0f, b_az = 0.0f, b_el = 0.0f;
    if (bwb) {
        vb_x = r00 * vx + r10 * vy + r20 * vz;
        vb_y = r01 * vx + r11 * vy + r21 * vz;
        brx = offsets.v[3] * 20.0f;
        const Quad4 b_offsets = quad_all(atanhf(quad_pick(a, ob_clamp(m[8], -0.9999f, 0.9999f),
                                                          ob_clamp(m[9], -0.9999f, 0.9999f),
                                                          0.0f, 0.0f)));
        bry = b_offsets.v[0] * 20.0f;
        const float brz = b_offsets.v[1] * 20.0f;
        btx = px + brx;
        bty = py + bry;
        float btz = pz + brz;
        const float rxy = hypotf(px, py);
        const float pull_b = ob_clamp(div_const(rxy - 235.0f, 45.0f), 0.0f, 0.85f);
        if (arena && rxy > 235.0f) { btx *= 1.0f - pull_b; bty *= 1.0f - pull_b; }
        if (arena) btz = ob_clamp(btz, 28.0f, 135.0f);
        const float gx = btx - px, gy = bty - py;
        gz = btz - pz;
        gdist = fmaxf(ob_norm3(gx, gy, gz), 1.0f);
        const float gs = hypotf(vx, vy);
        course_yaw = gs > 2.5f ? track_yaw : yaw;
        const float climb_des = ob_clamp(0.42f * gz, -5.0f, 5.0f);
        const float oppx = brx - vx * 0.10f, oppy = bry - vy * 0.10f, oppz = brz - vz * 0.10f;
        bdist = fmaxf(ob_norm3(oppx, oppy, oppz), 1.0f);
        const bool head_on = bwb_arena && btx * px + bty * py < -800.0f && bdist > 45.0f;
        const float closing = head_on ? 75.0f + 2.0f * fmaxf(vb_x, 0.0f) : 75.0f;
        const float bflight = bdist / closing;
        const float bax = oppx, bay = oppy;
        const float baz =
            oppz + (head_on ? -vz * (0.85f * bflight) : 0.0f) + 0.50f * gravity * bflight * bflight;
        bbx = r00 * bax + r10 * bay + r20 * baz;
        const float bby = r01 * bax + r11 * bay + r21 * baz;
        const float bbz = r02 * bax + r12 * bay + r22 * baz;
        const Quad4 b_angles = quad_all(ob_atan2(
            quad_pick(a, gy, climb_des, bby, bbz),
            quad_pick(a, gx, fmaxf(gs, 14.0f), fmaxf(bbx, 0.2f), fmaxf(hypotf(bbx, bby), 0.2f))));
        desired_yaw_b = b_angles.v[0];
        gamma_des = b_angles.v[1];
        b_az = ob_clamp(b_angles.v[2], -pi / 6.0f, pi / 6.0f);
        b_el = ob_clamp(b_angles.v[3], -cannon_el_lim, cannon_el_lim);
    }

    // The four angle wraps, one per lane: yaw error, cannon azimuth error,
    // BWB course error, BWB cannon azimuth error.
    const Quad4 wraps = quad_all(ob_wrap(quad_pick(a, desired_yaw, des_cannon_az, desired_yaw_b,
                                                   b_az),
                                         quad_pick(a, yaw, o[44], course_yaw, o[44])));
    const float yaw_err = wraps.v[0];

    const float parasite_scale = turbine_out ? 0.35f : 1.0f;
    const float tau_x_par = -0.1625f * fy_body * parasite_scale;
    const float tau_y_par = 0.1625f * fx_body * parasite_scale;
    const float tau_x_net = tau_x_actual + tau_x_par;
    const float tau_y_net = tau_y_actual + tau_y_par;
    const float max_txy = heavy_cargo ? 120.0f : 260.0f;
    const float tau_x_cmd = ob_clamp(95.0f * e_rx - 64.0f * ox - 0.90f * tau_x_net - tau_x_par,
                                     -max_txy, max_txy);
    const float tau_y_cmd = ob_clamp(95.0f * e_ry - 64.0f * oy - 0.90f * tau_y_net - tau_y_par,
                                     -max_txy, max_txy);
    const float tau_z_cmd = ob_clamp(22.0f * yaw_err - 18.0f * oz, -70.0f, 70.0f);
    // {q - ty, q + tx, q + ty, q - tx}[a]; q - t and q + (-t) are the same
    // IEEE operation.
    const float half_tx = tau_x_cmd * 0.5f, half_ty = tau_y_cmd * 0.5f;
    const float fz_cmd = 0.25f * fz_des + quad_pick(a, -half_ty, half_tx, half_ty, -half_tx);
    const float yaw_ft = (tau_z_cmd - 0.40f * jammed_yaw_ft) * 0.25f;
    float outer_cmd, inner_cmd, throttle;
    const float fx_outer = ft.v[3] - ft.v[1];
    const float fy_outer = ft.v[0] - ft.v[2];
    const float fx_rem = fx_body - fx_outer, fy_rem = fy_body - fy_outer;
    const float max_sin_inner =
        lateral ? 0.44f : (active_slalom ? 0.42f : (heavy_cargo ? 0.22f : 0.32f));
    const float spool_gain = turbine_out ? 10.5f : (heavy_cargo ? 4.5f : 2.4f);
    const bool land_idle = landing && pz <= 0.638f && up_horiz < 0.85f && fabsf(vz) < 0.20f;
    const float yaw_alpha = asinf(ob_clamp(yaw_ft / fmaxf(thrust, 30.0f), -0.35f, 0.35f));
    outer_cmd = ob_clamp(6.5f * ob_wrap(yaw_alpha, outer), -outer_limit, outer_limit);
    const float urx = quad_pick(a, 1.0f, 0.0f, -1.0f, 0.0f);
    const float ury = quad_pick(a, 0.0f, 1.0f, 0.0f, -1.0f);
    const float fr_req = 0.5f * (fx_rem * urx + fy_rem * ury);
    const float sin_in = ob_clamp(fr_req / fmaxf(thrust, 40.0f), -max_sin_inner, max_sin_inner);
    inner_cmd = ob_clamp(asinf(sin_in), -inner_limit * 0.90f, inner_limit * 0.90f);
    const float nominal_cos = fmaxf(cosf(yaw_alpha) * cosf(inner_cmd), 0.70f);
    float target_thrust = fmaxf(fz_cmd, 0.0f) / nominal_cos;
    if (land_idle) target_thrust = 0.15f * weight * 0.25f;
    const float u_des =
        ob_clamp(div_const(target_thrust - min_thrust, max_installed - min_thrust), 0.0f, 1.0f);
    const float u_raw = u_des + spool_gain * (u_des - spool);
    // The reference's running maximum over arms 0..3, from -inf.
    const Quad4 u_all = quad_all(u_raw);
    float max_raw = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 4; ++i) max_raw = fmaxf(max_raw, u_all.v[i]);
    const float excess = ob_clamp(max_raw - 1.0f, 0.0f, urgent_climb ? 0.10f : 0.45f);
    throttle = ob_clamp(u_raw - (need_headroom ? excess : 0.0f), 0.0f, 1.0f);
    const bool inv_mode = ct < 0.20f;
    if (inv_mode) {
        const float inv_rx = te_norm > 1.0e-5f ? e_rx : tilt;
        const float tx_inv = 130.0f * inv_rx - 52.0f * ox;
        const float ty_inv = 130.0f * e_ry - 52.0f * oy;
        const float arm_mom = quad_pick(a, -ty_inv, tx_inv, ty_inv, -tx_inv);
        throttle = arm_mom > 12.0f ? 0.58f : 0.0f;
        outer_cmd = ob_clamp(-outer * 6.0f, -outer_limit, outer_limit);
        inner_cmd = 0.0f;
    }

    const float aim_err = hypotf(wraps.v[1], des_cannon_el - o[45]);
    const bool fire = arena && !inv_mode && o[46] <= 0.02f && o[47] > 0.01f && aim_err < 0.28f &&
                      dist < 34.0f;
    const bool cannon = arena && !inv_mode;
    float norm_az =
        cannon ? ob_clamp(div_const(des_cannon_az - cannon_az_ctr, cannon_az_half), -1.0f, 1.0f) : 0.0f;
    if (inv_mode) norm_az = -1.0f;
    float norm_el = cannon ? ob_clamp(div_const(des_cannon_el, cannon_el_lim), -1.0f, 1.0f) : 0.0f;
    float norm_fire = fire ? 0.8f : -0.8f;

    if (bwb) {
        const float course_err = wraps.v[2];
        const float desired_speed =
            bwb_endurance ? 18.5f : (arena ? (gdist > 38.0f ? 26.0f : 24.0f) : 22.4f);
        const float speed_err = desired_speed - vb_x;
        const float u_coll = ob_clamp((bwb_endurance ? 0.36f : 0.44f) + 0.065f * speed_err +
                                          0.018f * gz, 0.12f, 0.90f);
        const float desired_roll = ob_clamp(-1.35f * course_err, -0.55f, 0.55f);
        const float diff_u =
            ob_clamp(0.90f * (desired_roll - roll_right) - 0.34f * ox, -0.45f, 0.45f);
        const float u0 = ob_clamp(u_coll + diff_u, 0.05f, 1.0f);
        const float u1 = ob_clamp(u_coll - diff_u, 0.05f, 1.0f);
        throttle = (a & 1) ? u1 : u0;
        const float pitch_up = asinf(ob_clamp(r20, -1.0f, 1.0f));
        const float climb_des = ob_clamp(0.42f * gz, -5.0f, 5.0f);
        const float climb_err = climb_des - vz;
        const float cos_bank = cosines.v[2], sin_bank = sines.v[2];
        float desired_pitch = ob_clamp(0.062831853f + 0.75f * gamma_des + 0.035f * climb_err +
                                           0.09f * (1.0f - fmaxf(cos_bank, 0.5f)),
                                       -0.15f, 0.25f);
        if (vb_x < 15.5f) desired_pitch = fminf(desired_pitch, 0.02f);
        const float theta_dot = 2.20f * (desired_pitch - pitch_up);
        const float psi_dot = (gravity / fmaxf(vb_x, 12.0f)) *
                                  tanf(ob_clamp(-roll_right, -0.75f, 0.75f)) +
                              0.35f * course_err;
        const float q_up = cos_bank * theta_dot - sin_bank * psi_dot;
        const float r_left = sin_bank * theta_dot + cos_bank * psi_dot;
        const float gimbal = pi / 6.0f;
        const float inner0 = ob_clamp(0.85f * (q_up + oy) + 0.03f, -gimbal, gimbal);
        const float inner1 = ob_clamp(-0.65f * (r_left - oz) - 0.025f * vb_y, -gimbal, gimbal);
        inner_cmd = quad_pick(a, inner0, inner1, 0.0f, 0.0f);
        outer_cmd = 0.0f;
        const float b_err = hypotf(wraps.v[3], b_el - o[45]);
        const bool b_fire = arena && o[46] <= 0.02f && o[47] > 0.01f && b_err < 0.045f &&
                            bdist < 165.0f && bbx > 0.0f;
        norm_az = arena ? ob_clamp(div_const(b_az, pi / 6.0f), -1.0f, 1.0f) : 0.0f;
        norm_el = arena ? ob_clamp(div_const(b_el, cannon_el_lim), -1.0f, 1.0f) : 0.0f;
        norm_fire = b_fire ? 0.8f : -0.8f;
    }
    ArmOutputs out;
    out.throttle = ob_clamp(throttle * 2.0f - 1.0f, -1.0f, 1.0f);
    out.outer = ob_clamp(outer_cmd / outer_limit, -1.0f, 1.0f);
    out.inner = ob_clamp(div_const(inner_cmd, inner_limit), -1.0f, 1.0f);
    out.az = norm_az;
    out.el = norm_el;
    out.fire = norm_fire;
    return out;
}

struct OnboardRows {
    const unsigned char *obs;
    size_t obs_stride;
    const unsigned char *mission;
    size_t mission_stride;
    float *tactical;
    float *prior;
    float *diag;
    float *proprio;      // optional [batch, 91]: tactical -> 52..75, prior -> 76..90
    float *mission_vec;  // optional [batch, 49]: tactical -> 10..33, prior -> 34..48
    float *lidar;        // optional [batch, 6, 16, 128]: channels of the scan rays
    size_t batch;
};

// log1p(x) for x >= 0 (any magnitude): 1 + x = u + c exactly (Fast2Sum),
// log1p(x) = log2(u)*ln2 + c/u with ln2 as a hi+lo pair.
__device__ __forceinline__ float log1p_pos(float x) {
    const float a = fmaxf(x, 1.0f), b = fminf(x, 1.0f);
    const float u = a + b;
    const float c = b - (u - a);
    const float l2 = __builtin_amdgcn_logf(u);
    const float t = c * __builtin_amdgcn_rcpf(u);
    const float r = __builtin_fmaf(l2, 0x1.62e43p-1f, __builtin_fmaf(l2, -0x1.05c61p-29f, t));
    return x == 0.0f ? x : r;
}

__device__ __forceinline__ float actor_scale(int i) {  // network_gpu.cu:287-293
    if (i < 3) return 0.05f;
    if (i < 6) return 0.10f;
    if (i >= 10 && i < 13) return 0.20f;
    if (i >= 13 && i < 16) return 0.10f;
    if (i >= 28 && i < 32) return 0.50f;
    if (i >= 32 && i < 36) return 0.20f;
    return 1.0f;
}

// network_gpu.cu:285-297 (scalar_inputs): lanes 0..51 of a wave write the
// environment's 52 symlog scalars, lanes 52..61 its 10 finite mission values.
// The input of lane l is obs[l] (l < 48), obs[4144 + l - 48] (l < 52) or
// mission[l - 52] (l < 62).  Branch-free: every lane forms both values, and
// buffer stores (discarded past num_records) write lanes 0..51 into proprio
// and 52..61 into mission_vec; an environment that is not `valid` writes
// nothing.
constexpr int kPastRecords = 0x40000000;  // past every resource
// RN_double(1 / sqrtf(1.0001f)): (float)((double)x * this) equals the IEEE
// quotient x / sqrtf(1.0001f) for every float |x| <= 8 (checked
// exhaustively by tests/csrc/check_div_by_constant.c), and |symlog| < 7.
constexpr double kInvSqrt10001 = 0x1.fff974156e01ep-1;

__device__ __forceinline__ void actor_scalars(float raw, int lane, float *proprio,
                                              float *mission_vec, bool valid) {
    const bool finite = __builtin_isfinite(raw);
    const float clamped = finite ? fmaxf(-1000.0f, fminf(1000.0f, raw)) : 0.0f;
    const float symlog = copysignf(log1p_pos(fabsf(clamped * actor_scale(lane))), clamped);
    const float scaled = fmaxf(-8.0f, fminf(8.0f, (float)((double)symlog * kInvSqrt10001)));
    __builtin_amdgcn_raw_buffer_store_b32(
        __builtin_bit_cast(unsigned, scaled),
        __builtin_amdgcn_make_buffer_rsrc(proprio, (short)0, valid ? 52 * 4 : 0, kBufferWord3),
        lane < 52 ? 4 * lane : kPastRecords, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(
        __builtin_bit_cast(unsigned, finite ? raw : 0.0f),
        __builtin_amdgcn_make_buffer_rsrc(mission_vec, (short)0, valid ? 10 * 4 : 0,
                                          kBufferWord3),
        lane >= 52 && lane < 62 ? 4 * (lane - 52) : kPastRecords, 0, 0);
}

// A scan result parked in its environment's prior row (7 of its 15 words)
// until the control kernel has read it.
__device__ __forceinline__ void park_scan(float *park, const ScanResult &s) {
    park[0] = s.min_r;
    park[1] = s.min_r_dx;
    park[2] = s.min_r_dy;
    park[3] = s.min_dx_c;
    park[4] = s.cluster_y_sum;
    park[5] = __int_as_float(s.min_ray);
    park[6] = __int_as_float(s.cluster_count);
}

// Phase 1 of the actor entry, and of the onboard entry below 2,560
// environments.  Each wave scans one environment at a time;
// workgroups are persistent (the ray table is loaded into LDS once per
// workgroup, the only barrier).  Wave g of the grid takes environments g,
// g + W, g + 2W, ... (W waves in the grid).  Their scan frames (attitude
// rows, py) and scan needs (scan_need) are formed up front, lane j for the
// wave's j-th environment, and each environment's frame and need are then
// read from its lane into scalar registers.  Each environment's ranges are
// requested while the previous one finishes, as far as its need goes (the
// PLANES form reads every range: it writes the LiDAR channels of each
// environment's scan rays).  The 32-byte result is parked in the
// environment's own prior row (60 bytes), which phase 2 reads before it
// writes the 15 prior values there: no scratch memory is needed.
template <bool PLANES>
__global__ __launch_bounds__(kBlockThreads) void onboard_scan_kernel(OnboardRows rows) {
    __shared__ RayPlanes rays;
    __shared__ u32x2 lists[kWavesPerBlock][kListCap + 64];  // + a spare entry per lane
    const int tid = threadIdx.x, lane = tid & 63;
    for (int i = tid; i < 1536; i += kBlockThreads) {
        rays.d[0][i] = kRayDir[i * 3 + 0];
        rays.d[1][i] = kRayDir[i * 3 + 1];
        rays.d[2][i] = kRayDir[i * 3 + 2];
    }
    __syncthreads();
    const size_t waves = (size_t)gridDim.x * kWavesPerBlock;
    size_t env = (size_t)blockIdx.x * kWavesPerBlock + __builtin_amdgcn_readfirstlane(tid >> 6);
    if (env >= rows.batch) return;
    auto obs_of = [&](size_t e) {
        return reinterpret_cast<const float *>(rows.obs + e * rows.obs_stride);
    };
    // Lane j forms the frame of the wave's j-th environment from here (a
    // lane past the batch repeats the current one, whose row exists), and
    // what its mission uses of the scan (all of it when the caller asks for
    // the scan's diagnostics).
    auto frame_obs = [&](size_t first) {
        const size_t e0 = first + (size_t)lane * waves, e = e0 < rows.batch ? e0 : first;
        return load_frame_obs(obs_of(e), reinterpret_cast<const float *>(
                                             rows.mission + e * rows.mission_stride));
    };
    auto frame_need = [&](const FrameObs &v) {
        return rows.diag ? kNeedAll : scan_need(v.m4, v.m5);
    };
    FrameObs first_obs = frame_obs(env);
    float rg[kScanRays];
    load_ranges(obs_rsrc(obs_of(env), true), obs_rsrc(obs_of(env), true), lane, rg);
    ScanFrame mine = scan_frame(first_obs);
    int need_mine = frame_need(first_obs);
    for (int k = 0;;) {
        ScanFrame f;
#pragma unroll
        for (int i = 0; i < 9; ++i)
            f.r[i] = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine.r[i]), k));
        f.py = __builtin_bit_cast(float,
                                  __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine.py), k));
        const size_t next_env = env + waves;
        const bool has_next = next_env < rows.batch;
        // The next environment's ranges are requested only when it uses
        // them (or when the actor's planes need them); the first
        // environment of the next 64 has no need formed yet and is loaded.
        const int need = __builtin_amdgcn_readlane(need_mine, k);
        const int need_next = k + 1 < 64 ? __builtin_amdgcn_readlane(need_mine, (k + 1) & 63)
                                         : kNeedAll;
        const float *next_obs = has_next ? obs_of(next_env) : nullptr;
        const __amdgpu_buffer_rsrc_t next =
            obs_rsrc(next_obs, has_next && (PLANES || need_next != kNeedNone));
        const __amdgpu_buffer_rsrc_t next_upper =
            obs_rsrc(next_obs, has_next && (PLANES || (need_next & kNeedCorridor)));
        if (PLANES)
            write_channel_planes(
                rg, __builtin_amdgcn_make_buffer_rsrc(rows.lidar + env * 12288, (short)0,
                                                      12288 * 4, kBufferWord3),
                lane);
        ScanResult s;
        scan_env(rg, rays, f, next, next_upper, lane, lists[__builtin_amdgcn_readfirstlane(tid >> 6)],
                 s, need);
        if (lane == 0) park_scan(rows.prior + env * 15, s);
        if (!has_next) break;
        env = next_env;
        if (++k == 64) {  // the next 64 environments of this wave
            k = 0;
            FrameObs v = frame_obs(env);
            mine = scan_frame(v);
            need_mine = frame_need(v);
        }
    }
}

// Phase 1 of the H2 entry: the scan of the environments whose mission uses
// it, shared out over a CU.  One workgroup of 16 waves per CU takes
// environments g, g + G, g + 2G, ... (G workgroups in the grid), up to 1,024
// per round.  Each wave forms the frames and needs of 64 of them (lane j the
// j-th); an environment whose mission uses no scan result parks the empty
// result from its lane, and the others are entered (frame, need) in the
// workgroup's pool in LDS.  The waves then take pool entries one at a time
// from a counter in LDS, the next one taken while the current one is
// scanned so that its ranges are requested as far as its need goes.  Which
// wave scans which environment varies from call to call; each result
// depends only on its environment.  A static share of the environments
// would leave the waves that drew several slalom missions working long after
// the others: at 16,384 environments (four per wave) that wave sets the
// kernel's time.  The onboard entry uses this kernel from 2,560
// environments, except for the batches that the one-kernel form takes.
constexpr int kPoolThreads = 1024;
constexpr int kPoolWaves = kPoolThreads / 64;
constexpr int kPoolRound = kPoolThreads;  // environments per round, one per thread
constexpr unsigned kPoolBlocks = 256;     // one workgroup per CU
// The onboard entry's batch from which the pool pays.  Measured on one box
// (static share -> pool, us): 2,048 envs 17.4 -> 17.9, 3,072 18.5 -> 18.1,
// 4,096 19.6 -> 18.2, 16,384 28.4 -> 25.3; below 2,048 the pool is 0.9-1.5
// us slower (the needs are formed before any range is requested, and a
// workgroup holds at most a few environments whose mission uses the scan).
constexpr size_t kPoolMinBatch = 2560;
// The onboard entry's batches that take the one-kernel form (each
// workgroup scans its own 64 environments, then runs their controller):
// those that fill at least 160 of the 256 CUs with one round of 64-
// environment workgroups.  Measured on one box (two kernels -> one, us):
// 8,192 envs 20.6 -> 21.4, 10,240 21.95 -> 21.65, 12,288 23.3 -> 21.8,
// 14,336 24.4 -> 22.1, 16,384 25.4 -> 22.4; with a second round it loses
// (18,432 36.3 -> 38.8, 65,536 79.4 -> 82.2), as it does with fewer
// workgroups than CUs (4,096 18.3 -> 21.1): the two-kernel form spreads the
// scan over every CU.
constexpr size_t kFusedMinBatch = 160 * 64, kFusedMaxBatch = 256 * 64;
struct PoolEntry {
    unsigned env;  // kMaxBatch < 2^31
    int need;
    float r[9], py;
};

__global__ __launch_bounds__(kPoolThreads) void onboard_scan_pool_kernel(OnboardRows rows) {
    __shared__ RayPlanes rays;
    __shared__ u32x2 lists[kPoolWaves][kListCap + 64];  // + a spare entry per lane
    __shared__ PoolEntry pool[kPoolRound];
    __shared__ int pool_count, pool_next;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t groups = gridDim.x;
    // The launch gives every workgroup at least one environment.
    const size_t mine = (rows.batch - blockIdx.x + groups - 1) / groups;
    const size_t rounds = (mine + kPoolRound - 1) / kPoolRound;
    auto obs_of = [&](size_t e) {
        return reinterpret_cast<const float *>(rows.obs + e * rows.obs_stride);
    };
    for (int i = tid; i < 1536; i += kPoolThreads) {
        rays.d[0][i] = kRayDir[i * 3 + 0];
        rays.d[1][i] = kRayDir[i * 3 + 1];
        rays.d[2][i] = kRayDir[i * 3 + 2];
    }
    if (tid == 0) {
        pool_count = 0;
        pool_next = 0;
    }
    __syncthreads();
    // One lane takes the next entry for its wave.
    auto take = [&]() {
        int t = 0;
        if (lane == 0)
            t = __hip_atomic_fetch_add(&pool_next, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
        return __builtin_amdgcn_readfirstlane(t);
    };
    auto entry_env = [&](int t, size_t &env, int &need) {
        env = (unsigned)__builtin_amdgcn_readfirstlane((int)pool[t].env);
        need = __builtin_amdgcn_readfirstlane(pool[t].need);
    };
    auto entry_frame = [&](int t) {
        ScanFrame f;
#pragma unroll
        for (int i = 0; i < 9; ++i)
            f.r[i] = __builtin_bit_cast(
                float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, pool[t].r[i])));
        f.py = __builtin_bit_cast(
            float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, pool[t].py)));
        return f;
    };
    u32x2 *list = lists[wave];
    float rg[kScanRays];
    for (size_t round = 0; round < rounds; ++round) {
        // Thread x forms environment i = x of the round.
        const size_t i = round * kPoolRound + (size_t)tid;
        const size_t e = blockIdx.x + i * groups;
        const bool valid = i < mine;
        if (__builtin_amdgcn_readfirstlane((int)valid)) {  // lane 0 is valid whenever any lane is
            const size_t row = valid ? e : blockIdx.x;
            FrameObs v = load_frame_obs(
                obs_of(row), reinterpret_cast<const float *>(rows.mission + row * rows.mission_stride));
            const ScanFrame f = scan_frame(v);
            const int need = rows.diag ? kNeedAll : scan_need(v.m4, v.m5);
            const bool entered = valid && need != kNeedNone;
            if (valid && !entered)
                park_scan(rows.prior + e * 15, ScanResult{30.0f, 0.0f, 0.0f, 30.0f, 0.0f, -1, 0, 0});
            const uint64_t m = __builtin_amdgcn_ballot_w64(entered);
            int base = 0;
            if (lane == 0 && m)
                base = __hip_atomic_fetch_add(&pool_count, (int)__builtin_popcountll(m),
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            base = __builtin_amdgcn_readfirstlane(base);
            if (entered) {
                PoolEntry &p = pool[base + (int)__builtin_amdgcn_mbcnt_hi(
                                               (unsigned)(m >> 32),
                                               __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u))];
                p.env = (unsigned)e;
                p.need = need;
#pragma unroll
                for (int k = 0; k < 9; ++k) p.r[k] = f.r[k];
                p.py = f.py;
            }
        }
        __syncthreads();
        const int count = __builtin_amdgcn_readfirstlane(pool_count);
        int t = take();
        if (t < count) {
            size_t env;
            int need;
            entry_env(t, env, need);
            load_ranges(obs_rsrc(obs_of(env), true),
                        obs_rsrc(obs_of(env), (need & kNeedCorridor) != 0), lane, rg);
            for (;;) {
                const ScanFrame f = entry_frame(t);
                // The next entry is taken before this one is scanned: the
                // scan requests its ranges once these are consumed.
                const int t_next = take();
                const bool has_next = t_next < count;
                size_t next_env = env;
                int next_need = kNeedNone;
                if (has_next) entry_env(t_next, next_env, next_need);
                const float *next_obs = obs_of(next_env);
                ScanResult s;
                scan_env(rg, rays, f, obs_rsrc(next_obs, has_next),
                         obs_rsrc(next_obs, has_next && (next_need & kNeedCorridor)), lane, list,
                         s, need);
                if (lane == 0) park_scan(rows.prior + env * 15, s);
                if (!has_next) break;
                t = t_next;
                env = next_env;
                need = next_need;
            }
        }
        // Every wave has taken past the end of this round's pool.
        __syncthreads();
        if (tid == 0) {
            pool_count = 0;
            pool_next = 0;
        }
        __syncthreads();
    }
}

// Phase 2's inputs for the 64 environments of a workgroup: obs[0..47],
// mission[0..9] and the parked scan result.  Odd row pitches put the rows a
// wave reads (64 lanes, or 16 quads) on different LDS banks.
constexpr int kStageObs = 48, kStageObsPitch = 49, kStageMissionPitch = 11, kStageScanPitch = 9;
struct ControlStage {
    float obs[64][kStageObsPitch];
    float mission[64][kStageMissionPitch];
    float scan[64][kStageScanPitch];
    float tail[64][5];  // obs[4144..4147], for the actor's scalar wave
};

// Phase 2: the tactical features and the controller, from the parked scan
// result (FUSED: from the workgroup's own scan, phase 1 and 2 in one
// kernel).  A workgroup covers 64 environments: waves 0..3 run the
// controller and waves 4..7 the tactical features, each on one quad of lanes
// per environment (16 per wave), so every SIMD holds one wave of each.
// Both are long scalar chains and few waves exist per launch, so splitting
// the work shortens the chains and spreads them over more SIMDs.  For the
// actor's inputs (SCALARS) each tactical wave then writes the symlog
// scalars and mission values of its 16 environments, one row per store (on
// the scan waves they cost the scan kernel 6 µs and the plane kernel of the
// next call 6 µs more).
//   * The workgroup first stages every input its chains read (all loads
//     issued at once, coalesced over the rows' first 192 bytes), so the
//     chains read LDS: read from global memory at their points of use, the
//     values came in a dozen dependent round trips.
//   * Values are formed in registers and then stored to each destination
//     (the tactical / prior rows and, for the actor, their copies in
//     proprio and mission_vec).
// Whether an environment's staged mission selects the BWB law
// (onboard_features.cuh:433-437, on the values the controller forms).
__device__ __forceinline__ bool bwb_mission(const float *raw) {
    const float m2 = ob_mission(raw[2]), m4 = ob_mission(raw[4]), m5 = ob_mission(raw[5]),
                m6 = ob_mission(raw[6]);
    return (m6 > 0.75f && m4 < -0.25f) || (m4 > 0.75f && m2 > 0.25f) ||
           (m6 > 0.75f && m5 > 0.60f);
}

// FUSED: the workgroup also scans its own environments (the onboard
// entry's one-kernel form), from a pool in LDS over its eight waves, and the
// results go straight into the stage.
struct FusedScanLds {
    RayPlanes rays;
    u32x2 lists[2 * kControlWaves][kListCap + 64];  // + a spare entry per lane
    PoolEntry pool[64];
    int count, next;
};

// The scan of the workgroup's 64 staged environments (base + e), called by
// every wave after the stage is written: wave 0 forms each environment's
// frame and need from the stage (lane e), writes the empty result of those
// whose mission uses no scan result and enters the others in the pool; then
// every wave takes entries one at a time, the next one taken before the
// current one is scanned so that its ranges are requested as far as its
// need goes, and lane 0 writes each result into the stage.  Ends with the
// workgroup's barrier, so the results are visible to the control phase.
__device__ __forceinline__ void fused_scan(const OnboardRows &rows, size_t base,
                                           ControlStage &stage, FusedScanLds &fused, int w,
                                           int lane) {
    auto obs_of = [&](size_t e) {
        return reinterpret_cast<const float *>(rows.obs + e * rows.obs_stride);
    };
    auto stage_result = [&](int e, const ScanResult &r) {
        float *sc = stage.scan[e];
        sc[0] = r.min_r;
        sc[1] = r.min_r_dx;
        sc[2] = r.min_r_dy;
        sc[3] = r.min_dx_c;
        sc[4] = r.cluster_y_sum;
        sc[5] = __int_as_float(r.min_ray);
        sc[6] = __int_as_float(r.cluster_count);
    };
    if (w == 0) {
        const int e = lane;
        const bool valid = base + (size_t)e < rows.batch;
        FrameObs v{stage.obs[e][1], stage.obs[e][6], stage.obs[e][7], stage.obs[e][8],
                   stage.obs[e][9], stage.mission[e][4], stage.mission[e][5]};
        const ScanFrame f = scan_frame(v);
        const int need = rows.diag ? kNeedAll : scan_need(v.m4, v.m5);
        const bool entered = valid && need != kNeedNone;
        if (valid && !entered) stage_result(e, ScanResult{30.0f, 0.0f, 0.0f, 30.0f, 0.0f, -1, 0, 0});
        // Corridor scans (the longest) first.
        const bool front = (need & kNeedCorridor) != 0;
        const uint64_t mf = __builtin_amdgcn_ballot_w64(entered && front);
        const uint64_t mb = __builtin_amdgcn_ballot_w64(entered && !front);
        const uint64_t m = mf | mb;
        if (entered) {
            const uint64_t mine = front ? mf : mb;
            const unsigned rank = __builtin_amdgcn_mbcnt_hi(
                (unsigned)(mine >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)mine, 0u));
            PoolEntry &p = fused.pool[(front ? 0u : (unsigned)__builtin_popcountll(mf)) + rank];
            p.env = (unsigned)e;
            p.need = need;
#pragma unroll
            for (int k = 0; k < 9; ++k) p.r[k] = f.r[k];
            p.py = f.py;
        }
        if (lane == 0) {
            fused.count = (int)__builtin_popcountll(m);
            fused.next = 0;
        }
    }
    __syncthreads();
    const int count = __builtin_amdgcn_readfirstlane(fused.count);
    auto take = [&]() {
        int t = 0;
        if (lane == 0)
            t = __hip_atomic_fetch_add(&fused.next, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
        return __builtin_amdgcn_readfirstlane(t);
    };
    auto entry = [&](int t, int &slot, int &need) {
        slot = __builtin_amdgcn_readfirstlane((int)fused.pool[t].env);
        need = __builtin_amdgcn_readfirstlane(fused.pool[t].need);
    };
    int t = take();
    if (t < count) {
        int slot, need;
        entry(t, slot, need);
        float rg[kScanRays];
        const float *o = obs_of(base + (size_t)slot);
        load_ranges(obs_rsrc(o, true), obs_rsrc(o, (need & kNeedCorridor) != 0), lane, rg);
        for (;;) {
            ScanFrame f;
#pragma unroll
            for (int i = 0; i < 9; ++i)
                f.r[i] = __builtin_bit_cast(
                    float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fused.pool[t].r[i])));
            f.py = __builtin_bit_cast(
                float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fused.pool[t].py)));
            const int t_next = take();
            const bool has_next = t_next < count;
            int next_slot = slot, next_need = kNeedNone;
            if (has_next) entry(t_next, next_slot, next_need);
            const float *next_obs = obs_of(base + (size_t)next_slot);
            ScanResult r;
            scan_env(rg, fused.rays, f, obs_rsrc(next_obs, has_next),
                     obs_rsrc(next_obs, has_next && (next_need & kNeedCorridor)), lane,
                     fused.lists[w], r, need);
            if (lane == 0) stage_result(slot, r);
            if (!has_next) break;
            t = t_next;
            slot = next_slot;
            need = next_need;
        }
    }
    __syncthreads();
}

template <bool SCALARS, bool FUSED>
__global__ __launch_bounds__(kControlThreads) void onboard_control_kernel(OnboardRows rows) {
    constexpr int CW = kControlWaves, N = 64, kThreads = kControlThreads;
    __shared__ ControlStage stage;
    // Per controller wave: the workgroup's environments, BWB missions first.
    __shared__ unsigned char order[CW][N];
    __shared__ std::conditional_t<FUSED, FusedScanLds, char> fused;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int a = lane & 3;
    if constexpr (FUSED) {
        for (int i = tid; i < 1536; i += kThreads) {
            fused.rays.d[0][i] = kRayDir[i * 3 + 0];
            fused.rays.d[1][i] = kRayDir[i * 3 + 1];
            fused.rays.d[2][i] = kRayDir[i * 3 + 2];
        }
    }
    for (size_t base = (size_t)blockIdx.x * N; base < rows.batch;
         base += (size_t)gridDim.x * N) {
        // Rows past the batch end re-read the last row; nothing uses them.
        auto row_of = [&](int e) {
            const size_t env = base + (size_t)e;
            return env < rows.batch ? env : rows.batch - 1;
        };
        constexpr int kObsLoads = (N * kStageObs + kThreads - 1) / kThreads;
        constexpr int kMissionLoads = (N * 10 + kThreads - 1) / kThreads;
        constexpr int kScanLoads = (N * 7 + kThreads - 1) / kThreads;
        // Every thread issues all its loads unconditionally (an index past
        // the stage re-reads the stage's last value), so they leave at once.
        float vo[kObsLoads], vm[kMissionLoads], vs[kScanLoads], vt = 0.0f;
#pragma unroll
        for (int k = 0; k < kObsLoads; ++k) {
            const int idx = min(tid + kThreads * k, N * kStageObs - 1);
            const int e = idx / kStageObs, i = idx - kStageObs * e;
            vo[k] = reinterpret_cast<const float *>(rows.obs + row_of(e) * rows.obs_stride)[i];
        }
#pragma unroll
        for (int k = 0; k < kMissionLoads; ++k) {
            const int idx = min(tid + kThreads * k, N * 10 - 1);
            const int e = idx / 10, i = idx - 10 * e;
            vm[k] = reinterpret_cast<const float *>(rows.mission + row_of(e) * rows.mission_stride)[i];
        }
#pragma unroll
        for (int k = 0; k < kScanLoads; ++k) {
            const int idx = min(tid + kThreads * k, N * 7 - 1);
            const int e = idx / 7, i = idx - 7 * e;
            vs[k] = FUSED ? 0.0f : rows.prior[row_of(e) * 15 + i];
        }
        if (SCALARS) {
            const int idx = min(tid, N * 4 - 1);
            const int e = idx / 4;
            vt = reinterpret_cast<const float *>(
                rows.obs + row_of(e) * rows.obs_stride)[4144 + idx - 4 * e];
        }
#pragma unroll
        for (int k = 0; k < kObsLoads; ++k) {
            const int idx = tid + kThreads * k;
            const int e = idx / kStageObs;
            if (idx < N * kStageObs) stage.obs[e][idx - kStageObs * e] = vo[k];
        }
#pragma unroll
        for (int k = 0; k < kMissionLoads; ++k) {
            const int idx = tid + kThreads * k;
            const int e = idx / 10;
            if (idx < N * 10) stage.mission[e][idx - 10 * e] = vm[k];
        }
#pragma unroll
        for (int k = 0; k < kScanLoads; ++k) {
            const int idx = tid + kThreads * k;
            const int e = idx / 7;
            if (!FUSED && idx < N * 7) stage.scan[e][idx - 7 * e] = vs[k];
        }
        if (SCALARS && tid < N * 4) stage.tail[tid / 4][tid % 4] = vt;
        __syncthreads();
        if constexpr (FUSED) fused_scan(rows, base, stage, fused, w, lane);

        // The controller waves take the workgroup's environments BWB
        // missions first, so that all but about one wave of them have no
        // BWB environment and skip the BWB blocks, which a wave runs when
        // any of its quads needs them.  (18% of the benchmark's missions are
        // BWB, and 96% of 16-environment waves held one: 34.47 -> 34.06 us
        // for the entry.  The wave that keeps BWB environments still runs
        // the whole chain, and its SIMD sets the time; with the BWB blocks
        // removed from every wave the entry would take 1.4 us less.)  Each
        // controller wave ranks the 64 environments itself (lane e ranks
        // environment e) into its own table and reads back its quads'
        // environments.  Every environment's values are the same in any
        // order.
        // Tactical waves: environment 16 (w - 4) + lane / 4.
        int slot = 16 * (w - CW) + (lane >> 2);
        if (w < CW) {
            const bool b = bwb_mission(stage.mission[lane]);
            const uint64_t bm = __builtin_amdgcn_ballot_w64(b);
            const unsigned nb = (unsigned)__builtin_popcountll(bm);
            const uint64_t mine = b ? bm : ~bm;
            const unsigned below = __builtin_amdgcn_mbcnt_hi(
                (unsigned)(mine >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)mine, 0u));
            order[w][b ? below : nb + below] = (unsigned char)lane;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            slot = order[w][16 * w + (lane >> 2)];
        }

        const size_t env = base + (size_t)slot;
        if (env < rows.batch) {
            const float *obs = stage.obs[slot];
            const float *mission = stage.mission[slot];
            if (w >= CW) {
                // Lane a of the quad writes features 6a .. 6a + 5.
                float t[6];
                tactical_quad(obs, mission, a, t);
                float *tac = rows.tactical + env * 24 + 6 * a;
#pragma unroll
                for (int i = 0; i < 6; ++i) tac[i] = t[i];
                if (rows.proprio) {
                    float *p = rows.proprio + env * 91 + 52 + 6 * a,
                          *mv = rows.mission_vec + env * 49 + 10 + 6 * a;
#pragma unroll
                    for (int i = 0; i < 6; ++i) {
                        p[i] = t[i];
                        mv[i] = t[i];
                    }
                }
            } else {
                const float *sc = stage.scan[slot];
                ScanResult s;
                s.min_r = sc[0];
                s.min_r_dx = sc[1];
                s.min_r_dy = sc[2];
                s.min_dx_c = sc[3];
                s.cluster_y_sum = sc[4];
                s.min_ray = __float_as_int(sc[5]);
                s.cluster_count = __float_as_int(sc[6]);
                // Read from LDS before the chain, like the other inputs.
                asm volatile("" : "+v"(s.min_r), "+v"(s.min_r_dx), "+v"(s.min_r_dy), "+v"(s.min_dx_c),
                             "+v"(s.cluster_y_sum), "+v"(s.min_ray), "+v"(s.cluster_count));
                const ArmOutputs n = prior_features(obs, mission, s, a);
                // The parked result was staged before the chain; each lane
                // now writes its arm's three values, lane 0 the cannon's.
                float *prior = rows.prior + env * 15;
                prior[a] = n.throttle;
                prior[4 + a] = n.outer;
                prior[8 + a] = n.inner;
                if (a == 0) {
                    prior[12] = n.az;
                    prior[13] = n.el;
                    prior[14] = n.fire;
                }
                if (rows.proprio) {
                    float *p = rows.proprio + env * 91 + 76, *mv = rows.mission_vec + env * 49 + 34;
                    p[a] = n.throttle;
                    p[4 + a] = n.outer;
                    p[8 + a] = n.inner;
                    mv[a] = n.throttle;
                    mv[4 + a] = n.outer;
                    mv[8 + a] = n.inner;
                    if (a == 0) {
                        p[12] = n.az;
                        p[13] = n.el;
                        p[14] = n.fire;
                        mv[12] = n.az;
                        mv[13] = n.el;
                        mv[14] = n.fire;
                    }
                }
                if (rows.diag && a == 0) {
                    float *d = rows.diag + env * 5;
                    d[0] = s.min_r;
                    d[1] = (float)s.min_ray;
                    d[2] = s.min_dx_c;
                    d[3] = (float)s.cluster_count;
                    d[4] = s.cluster_y_sum;
                }
            }
        }
        if (SCALARS && w >= CW) {
            // Lane l's input: obs[l] (l < 48), obs[4144 + l - 48] (l < 52),
            // mission[l - 52] (l < 62).
            const int lo = min(lane, kStageObs - 1), lt = min(max(lane - 48, 0), 3),
                      lm = min(max(lane - 52, 0), 9);
            // All 16 inputs are read first, so the 16 chains are
            // independent; rows past the batch end (staged as copies of the
            // last row) store nothing.
            float raw[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int e = 16 * (w - CW) + j;
                raw[j] = lane < 48 ? stage.obs[e][lo]
                                   : (lane < 52 ? stage.tail[e][lt] : stage.mission[e][lm]);
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const size_t env = base + (size_t)(16 * (w - CW) + j);
                const bool valid = env < rows.batch;
                const size_t row = valid ? env : base;
                actor_scalars(raw[j], lane, rows.proprio + row * 91, rows.mission_vec + row * 49,
                              valid);
            }
        }

        // The stage is reused by this workgroup's next 64 environments.
        if (base + (size_t)gridDim.x * N < rows.batch) __syncthreads();
    }
}

// `pooled` selects the pooled scan, which holds a whole CU per workgroup:
// for calls whose scan runs alone, not beside the actor's plane kernel.
int launch_onboard(const OnboardRows &rows, hipStream_t s, bool pooled) {
    const size_t scan_want = (rows.batch + kWavesPerBlock - 1) / kWavesPerBlock;
    const unsigned scan_blocks = scan_want > kScanBlocks ? kScanBlocks : (unsigned)scan_want;
    const size_t ctrl_want = (rows.batch + 63) / 64;
    if (rows.lidar) {
        onboard_scan_kernel<true><<<scan_blocks, kBlockThreads, 0, s>>>(rows);
    } else if (pooled) {
        // At least 16 environments per workgroup (one per wave) while that
        // fills the chip.
        const size_t want = (rows.batch + kPoolWaves - 1) / kPoolWaves;
        onboard_scan_pool_kernel<<<want > kPoolBlocks ? kPoolBlocks : (unsigned)want,
                                   kPoolThreads, 0, s>>>(rows);
    } else {
        onboard_scan_kernel<false><<<scan_blocks, kBlockThreads, 0, s>>>(rows);
    }
    const unsigned ctrl_blocks = ctrl_want > kControlBlocks ? kControlBlocks : (unsigned)ctrl_want;
    if (rows.proprio)
        onboard_control_kernel<true, false><<<ctrl_blocks, kControlThreads, 0, s>>>(rows);
    else
        onboard_control_kernel<false, false><<<ctrl_blocks, kControlThreads, 0, s>>>(rows);
    return hipGetLastError() == hipSuccess;
}

}  // namespace

extern "C" int tb_hip_onboard_tactical_prior_device(const float *obs, const float *mission,
                                                    float *tactical, float *prior, float *diag,
                                                    size_t batch_size, void *stream) {
    if (!obs || !mission || !tactical || !prior || batch_size == 0 || batch_size > kMaxBatch)
        return 0;
    OnboardRows rows;
    rows.obs = reinterpret_cast<const unsigned char *>(obs);
    rows.obs_stride = 4148 * sizeof(float);
    rows.mission = reinterpret_cast<const unsigned char *>(mission);
    rows.mission_stride = 10 * sizeof(float);
    rows.tactical = tactical;
    rows.prior = prior;
    rows.diag = diag;
    rows.proprio = nullptr;
    rows.mission_vec = nullptr;
    rows.lidar = nullptr;
    rows.batch = batch_size;
    (void)hipGetLastError();
    if (batch_size >= kFusedMinBatch && batch_size <= kFusedMaxBatch) {
        // One round of 64-environment workgroups, one per CU.
        onboard_control_kernel<false, true>
            <<<(unsigned)((batch_size + 63) / 64), kControlThreads, 0,
               reinterpret_cast<hipStream_t>(stream)>>>(rows);
        return hipGetLastError() == hipSuccess;
    }
    return launch_onboard(rows, reinterpret_cast<hipStream_t>(stream),
                          batch_size >= kPoolMinBatch);
}

// ---------------------------------------------------------------------------
// The 618M actor's sensor preparation, fused (reference
// src/network/network_gpu.cu:274-304 scalar_inputs, :467-479 lidar_channels,
// :480-483 camera_luma, launched back to back at :1446-1451).  One workgroup
// per environment streams the LiDAR block once into the six channel planes
// and the cameras once into luma: LiDAR in 16-byte loads, camera bytes in
// 4-byte loads so that each lane's 4 luma values are one float4 and every
// store instruction writes 1 KiB of consecutive output.  From the split
// threshold on, the scan kernel writes the channels of the rays it reads
// (elevation rows 0..5) and this kernel only those of rows 6..15, so each
// LiDAR range is read from HBM once.
// The control kernel's controller waves add each environment's 52 symlog
// scalars and mission values after their chains, and store tactical / prior
// and their copies.  Fusing the scan into the streaming launch was measured
// slower: next to saturated HBM traffic the scan's dependent loads stall.  Luma is
// the reference's `(float)b * (1.0f / 255.0f) - 0.5f` as its CUDA build
// evaluates it: nvcc contracts the product and difference into one fused
// multiply-add by default, so it is one explicit fma here (this file is built
// without automatic contraction, like every restatement of the reference's
// arithmetic here).

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Threads of a head whose LiDAR float4 lies in the scan's elevation rows
// 0..5 (6 rows of 32 float4).
constexpr int kScanRowThreads = 6 * 128 / 4;

struct ActorRows {
    const float *obs;
    const unsigned char *cameras;
    float *lidar, *luma;
    size_t batch;
    bool scan_rows;  // also the channels of the scan rows (else the scan kernel writes them)
};

__device__ __forceinline__ f32x4 lidar_channel4(f32x4 r, int kind) {
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = lidar_channel(r[e], kind);
    return o;
}

// One 1,024-thread workgroup per environment: thread t loads LiDAR float4 t
// and camera words t + 1024 k, and every store instruction of the
// workgroup writes 16 KB of consecutive output (the two heads' planes of a
// channel kind are adjacent, as are consecutive luma float4).  With the
// XCD-contiguous environment order a pure fill of this pattern reaches
// 6.3 TB/s on MI355X, against 5.5 TB/s for 256-thread workgroups in
// dispatch order.
// One 16-byte store into an environment's output block (`bytes` long) with
// cache policy nt + sc1.  Entry at 16,384 environments on MI355X, one
// workgroup per CU, identical outputs: default policy 461.5 us, nt 450.7,
// sc0 + nt 449.9, sc1 442.4, sc0 + sc1 442.4, nt + sc1 434.1, sc0 + nt +
// sc1 434.3 (with two workgroups per CU: default 440.3 us for the plane
// kernel, sc1 416.7).
__device__ __forceinline__ void store_plane(float *block, unsigned bytes, unsigned index, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(u32x4, v),
        __builtin_amdgcn_make_buffer_rsrc(block, (short)0, (int)bytes, 0x00020000), index * 16u,
        0, kStorePolicy);
}

__global__ __launch_bounds__(kStreamThreads) void actor_stream_kernel(ActorRows rows) {
    const int t = threadIdx.x;
    for (size_t env = xcd_contiguous(blockIdx.x, gridDim.x); env < rows.batch;
         env += gridDim.x) {
        // float4 t is bins 4(t%512).. of head t/512, elevation row
        // (t%512)/32.  Unless `scan_rows`, the scan kernel writes rows 0..5
        // (threads with t%512 < 192, whole waves) and this kernel the other
        // ten.
        const bool lidar = rows.lidar && (rows.scan_rows || (t & 511) >= kScanRowThreads);
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (lidar)
            v = __builtin_nontemporal_load(
                reinterpret_cast<const f32x4 *>(rows.obs + env * 4148 + 48) + t);
        unsigned px[4];
        if (rows.luma) {
            const unsigned *cam = reinterpret_cast<const unsigned *>(rows.cameras + env * 16384);
#pragma unroll
            for (int k = 0; k < 4; ++k) px[k] = __builtin_nontemporal_load(cam + t + 1024 * k);
        }
        if (lidar) {
            // Head h feeds channels h, h+2, h+4.
            float *dst = rows.lidar + env * 12288;
            const int head = t >> 9, q = t & 511;
#pragma unroll
            for (int kind = 0; kind < 3; ++kind)
                store_plane(dst, 12288 * 4, (head + 2 * kind) * 512 + q, lidar_channel4(v, kind));
        }
        if (rows.luma) {
            float *dst = rows.luma + env * 16384;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const unsigned w = px[k];
                f32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = __builtin_fmaf((float)((w >> (8 * e)) & 0xffu), 1.0f / 255.0f,
                                          -0.5f);
                store_plane(dst, 16384 * 4, t + 1024 * k, o);
            }
        }
    }
}

// The scan and control kernels run beside the plane kernel on a second
// stream of the device, forked from and joined back to the caller's stream.
// The plane kernel is write-bound and keeps one workgroup per CU; the scan
// and control workgroups fit beside it, and their latency-bound chains
// overlap its streams.  It is the controller that gains most: the scan alone
// on the second stream, with the controller after the join, measured 437.9
// against 433.0 us at 16,384 environments (before the split below).
//
// Split of the LiDAR channel planes: from kSplitMinBatch environments the
// scan kernel writes the channels of the 1,536 rays it reads (elevation rows
// 0..5 of each head) and the plane kernel only the other rows, so the entry
// reads every LiDAR range from HBM once instead of reading the scan rows
// twice.  Measured on the entry (one box, outputs bit-equal in every mode;
// one stream without / with the split, two streams without / with it):
//    batch    one stream     two streams
//      256    25.1 / 26.3    41.7 / 44.1
//      512    32.0 / 31.0    45.6 / 45.7
//    1,536    59.7 / 55.8    58.5 / 63.0
//    1,792    65.4 / 62.9    62.7 / 66.5
//    2,048    76.3 / 70.8    67.8 / 70.4
//    2,432    88.8 / 86.8    73.7 / 75.4
//    2,560    88.8 / 86.6    81.2 / 80.2
//    4,096   128.9 / 123.6  124.1 / 111.7
//    8,192   230.4 / 222.9  225.3 / 214.5
//   16,384       --          428.5 / 412.5
// So batches below kOverlapMinBatch keep one stream (the fork and join cost
// several microseconds), with the split from kSplitMinBatch; from
// kOverlapMinBatch two streams, with the split from kSplitOverlapMinBatch
// (below it the longer scan holds up the second stream).
constexpr size_t kSplitMinBatch = 512;
constexpr size_t kSplitOverlapMinBatch = 2560;
constexpr size_t kOverlapMinBatch = 1792;
constexpr int kMaxDevices = 64;

struct SideStream {
    std::mutex order;           // one fork ... join sequence at a time
    std::atomic<int> state{0};  // 0 not made, 1 ready, -1 creation failed
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
SideStream side_streams[kMaxDevices];

// The current device's side stream (default priority, non-blocking), made
// on first use.  nullptr when it cannot be made, and while `s` is being
// captured into a graph before it exists (a capture may use one made
// earlier: the fork and join events bring it into the capture).  A failed
// query or creation is cleared from the runtime's last error, so the call
// goes on with one stream and its own launch check stays meaningful.
SideStream *side_stream(hipStream_t s) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return nullptr;
    }
    SideStream &ss = side_streams[dev];
    int state = ss.state.load(std::memory_order_acquire);
    if (state == 0) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(s, &capture) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        if (capture != hipStreamCaptureStatusNone) return nullptr;
        std::lock_guard<std::mutex> made(ss.order);
        state = ss.state.load(std::memory_order_acquire);
        if (state == 0) {
            const bool ok =
                hipStreamCreateWithFlags(&ss.stream, hipStreamNonBlocking) == hipSuccess &&
                hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) == hipSuccess &&
                hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) == hipSuccess;
            state = ok ? 1 : -1;
            if (!ok) (void)hipGetLastError();
            ss.state.store(state, std::memory_order_release);
        }
    }
    return state == 1 ? &ss : nullptr;
}

}  // namespace

extern "C" int tb_hip_actor_inputs_device(const float *obs, const float *mission,
                                          const unsigned char *cameras, float *proprio,
                                          float *mission_vec, float *tactical, float *prior,
                                          float *lidar_channels, float *camera_luma,
                                          size_t batch_size, void *stream) {
    if (!obs || !mission || !proprio || !mission_vec || !tactical || !prior || batch_size == 0 ||
        batch_size > kMaxBatch || (camera_luma && !cameras))
        return 0;
    const uintptr_t align = reinterpret_cast<uintptr_t>(obs) |
                            reinterpret_cast<uintptr_t>(lidar_channels) |
                            reinterpret_cast<uintptr_t>(camera_luma) |
                            reinterpret_cast<uintptr_t>(cameras);
    if ((align & 15u) != 0) return 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    (void)hipGetLastError();
    const bool planes = lidar_channels || camera_luma;
    SideStream *side = planes && batch_size >= kOverlapMinBatch ? side_stream(s) : nullptr;
    const bool split = lidar_channels && batch_size >= kSplitMinBatch &&
                       (!side || batch_size >= kSplitOverlapMinBatch);
    std::unique_lock<std::mutex> order;
    if (side) {
        order = std::unique_lock<std::mutex>(side->order);
        if (hipEventRecord(side->fork, s) != hipSuccess ||
            hipStreamWaitEvent(side->stream, side->fork, 0) != hipSuccess)
            return 0;
    }
    if (planes) {
        ActorRows ar;
        ar.obs = obs;
        ar.cameras = cameras;
        ar.lidar = lidar_channels;
        ar.luma = camera_luma;
        ar.batch = batch_size;
        ar.scan_rows = !split;
        // One workgroup per CU: the launch asks for more than half of the
        // CU's 160 KB of LDS, which the kernel does not use (by registers a
        // CU holds two; one measured 462.7 -> 445.0 us for the entry,
        // identical outputs: fewer requests in flight keep the write-bound
        // streams more efficient).
        constexpr unsigned kOneWorkgroupLds = (160 * 1024 / 2 + 1 + 1023) / 1024 * 1024;
        actor_stream_kernel<<<batch_size > kMaxBlocks ? kMaxBlocks : (unsigned)batch_size,
                              kStreamThreads, kOneWorkgroupLds, s>>>(ar);
    }
    OnboardRows rows;
    rows.obs = reinterpret_cast<const unsigned char *>(obs);
    rows.obs_stride = 4148 * sizeof(float);
    rows.mission = reinterpret_cast<const unsigned char *>(mission);
    rows.mission_stride = 10 * sizeof(float);
    rows.tactical = tactical;
    rows.prior = prior;
    rows.diag = nullptr;
    rows.proprio = proprio;
    rows.mission_vec = mission_vec;
    rows.lidar = split ? lidar_channels : nullptr;
    rows.batch = batch_size;
    if (!side) return launch_onboard(rows, s, false);
    const int ok = launch_onboard(rows, side->stream, false);
    if (hipEventRecord(side->join, side->stream) != hipSuccess ||
        hipStreamWaitEvent(s, side->join, 0) != hipSuccess)
        return 0;
    return ok;
}
