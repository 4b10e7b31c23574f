/*
 * TEST INFRASTRUCTURE ONLY: the CPU checker for the 618M actor's sensor
 * preparation, restating the reference kernels
 *   scalar_inputs   src/network/network_gpu.cu:274-304
 *   lidar_channels  src/network/network_gpu.cu:467-479
 *   camera_luma     src/network/network_gpu.cu:480-483
 * for one environment, in C11 single precision with libm (log1pf), no FMA
 * contraction.  Tactical / prior come from orc_onboard_env
 * (onboard_features.cuh, restated in onboard_oracle.c).
 *
 * Outputs per environment:
 *   proprio[91]   52 symlog scalars, tactical[24], prior[15]
 *   mission[49]   10 finite mission values, tactical[24], prior[15]
 *   tactical[24], prior[15]
 *   lidar[6*2048] channel c of bin (row, az): c = 0,1 inverse range of head
 *                 c%2, c = 2,3 range/30, c = 4,5 validity
 *   luma[16384]   byte * fl(1/255) - 0.5, two roundings (no contraction)
 */
#include "oracle.h"

#include <math.h>

/* network_gpu.cu:285-297: per-scalar scale of the symlog inputs. */
static float ai_scale(int i) {
    if (i < 3) return 0.05f;
    if (i < 6) return 0.10f;
    if (i >= 10 && i < 13) return 0.20f;
    if (i >= 13 && i < 16) return 0.10f;
    if (i >= 28 && i < 32) return 0.50f;
    if (i >= 32 && i < 36) return 0.20f;
    return 1.0f;
}

void orc_actor_inputs_env(const float *obs, const float *mission, const uint8_t *cameras,
                          float *proprio, float *mission_vec, float *tactical, float *prior,
                          float *lidar, float *luma) {
    for (int i = 0; i < 52; ++i) {
        float raw = i < 48 ? obs[i] : obs[4144 + i - 48];
        raw = isfinite(raw) ? fmaxf(-1000.0f, fminf(1000.0f, raw)) : 0.0f;
        const float symlog = copysignf(log1pf(fabsf(raw * ai_scale(i))), raw);
        proprio[i] = fmaxf(-8.0f, fminf(8.0f, symlog / sqrtf(1.0001f)));
    }
    orc_onboard_env(obs, mission, tactical, prior, NULL);
    for (int i = 0; i < 24; ++i) proprio[52 + i] = tactical[i];
    for (int i = 0; i < 15; ++i) proprio[76 + i] = prior[i];
    for (int i = 0; i < 10; ++i) mission_vec[i] = isfinite(mission[i]) ? mission[i] : 0.0f;
    for (int i = 0; i < 24; ++i) mission_vec[10 + i] = tactical[i];
    for (int i = 0; i < 15; ++i) mission_vec[34 + i] = prior[i];
    if (lidar) {
        for (int c = 0; c < 6; ++c)
            for (int bin = 0; bin < 2048; ++bin) {
                const float range = obs[48 + (c % 2) * 2048 + bin];
                const int valid = range > 0.0f && isfinite(range);
                const float clamped = fmaxf(0.05f, fminf(30.0f, range));
                lidar[c * 2048 + bin] =
                    c < 2 ? (valid ? 1.0f / fmaxf(0.2f, clamped) : 0.0f)
                          : (c < 4 ? (valid ? clamped / 30.0f : 1.0f) : (float)valid);
            }
    }
    /* network_gpu.cu:482, `(float)b * (1.0f / 255.0f) - 0.5f`, exists only
     * as CUDA device code, and nvcc's default --fmad=true (the reference's
     * CMakeLists.txt:32-36 sets no CUDA flags) contracts a product followed
     * by a difference into one fused multiply-add: one rounding.  Two
     * roundings, as ISO C evaluates the line, differ for 158 of the 256
     * byte values. */
    if (luma && cameras)
        for (int p = 0; p < 16384; ++p)
            luma[p] = fmaf((float)cameras[p], 1.0f / 255.0f, -0.5f);
}
