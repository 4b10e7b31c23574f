/*
 * TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference's sensor-feature
 * algorithms, used by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker.  Nothing in turbinator_c_amd/ may link,
 * load or call it.
 */
#ifndef TB_ORACLE_H
#define TB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OBS = 4148,
    ORC_MISSION = 10,
    ORC_CAMERA = 16384,
    ORC_FEATURES = 142,
    ORC_DIAG_BYTES = 432
};

/* One environment, reference src/training/training.c:102-142. */
void orc_features_env(const float *obs, const float *mission,
                      const uint8_t *cameras, float *out);

/* Strided batch over `threads` POSIX threads (static env partition).
 * Strides are in bytes between consecutive environments.  cameras may be
 * NULL.  out rows are dense [batch,142]. */
void orc_features_batch(const unsigned char *obs, size_t obs_stride,
                        const unsigned char *mission, size_t mission_stride,
                        const unsigned char *cameras, size_t camera_stride,
                        float *out, size_t batch, int threads);

/* The reference's LiDAR bin transform f(r) (training.c:65-68). */
float orc_lidar_feature(float range_m);

/* orc_lidar_feature over an array, on `threads` POSIX threads. */
void orc_lidar_feature_array(const float *in, float *out, size_t n, int threads);

/* Depth (metres) -> luma byte map used for fp32-depth camera inputs. */
uint8_t orc_depth_to_luma(float depth_m);
void orc_depth_to_luma_array(const float *depth, uint8_t *luma, size_t n);

/* Per-environment diagnostics with no counterpart in the 142-vector, one
 * 432-byte row (little-endian):
 * bytes 0..255    float[64] LiDAR sector minimum over valid bins (-1 if none)
 * bytes 256..383  uint16[64] first-minimum position p = 16*row + bin inside
 *                 the sector (scan order; 0xff if none) | valid count << 8
 * bytes 384..399  uint8[16] camera quadrant minimum byte (0 when cameras NULL)
 * bytes 400..431  uint16[16] camera quadrant occupancy: bytes != 0          */
void orc_diagnostics_env(const float *obs, const uint8_t *cameras, uint8_t *diag);

/* Onboard tactical (24) and prior (15) features, reference
 * src/network/onboard_features.cuh:25-519.  `diag` (nullable) receives
 * {min_r, argmin ray (as float), min_dx_c, cluster_count (as float),
 * cluster_y_sum}. */
void orc_onboard_env(const float *obs, const float *mission,
                     float *tactical24, float *prior15, float *diag5);

/* The 618M actor's sensor preparation (network_gpu.cu:274-304,467-483):
 * proprio[91], mission_vec[49], tactical[24], prior[15], lidar[6*2048]
 * (nullable), luma[16384] (nullable; needs cameras). */
void orc_actor_inputs_env(const float *obs, const float *mission, const uint8_t *cameras,
                          float *proprio, float *mission_vec, float *tactical, float *prior,
                          float *lidar, float *luma);

/* Compact SAC actor (training.c:82-100, 219-233, 306-329): the agent's
 * normal draws, and one environment's action / log-probability / raw
 * network outputs (raw_out may be NULL; normals NULL = deterministic). */
void orc_sac_normals(uint64_t *state, float *out, size_t count);
void orc_sac_actor_env(const float *w0, const float *b0, const float *w1, const float *b1,
                       const float *w2, const float *b2, int hidden, const float *feature,
                       const float *normals, float *action, float *log_prob, float *raw_out);

/* Body-frame direction of onboard ray head*768 + el*128 + azi. */
void orc_onboard_ray_dir(int ray, float *xyz);

#ifdef __cplusplus
}
#endif

#endif
