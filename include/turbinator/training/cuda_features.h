/*
 * Drop-in boundary of the batched sensor-feature path, served by the gfx950
 * HIP backend (libturbinator_hip).  The six entry points keep the names,
 * argument order, argument meaning and return conventions of the reference
 * header include/turbinator/training/cuda_features.h:14-34, so the trainer
 * (src/trainer/main.c:513-712) and tests/test_cuda_features.c link against
 * this library without source changes.  `stream` is a hipStream_t carried as
 * void*; NULL selects the null stream.
 *
 * Tensor layouts (row-major, one row per environment):
 *   obs       [batch, 4148] float   (48 proprio, 2x2048 LiDAR, 4 scan stats)
 *   mission   [batch,   10] float
 *   cameras   [batch,16384] uint8   (4 cameras x 64 rows x 64 columns)
 *   features  [batch,  142] float
 */
#ifndef TURBINATOR_CUDA_FEATURES_H
#define TURBINATOR_CUDA_FEATURES_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces cuda_features.h:14-19 (src/cuda/features.cu:158-169).
 * Device pointers.  `device_cameras` may be NULL, which zeroes features
 * 126..141.  Returns 0 without launching when obs, mission or features is
 * NULL, batch_size is 0 or batch_size > 0x7fffffff; otherwise enqueues the
 * extraction on `stream` and returns 1 iff the launch was accepted.  The call
 * is asynchronous: synchronise before reading `device_features`. */
int tb_cuda_extract_features_device(const float *device_obs,
                                    const float *device_mission,
                                    const unsigned char *device_cameras,
                                    float *device_features,
                                    size_t batch_size,
                                    void *stream);

/* Replaces cuda_features.h:20 (features.cu:171-173).  Returns 1 iff the
 * stream drained without error. */
int tb_cuda_synchronize(void *stream);

typedef struct tb_cuda_feature_batch tb_cuda_feature_batch;

/* Replaces cuda_features.h:26 (features.cu:27-44).  Makes `device_id`
 * current on the calling thread, creates a non-blocking stream and device
 * staging buffers for `max_batch` environments.  NULL when max_batch is 0 or
 * above 1024, when the device cannot be selected, or on any allocation
 * failure (partial state is released). */
tb_cuda_feature_batch *tb_cuda_feature_batch_create(int device_id, size_t max_batch);

/* Replaces cuda_features.h:27 (features.cu:46-56).  NULL-safe.  Drains the
 * handle's stream before releasing its buffers. */
void tb_cuda_feature_batch_destroy(tb_cuda_feature_batch *batch);

/* Replaces cuda_features.h:28 (features.cu:58-60).  The handle's last error
 * text ("<stage>: <runtime message>", empty after a successful call), or a
 * fixed message for a NULL handle.  Owned by the library. */
const char *tb_cuda_feature_batch_error(const tb_cuda_feature_batch *batch);

/* Replaces cuda_features.h:29-34 (features.cu:62-88).  Host pointers, all
 * required.  Returns 0 with the error text untouched when an argument is NULL
 * or count is outside 1..max_batch.  Otherwise copies the inputs to the
 * device, extracts, copies the features back and waits; returns 1, or 0 with
 * the failing stage recorded.  Not thread-safe per handle. */
int tb_cuda_extract_features_host(tb_cuda_feature_batch *batch,
                                  const float *obs_4148,
                                  const float *mission_10,
                                  const unsigned char *cameras_16384,
                                  size_t count,
                                  float *out_features_142);

#ifdef __cplusplus
}
#endif

#endif
