/*
 * Extensions of the sensor-feature boundary offered by the gfx950 backend
 * (libturbinator_hip).  They have no declaration in the reference header
 * include/turbinator/training/cuda_features.h; each one states the
 * reference code whose semantics it reuses.  All entries are asynchronous on
 * `stream` (a hipStream_t as void*, NULL = null stream) and return 1 iff the
 * launch was accepted, 0 on invalid arguments (nothing is launched then).
 */
#ifndef TURBINATOR_HIP_FEATURES_H
#define TURBINATOR_HIP_FEATURES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layout version of these extensions, for callers that size the optional
 * diagnostics outputs themselves.  The entries kept their names and
 * signatures across these changes:
 *   2  TB_HIP_ONBOARD_DIAG_DIM 4 -> 5 (cluster y sum appended to the onboard
 *      scan diagnostics); diagnostics rows 896 bytes (224 words) -> 432
 *      bytes (TB_HIP_DIAG_BYTES, layout below)
 *   3  the diagnostics pointer must be 16-byte aligned (was 4-byte) */
#define TB_HIP_FEATURES_ABI_VERSION 3

enum {
    TB_HIP_OBS_DIM = 4148,
    TB_HIP_MISSION_DIM = 10,
    TB_HIP_CAMERA_BYTES = 16384,
    TB_HIP_FEATURE_DIM = 142,
    TB_HIP_DIAG_BYTES = 432,
    TB_HIP_TACTICAL_DIM = 24,
    TB_HIP_PRIOR_DIM = 15,
    TB_HIP_ONBOARD_DIAG_DIM = 5
};

/* The 142 features of tb_cuda_extract_features_device (reference
 * src/cuda/features.cu:158-169 / src/training/training.c:102-142) read in
 * place from strided records, e.g. the 66,672-byte replay transitions whose
 * field order is tb_gpu_host_batch (include/turbinator/gpu/replay.h:17-30).
 * Strides are bytes between consecutive environments.  obs and mission rows
 * must be 4-byte aligned (base and stride); cameras may have any alignment
 * and may be NULL (features 126..141 = 0).  features rows are dense
 * [batch,142].  Returns 0 for NULL obs/mission/features, batch 0 or above
 * 0x7fffffff, or misaligned float rows. */
int tb_hip_extract_features_strided_device(const void *obs, size_t obs_stride,
                                           const void *mission, size_t mission_stride,
                                           const void *cameras, size_t camera_stride,
                                           float *features,
                                           size_t batch_size, void *stream);

/* Fused replay sampling + features: output row e holds the 142 features of
 * input row indices[e], read in place from storage laid out like the
 * strided entry's (byte strides; e.g. the SoA replay fields of
 * src/gpu/replay.cu:27-48 with strides 16,592 / 40 / 16,384, or 66,672-byte
 * transition records).  This replaces the reference's gather of every
 * sampled field into a batch followed by feature extraction
 * (replay.cu:130-187 then features.cu:158-169) with one pass that reads
 * only the sampled observation bytes.  indices are device uint32 with
 * values < capacity; an output row whose index is >= capacity reads nothing
 * and is filled with NaN.  Same argument rules as the strided entry, plus
 * NULL indices or capacity 0 -> 0. */
int tb_hip_extract_features_indexed_device(const void *obs, size_t obs_stride,
                                           const void *mission, size_t mission_stride,
                                           const void *cameras, size_t camera_stride,
                                           size_t capacity, const unsigned int *indices,
                                           float *features, size_t batch_size, void *stream);

/* The 142 features of tb_cuda_extract_features_device plus, from the same
 * single pass, per-environment diagnostics that have no counterpart in the
 * reference feature vector (training.c:107-141).  `diagnostics` receives
 * [batch, TB_HIP_DIAG_BYTES] bytes per environment, little-endian:
 *   bytes 0..255    float[64]: LiDAR sector minimum range over valid bins
 *                   (-1.0 if the sector has none); valid = finite and >= 0
 *   bytes 256..383  uint16[64]: low byte = position of the sector's first
 *                   minimum in the reference scan order (row outer, bin
 *                   inner) among its 64 bins, p = 16*row + bin, 0xff if
 *                   none; high byte = valid-bin count (0..64).  The bin
 *                   index in the 4,096-bin block is
 *                   head*2048 + (4*el_sector + p/16)*128 + 16*az_sector + p%16
 *   bytes 384..399  uint8[16]: camera quadrant minimum byte (0 when cameras
 *                   is NULL)
 *   bytes 400..431  uint16[16]: camera quadrant occupancy, bytes != 0 (0
 *                   when cameras is NULL)
 * Sector s = head*32 + el_sector*8 + az_sector and quadrant
 * q = cam*4 + qy*2 + qx, the feature vector's orders.  Same argument rules as
 * tb_cuda_extract_features_device; diagnostics must be 16-byte aligned
 * (returns 0 otherwise): the rows are written with 16-byte stores. */
int tb_hip_extract_features_diagnostics_device(const float *obs, const float *mission,
                                               const unsigned char *cameras,
                                               float *features, void *diagnostics,
                                               size_t batch_size, void *stream);

/* The 142 features with the cameras given as fp32 depth in metres
 * ([batch, 16384] floats, 16-byte aligned), the 4x64x64 fp32 cameras of the
 * benchmark configurations.  Each pixel is quantised to the luma byte the
 * reference ABI carries, 255 * (1 - clamp(d, 0, 200) / 200) rounded half to
 * even (far plane 200 m -> 0; non-finite -> 0 m), then features 126..141
 * are the reference quadrant means of those bytes (training.c:128-141).
 * Returns 0 for NULL pointers, a misaligned depth array, batch 0 or above
 * 0x7fffffff. */
int tb_hip_extract_features_depth_device(const float *obs, const float *mission,
                                         const float *depth, float *features,
                                         size_t batch_size, void *stream);

/* Allocation-free variant of the host entry tb_cuda_extract_features_host.
 * It has no counterpart in the reference: it is for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc), which cannot create a tb_cuda_feature_batch.  Host arrays obs
 * [count,4148], mission [count,10], cameras [count,16384] in; out_features
 * [count,142] out.  Synchronous, like the host entry, and it copies pageable
 * host memory, so it cannot be captured into a HIP graph: on a stream under
 * capture it returns 0 with nothing enqueued and the capture intact.  The
 * device staging is a static array of the library, for up to
 * TB_HIP_STATIC_MAX_BATCH environments (8.6 MB, held on every GPU the
 * library runs on until the process ends), on `stream` (NULL: the null
 * stream).  Returns 0 with nothing enqueued for NULL pointers, count 0 or
 * count above TB_HIP_STATIC_MAX_BATCH; 0 also if a copy or the launch
 * fails, after waiting for whatever it had queued, so the host arrays are
 * free again when it returns.  Every call on a GPU uses that GPU's one
 * array: calls that overlap on one GPU race. */
#define TB_HIP_STATIC_MAX_BATCH 256
int tb_hip_extract_features_host_static(const float *obs, const float *mission,
                                        const unsigned char *cameras, size_t count,
                                        float *out_features, void *stream);

/* Per-bin LiDAR transform of the feature kernel, elementwise over `count`
 * floats: -1 for non-finite or negative ranges, otherwise
 * log1p(min(r,120)) / log1pf(120) (reference training.c:65-68).  Exposed so
 * the transform's accuracy can be measured over every float input. */
int tb_hip_lidar_transform_device(const float *ranges, float *out,
                                  size_t count, void *stream);

/* Onboard tactical (24) and physics-prior (15) features of the reference
 * device function tb_onboard_tactical_prior
 * (src/network/onboard_features.cuh:515-519), which has no C entry in the
 * reference: it runs inside the actor input kernel
 * (src/network/network_gpu.cu:274-304).  Device pointers: obs [batch,4148],
 * mission [batch,10] -> tactical [batch,24], prior [batch,15].  `diag`
 * (nullable, [batch,5]) receives the LiDAR scan results the prior uses:
 * closest in-window return of elevations 0..3, its ray index
 * head*768 + el*128 + azi (-1 if none, as float), the corridor minimum, the
 * cluster count (as float) and the cluster's y sum, accumulated in float in
 * the reference's scan order (onboard_features.cuh:231-234).  Without
 * `diag`, each environment's scan covers only what its mission uses (the
 * closest return for dodge, the corridor and cluster for slalom, nothing
 * otherwise), which is faster; tactical and prior are the same either way.
 * Returns 0 for NULL obs/mission/tactical/prior or batch 0 / above
 * 0x7fffffff. */
int tb_hip_onboard_tactical_prior_device(const float *obs, const float *mission,
                                         float *tactical, float *prior, float *diag,
                                         size_t batch_size, void *stream);

/* The 618M actor's sensor preparation in one call, replacing the reference
 * kernels scalar_inputs, lidar_channels and camera_luma
 * (src/network/network_gpu.cu:274-304, 467-483; launched at :1446-1451).
 * Device pointers, row-major per environment:
 *   proprio      [batch, 91]  52 symlog scalars, tactical[24], prior[15]
 *   mission_vec  [batch, 49]  10 finite mission values, tactical, prior
 *   tactical     [batch, 24], prior [batch, 15]
 *   lidar_channels [batch, 6, 16, 128] (nullable): inverse range, range/30
 *                and validity of head c%2 for channel c
 *   camera_luma  [batch, 16384] (nullable): byte / 255 - 0.5
 * obs, cameras, lidar_channels and camera_luma must be 16-byte aligned;
 * camera_luma needs cameras.  Returns 0 for NULL required pointers,
 * misalignment, batch 0 or above 0x7fffffff.  From 1,792 environments with a
 * plane output the scan and control kernels run on a second stream of the
 * device (made once, on first use), forked from `stream` and joined back to
 * it: later work on `stream` sees every output.  Outputs do not depend on
 * the batch size or on the stream mode. */
int tb_hip_actor_inputs_device(const float *obs, const float *mission,
                               const unsigned char *cameras, float *proprio,
                               float *mission_vec, float *tactical, float *prior,
                               float *lidar_channels, float *camera_luma,
                               size_t batch_size, void *stream);

/* Batched compact SAC actor: tb_sac_act_features (src/training/training.c:
 * 382-392 -> tb_actor_sample :306-329 -> tb_net_forward :219-233) for a whole
 * batch of device-resident feature rows, so features need not return to the
 * host between extraction and acting.
 *
 * Weights come in the reference's tb_dense layout, one network of
 * 142 -> hidden -> hidden -> 30 (hidden 16..256): w0[hidden][142], b0[hidden],
 * w1[hidden][hidden], b1[hidden], w2[30][hidden], b2[30].  They are packed
 * once per weight update into a device buffer of
 * tb_hip_sac_actor_packed_bytes(hidden) bytes (16-byte aligned), which the
 * act entry reads; packed_bytes returns 0 for a hidden width out of range.
 * The buffer holds each weight row scaled by a power of two and split into
 * two fp16 pieces for the fp16 matrix cores (products within about 7e-7 of
 * their fp32 value, plus up to 2^-39 of the row's largest magnitude times
 * the other operand for an operand more than 2^28 below its row's largest,
 * whose pieces are fp16 subnormals); weights must be finite: a non-finite
 * weight makes its output NaN for every row, where the reference's would be
 * +-inf or NaN. */
size_t tb_hip_sac_actor_packed_bytes(int hidden);
int tb_hip_sac_actor_pack_device(const float *w0, const float *b0, const float *w1,
                                 const float *b1, const float *w2, const float *b2,
                                 int hidden, void *packed, void *stream);

/* features [batch,142] -> actions [batch,15] in [-1,1].  normals [batch,15]
 * are the standard normal draws of the stochastic policy (the reference
 * scales draw 14 by 0.15 itself); NULL selects the deterministic action, as
 * deterministic = 1 does.  log_prob [batch] (nullable) receives the
 * tanh-squashed Gaussian log-probability, 0 when deterministic.  raw
 * [batch,30] (nullable) receives the network outputs before sampling (15
 * means, 15 unclamped log-std).  Returns 0 for NULL packed / features /
 * actions, a hidden width out of range, misaligned packed weights, batch 0
 * or above 0x7fffffff. */
int tb_hip_sac_actor_act_device(const void *packed, int hidden, const float *features,
                                const float *normals, float *actions, float *log_prob,
                                float *raw, size_t batch_size, void *stream);

/* Host side.  Reads the actor of a tb_sac_save checkpoint (training.c:
 * 580-590, 605-620) as the concatenation w0 b0 w1 b1 w2 b2 above.  Returns
 * the number of floats the actor has (weights are written only when
 * `weights` holds that many; pass NULL to query), with the hidden width and
 * the agent's rng state in the optional out-parameters; 0 for a missing or
 * malformed file. */
size_t tb_hip_sac_read_actor(const char *path, float *weights, size_t capacity, int *hidden,
                             uint64_t *rng_state);

/* The agent's normal stream (training.c:82-100) from `*state`, which is
 * advanced: 15 draws per environment in order reproduce what consecutive
 * stochastic tb_sac_act_features calls consume. */
void tb_hip_sac_normals(uint64_t *state, float *out, size_t count);

/* Pinned, double-buffered staging for host-side producers: the counterpart
 * of the reference host object (cuda_features.h:22-34, features.cu:62-88)
 * for callers that can write their observations into staging memory the
 * library owns.  A pipeline has `slots` (1..8) slots of `max_batch`
 * environments each; every slot owns pinned host buffers, device buffers
 * and a non-blocking stream.  The producer fills a slot's inputs in place
 * (the arrays returned by _inputs, rows laid out as in the reference ABI:
 * obs [max_batch,4148] float, mission [max_batch,10] float, cameras
 * [max_batch,16384] uint8), _submit queues host-to-device copy, extraction
 * and device-to-host copy of the first `count` rows on the slot's stream and
 * returns without waiting, and _wait blocks until the slot is done and
 * returns its pinned [count,142] feature rows (valid until the slot's next
 * submit).  While a slot is in flight its inputs must not be written.
 * Not thread-safe per handle; create selects `device_id` on the calling
 * thread, as the reference create does. */
enum {
    TB_HIP_PIPELINE_MAX_SLOTS = 8,
    TB_HIP_PIPELINE_MAX_BATCH = 0x7fffffff
};

typedef struct tb_hip_feature_pipeline tb_hip_feature_pipeline;

/* NULL for max_batch 0 or above TB_HIP_PIPELINE_MAX_BATCH, slots outside
 * 1..8, a device that cannot be selected, or any allocation failure. */
tb_hip_feature_pipeline *tb_hip_feature_pipeline_create(int device_id, size_t max_batch,
                                                        int slots);

/* NULL-safe; drains every slot's stream before freeing. */
void tb_hip_feature_pipeline_destroy(tb_hip_feature_pipeline *pipeline);

/* Last error text ("<stage>: <runtime message>", or a slot-state message
 * such as "submit: slot 1 is in flight"); a fixed message for NULL. */
const char *tb_hip_feature_pipeline_error(const tb_hip_feature_pipeline *pipeline);

/* Writes the slot's pinned input arrays to the non-NULL out-parameters.
 * Returns 0 for a NULL pipeline or a slot out of range. */
int tb_hip_feature_pipeline_inputs(tb_hip_feature_pipeline *pipeline, int slot, float **obs,
                                   float **mission, unsigned char **cameras);

/* Queues the slot's first `count` environments.  with_cameras = 0 skips the
 * camera copy and zeroes features 126..141 (the device entry's NULL-cameras
 * rule).  Returns 1 when queued; 0 with the error text untouched for a NULL
 * pipeline, a slot out of range or count outside 1..max_batch; 0 with the
 * error set when the slot is still in flight or a runtime call fails. */
int tb_hip_feature_pipeline_submit(tb_hip_feature_pipeline *pipeline, int slot, size_t count,
                                   int with_cameras);

/* Like _submit, but the extraction runs on the slot's pinned memory itself:
 * the kernel reads the inputs over PCIe and writes the features into the
 * pinned rows that _wait returns, with no copy-engine transfers.  Same
 * argument and slot-state rules as _submit; 0 with the error set when the
 * runtime cannot map the slot's pinned memory for the device. */
int tb_hip_feature_pipeline_submit_direct(tb_hip_feature_pipeline *pipeline, int slot,
                                          size_t count, int with_cameras);

/* Waits for the slot and returns its feature rows, or NULL (error set) when
 * the slot has never been submitted or the stream failed.  Waiting again on
 * a completed slot returns the same rows. */
const float *tb_hip_feature_pipeline_wait(tb_hip_feature_pipeline *pipeline, int slot);

#ifdef __cplusplus
}
#endif

#endif
