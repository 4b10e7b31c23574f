/*
 * Pinned, double-buffered staging for the host side of the sensor-feature
 * path, in C11 over the HIP runtime C API.
 *
 * The reference host object (src/cuda/features.cu:62-88) copies the
 * caller's pageable arrays in, extracts, copies the features out and waits,
 * once per call: every call pays a pageable copy and a full round trip, and
 * the simulator's next step cannot overlap the transfer.  Here the producer
 * writes its observations straight into pinned staging slots (the
 * simulator's tb_observe_training_batch, src/sim/c_api.c:104-112, fills
 * caller-provided arrays), a submit queues host-to-device copy, extraction
 * and device-to-host copy of one slot on that slot's own stream and returns
 * at once, and a wait hands back the slot's pinned feature rows.  With two
 * slots the next batch is produced while the previous one crosses PCIe.
 * A direct submit instead runs the extraction on the pinned slot itself:
 * the kernel reads the inputs over PCIe and writes the features back into
 * pinned memory, with no copy-engine transfers (the lower-latency choice
 * for small batches).
 *
 * Layout of one slot, identical in pinned host memory and in device memory
 * (n = max_batch):
 *   [0, 16592 n)          obs      [n, 4148] float
 *   [16592 n, 16632 n)    mission  [n, 10]   float
 *   [16632 n, 33016 n)    cameras  [n, 16384] uint8
 *   [33016 n, 33584 n)    features [n, 142]  float
 * so a full slot's inputs are one contiguous copy.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "turbinator/training/cuda_features.h"
#include "turbinator/training/hip_features.h"

enum {
    FP_OBS_BYTES = TB_HIP_OBS_DIM * 4,
    FP_MISSION_BYTES = TB_HIP_MISSION_DIM * 4,
    FP_CAMERA_BYTES = TB_HIP_CAMERA_BYTES,
    FP_FEATURE_BYTES = TB_HIP_FEATURE_DIM * 4,
    FP_ENV_BYTES = FP_OBS_BYTES + FP_MISSION_BYTES + FP_CAMERA_BYTES + FP_FEATURE_BYTES
};

typedef struct {
    hipStream_t stream;
    unsigned char *host;    /* pinned, slot layout above */
    unsigned char *mapped;  /* the same pinned memory as the device addresses it */
    unsigned char *device;  /* device, same layout */
    size_t count;           /* environments of the last submission */
    int in_flight;          /* submitted and not yet waited for */
    int has_result;         /* a completed submission's features are in `host` */
} fp_slot;

struct tb_hip_feature_pipeline {
    int device_id;
    int nslots;
    size_t max_batch;
    fp_slot slot[TB_HIP_PIPELINE_MAX_SLOTS];
    char error[192];
};

static size_t off_mission(size_t n) { return (size_t)FP_OBS_BYTES * n; }
static size_t off_cameras(size_t n) { return (size_t)(FP_OBS_BYTES + FP_MISSION_BYTES) * n; }
static size_t off_features(size_t n) {
    return (size_t)(FP_OBS_BYTES + FP_MISSION_BYTES + FP_CAMERA_BYTES) * n;
}

/* The device entry reads (and so clears) the launch error itself; a refused
 * launch whose error is already cleared is reported as a launch failure
 * rather than as "no error". */
static hipError_t launch_status(void) {
    const hipError_t status = hipGetLastError();
    return status == hipSuccess ? hipErrorLaunchFailure : status;
}

static int fp_fail(tb_hip_feature_pipeline *p, const char *stage, hipError_t status) {
    snprintf(p->error, sizeof(p->error), "%s: %s", stage, hipGetErrorString(status));
    return 0;
}

/* A submit that fails after it has queued work waits for that work before it
 * returns, so the caller may refill the slot's pinned arrays at once. */
static int fp_fail_queued(tb_hip_feature_pipeline *p, fp_slot *q, const char *stage,
                          hipError_t status) {
    fp_fail(p, stage, status);
    (void)hipStreamSynchronize(q->stream);
    (void)hipGetLastError();
    return 0;
}

static int fp_valid_slot(const tb_hip_feature_pipeline *p, int slot) {
    return p && slot >= 0 && slot < p->nslots;
}

tb_hip_feature_pipeline *tb_hip_feature_pipeline_create(int device_id, size_t max_batch,
                                                        int slots) {
    if (max_batch == 0 || max_batch > TB_HIP_PIPELINE_MAX_BATCH || slots < 1 ||
        slots > TB_HIP_PIPELINE_MAX_SLOTS)
        return NULL;
    if (hipSetDevice(device_id) != hipSuccess) return NULL;
    tb_hip_feature_pipeline *p = (tb_hip_feature_pipeline *)calloc(1, sizeof(*p));
    if (!p) return NULL;
    p->device_id = device_id;
    p->nslots = slots;
    p->max_batch = max_batch;
    const size_t bytes = (size_t)FP_ENV_BYTES * max_batch;
    for (int s = 0; s < slots; ++s) {
        fp_slot *q = &p->slot[s];
        if (hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking) != hipSuccess) {
            q->stream = NULL;
            tb_hip_feature_pipeline_destroy(p);
            return NULL;
        }
        if (hipHostMalloc((void **)&q->host, bytes, hipHostMallocDefault) != hipSuccess) {
            q->host = NULL;
            tb_hip_feature_pipeline_destroy(p);
            return NULL;
        }
        if (hipHostGetDevicePointer((void **)&q->mapped, q->host, 0) != hipSuccess) {
            q->mapped = NULL;  /* direct submits report this */
            (void)hipGetLastError();
        }
        if (hipMalloc((void **)&q->device, bytes) != hipSuccess) {
            q->device = NULL;
            tb_hip_feature_pipeline_destroy(p);
            return NULL;
        }
    }
    return p;
}

void tb_hip_feature_pipeline_destroy(tb_hip_feature_pipeline *p) {
    if (!p) return;
    (void)hipSetDevice(p->device_id);
    for (int s = 0; s < p->nslots; ++s) {
        fp_slot *q = &p->slot[s];
        if (q->stream) (void)hipStreamSynchronize(q->stream);
        if (q->device) (void)hipFree(q->device);
        if (q->host) (void)hipHostFree(q->host);
        if (q->stream) (void)hipStreamDestroy(q->stream);
    }
    free(p);
}

const char *tb_hip_feature_pipeline_error(const tb_hip_feature_pipeline *p) {
    return p ? p->error : "HIP feature pipeline unavailable";
}

int tb_hip_feature_pipeline_inputs(tb_hip_feature_pipeline *p, int slot, float **obs,
                                   float **mission, unsigned char **cameras) {
    if (!fp_valid_slot(p, slot)) return 0;
    unsigned char *h = p->slot[slot].host;
    if (obs) *obs = (float *)h;
    if (mission) *mission = (float *)(h + off_mission(p->max_batch));
    if (cameras) *cameras = h + off_cameras(p->max_batch);
    return 1;
}

int tb_hip_feature_pipeline_submit(tb_hip_feature_pipeline *p, int slot, size_t count,
                                   int with_cameras) {
    if (!fp_valid_slot(p, slot) || count == 0 || count > p->max_batch) return 0;
    fp_slot *q = &p->slot[slot];
    if (q->in_flight) {
        snprintf(p->error, sizeof(p->error), "submit: slot %d is in flight", slot);
        return 0;
    }
    p->error[0] = 0;
    const size_t n = p->max_batch;
    hipError_t status = hipSetDevice(p->device_id);
    if (status != hipSuccess) return fp_fail(p, "select device", status);
    q->has_result = 0;
    if (count == n && with_cameras) {
        /* A full slot's obs, mission and cameras are one contiguous range. */
        status = hipMemcpyAsync(q->device, q->host, off_features(n), hipMemcpyHostToDevice,
                                q->stream);
        if (status != hipSuccess) return fp_fail(p, "copy inputs", status);
    } else {
        status = hipMemcpyAsync(q->device, q->host, count * FP_OBS_BYTES, hipMemcpyHostToDevice,
                                q->stream);
        if (status != hipSuccess) return fp_fail(p, "copy observations", status);
        status = hipMemcpyAsync(q->device + off_mission(n), q->host + off_mission(n),
                                count * FP_MISSION_BYTES, hipMemcpyHostToDevice, q->stream);
        if (status != hipSuccess) return fp_fail_queued(p, q, "copy mission", status);
        if (with_cameras) {
            status = hipMemcpyAsync(q->device + off_cameras(n), q->host + off_cameras(n),
                                    count * FP_CAMERA_BYTES, hipMemcpyHostToDevice, q->stream);
            if (status != hipSuccess) return fp_fail_queued(p, q, "copy cameras", status);
        }
    }
    if (!tb_cuda_extract_features_device((const float *)q->device,
                                         (const float *)(q->device + off_mission(n)),
                                         with_cameras ? q->device + off_cameras(n) : NULL,
                                         (float *)(q->device + off_features(n)), count,
                                         q->stream))
        return fp_fail_queued(p, q, "extract features", launch_status());
    status = hipMemcpyAsync(q->host + off_features(n), q->device + off_features(n),
                            count * FP_FEATURE_BYTES, hipMemcpyDeviceToHost, q->stream);
    if (status != hipSuccess) return fp_fail_queued(p, q, "copy features", status);
    q->count = count;
    q->in_flight = 1;
    return 1;
}

int tb_hip_feature_pipeline_submit_direct(tb_hip_feature_pipeline *p, int slot, size_t count,
                                          int with_cameras) {
    if (!fp_valid_slot(p, slot) || count == 0 || count > p->max_batch) return 0;
    fp_slot *q = &p->slot[slot];
    if (q->in_flight) {
        snprintf(p->error, sizeof(p->error), "submit: slot %d is in flight", slot);
        return 0;
    }
    if (!q->mapped) {
        snprintf(p->error, sizeof(p->error), "submit: slot %d is not device-mapped", slot);
        return 0;
    }
    p->error[0] = 0;
    const size_t n = p->max_batch;
    hipError_t status = hipSetDevice(p->device_id);
    if (status != hipSuccess) return fp_fail(p, "select device", status);
    q->has_result = 0;
    if (!tb_cuda_extract_features_device((const float *)q->mapped,
                                         (const float *)(q->mapped + off_mission(n)),
                                         with_cameras ? q->mapped + off_cameras(n) : NULL,
                                         (float *)(q->mapped + off_features(n)), count,
                                         q->stream))
        return fp_fail(p, "extract features", launch_status());
    q->count = count;
    q->in_flight = 1;
    return 1;
}

const float *tb_hip_feature_pipeline_wait(tb_hip_feature_pipeline *p, int slot) {
    if (!fp_valid_slot(p, slot)) return NULL;
    fp_slot *q = &p->slot[slot];
    if (!q->in_flight) {
        if (q->has_result) return (const float *)(q->host + off_features(p->max_batch));
        snprintf(p->error, sizeof(p->error), "wait: slot %d has nothing submitted", slot);
        return NULL;
    }
    q->in_flight = 0;
    hipError_t status = hipSetDevice(p->device_id);
    if (status != hipSuccess) {
        fp_fail(p, "select device", status);
        return NULL;
    }
    status = hipStreamSynchronize(q->stream);
    if (status != hipSuccess) {
        fp_fail(p, "synchronize features", status);
        return NULL;
    }
    q->has_result = 1;
    return (const float *)(q->host + off_features(p->max_batch));
}
