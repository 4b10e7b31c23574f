/*
 * Host staging object of the sensor-feature boundary, in C11 over the HIP
 * runtime C API.  Behaviour follows the reference host object
 * src/cuda/features.cu:9-88: a handle owns one non-blocking stream and
 * device buffers for up to max_batch (<= 1024) environments; extraction
 * copies the caller's host arrays in, runs the device entry, copies the 142
 * features out and waits.  Failures record "<stage>: <runtime message>" in
 * the handle; argument errors return 0 and leave the text untouched.
 */
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "turbinator/training/cuda_features.h"

enum {
    FB_OBS = 4148,
    FB_MISSION = 10,
    FB_CAMERA = 16384,
    FB_FEATURES = 142,
    FB_MAX_BATCH = 1024
};

struct tb_cuda_feature_batch {
    int device_id;
    size_t max_batch;
    hipStream_t stream;
    float *obs;
    float *mission;
    unsigned char *cameras;
    float *features;
    char error[192];
};

/* The device entry reads (and so clears) the launch error itself; a refused
 * launch whose error is already cleared is reported as a launch failure
 * rather than as "no error". */
static hipError_t launch_status(void) {
    const hipError_t status = hipGetLastError();
    return status == hipSuccess ? hipErrorLaunchFailure : status;
}

static int fb_fail(tb_cuda_feature_batch *batch, const char *stage, hipError_t status) {
    snprintf(batch->error, sizeof(batch->error), "%s: %s", stage, hipGetErrorString(status));
    return 0;
}

tb_cuda_feature_batch *tb_cuda_feature_batch_create(int device_id, size_t max_batch) {
    if (max_batch == 0 || max_batch > FB_MAX_BATCH) return NULL;
    if (hipSetDevice(device_id) != hipSuccess) return NULL;
    tb_cuda_feature_batch *batch = (tb_cuda_feature_batch *)calloc(1, sizeof(*batch));
    if (!batch) return NULL;
    batch->device_id = device_id;
    batch->max_batch = max_batch;
    if (hipStreamCreateWithFlags(&batch->stream, hipStreamNonBlocking) != hipSuccess) {
        batch->stream = NULL;
        tb_cuda_feature_batch_destroy(batch);
        return NULL;
    }
    if (hipMalloc((void **)&batch->obs, max_batch * FB_OBS * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&batch->mission, max_batch * FB_MISSION * sizeof(float)) != hipSuccess ||
        hipMalloc((void **)&batch->cameras, max_batch * FB_CAMERA) != hipSuccess ||
        hipMalloc((void **)&batch->features, max_batch * FB_FEATURES * sizeof(float)) != hipSuccess) {
        tb_cuda_feature_batch_destroy(batch);
        return NULL;
    }
    return batch;
}

void tb_cuda_feature_batch_destroy(tb_cuda_feature_batch *batch) {
    if (!batch) return;
    (void)hipSetDevice(batch->device_id);
    if (batch->stream) (void)hipStreamSynchronize(batch->stream);
    if (batch->obs) (void)hipFree(batch->obs);
    if (batch->mission) (void)hipFree(batch->mission);
    if (batch->cameras) (void)hipFree(batch->cameras);
    if (batch->features) (void)hipFree(batch->features);
    if (batch->stream) (void)hipStreamDestroy(batch->stream);
    free(batch);
}

const char *tb_cuda_feature_batch_error(const tb_cuda_feature_batch *batch) {
    return batch ? batch->error : "CUDA feature batch unavailable";
}

int tb_cuda_extract_features_host(tb_cuda_feature_batch *batch, const float *obs,
                                  const float *mission, const unsigned char *cameras,
                                  size_t count, float *out_features) {
    if (!batch || !obs || !mission || !cameras || !out_features || count == 0 ||
        count > batch->max_batch)
        return 0;
    batch->error[0] = 0;
    hipError_t status = hipSetDevice(batch->device_id);
    if (status != hipSuccess) return fb_fail(batch, "select device", status);
    status = hipMemcpyAsync(batch->obs, obs, count * FB_OBS * sizeof(float),
                            hipMemcpyHostToDevice, batch->stream);
    if (status != hipSuccess) return fb_fail(batch, "copy observations", status);
    status = hipMemcpyAsync(batch->mission, mission, count * FB_MISSION * sizeof(float),
                            hipMemcpyHostToDevice, batch->stream);
    if (status != hipSuccess) return fb_fail(batch, "copy mission", status);
    status = hipMemcpyAsync(batch->cameras, cameras, count * FB_CAMERA, hipMemcpyHostToDevice,
                            batch->stream);
    if (status != hipSuccess) return fb_fail(batch, "copy cameras", status);
    if (!tb_cuda_extract_features_device(batch->obs, batch->mission, batch->cameras,
                                         batch->features, count, batch->stream))
        return fb_fail(batch, "extract features", launch_status());
    status = hipMemcpyAsync(out_features, batch->features, count * FB_FEATURES * sizeof(float),
                            hipMemcpyDeviceToHost, batch->stream);
    if (status != hipSuccess) return fb_fail(batch, "copy features", status);
    status = hipStreamSynchronize(batch->stream);
    return status == hipSuccess ? 1 : fb_fail(batch, "synchronize features", status);
}
