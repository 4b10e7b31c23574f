/*
 * TEST INFRASTRUCTURE ONLY: the CPU checker for the 142-feature path.
 *
 * Restates the reference CPU twin tb_train_extract_features_cpu
 * (src/training/training.c:57-142) operation for operation: the same clamp
 * form, the same finiteness substitution before the division, the same
 * sequential single-precision sector sums (elevation row outer, azimuth bin
 * inner) and the same libm log1pf.  Build with -std=c11 (no FMA contraction,
 * no fast-math) so the arithmetic is the reference's.
 *
 * Pinned by tests/test_oracle.py against: the fixtures written by the
 * reference's own training.c (tests/golden/, oracle/_ref), the reference's
 * 3-environment closed-form fixture and assertions
 * (tests/test_cuda_features.c:17-25, tests/test_training.c:25-35), and closed
 * forms (constant-pixel quadrants, all-sentinel and all-far sectors, scale
 * boundaries).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <string.h>

#define ORC_PI 3.14159265358979323846f

/* training.c:57-59 */
static float orc_clamp(float x, float lo, float hi) {
    if (x < lo) return lo;
    if (x > hi) return hi;
    return x;
}

/* training.c:61-63 */
static float orc_finite_or_zero(float x) {
    return isfinite(x) ? x : 0.0f;
}

/* training.c:65-68.  The denominator is the float log1p of 120. */
float orc_lidar_feature(float range_m) {
    if (!isfinite(range_m) || range_m < 0.0f) return -1.0f;
    return log1pf(orc_clamp(range_m, 0.0f, 120.0f)) / log1pf(120.0f);
}

/* training.c:70-81: per-index divisor of the 48 proprioceptive scalars. */
static float orc_scalar_scale(int i) {
    if (i < 2) return 300.0f;
    if (i == 2) return 100.0f;
    if (i < 6) return 50.0f;
    if (i >= 10 && i < 13) return 5.0f;
    if (i >= 13 && i < 16) return 30.0f;
    if (i >= 28 && i < 32) return ORC_PI / 4.0f;
    if (i >= 32 && i < 40) return 5.0f;
    if (i == 44 || i == 45) return ORC_PI / 2.0f;
    return 1.0f;
}

void orc_features_env(const float *obs, const float *mission,
                      const uint8_t *cameras, float *out) {
    if (!obs || !mission || !out) return;                       /* :106 */
    for (int i = 0; i < 48; ++i)                                /* :107 */
        out[i] = orc_clamp(orc_finite_or_zero(obs[i]) / orc_scalar_scale(i), -1.0f, 1.0f);
    for (int i = 0; i < 4; ++i)                                 /* :108 */
        out[48 + i] = orc_clamp(orc_finite_or_zero(obs[4144 + i]), 0.0f, 1.0f);
    const int arena = orc_finite_or_zero(mission[6]) > 0.5f;    /* :110 */
    for (int i = 0; i < 10; ++i) {                              /* :109-112 */
        const float v = (i >= 7 && arena) ? 0.0f : mission[i];
        out[52 + i] = orc_clamp(orc_finite_or_zero(v), -1.0f, 1.0f);
    }
    /* :113-127: sector (head, el_sector, az_sector) averages rows
     * el_sector*4 .. +3 and bins az_sector*16 .. +15 of its head. */
    for (int head = 0; head < 2; ++head)
        for (int es = 0; es < 4; ++es)
            for (int as = 0; as < 8; ++as) {
                const float *base = obs + 48 + head * 2048 + es * 4 * 128 + as * 16;
                float sum = 0.0f;
                for (int el = 0; el < 4; ++el)
                    for (int az = 0; az < 16; ++az)
                        sum += orc_lidar_feature(base[el * 128 + az]);
                out[62 + head * 32 + es * 8 + as] = sum / 64.0f;
            }
    /* :128-141: integer sum of each 32x32 quadrant, then one division. */
    for (int cam = 0; cam < 4; ++cam)
        for (int qy = 0; qy < 2; ++qy)
            for (int qx = 0; qx < 2; ++qx) {
                unsigned int sum = 0;
                if (cameras) {
                    const uint8_t *q = cameras + cam * 4096 + qy * 32 * 64 + qx * 32;
                    for (int y = 0; y < 32; ++y)
                        for (int x = 0; x < 32; ++x) sum += q[y * 64 + x];
                }
                out[126 + cam * 4 + qy * 2 + qx] = (float)sum / (1024.0f * 255.0f);
            }
}

typedef struct {
    const float *in;
    float *out;
    size_t begin, end;
} orc_map_job;

static void *orc_run_map(void *arg) {
    const orc_map_job *j = (const orc_map_job *)arg;
    for (size_t i = j->begin; i < j->end; ++i) j->out[i] = orc_lidar_feature(j->in[i]);
    return NULL;
}

void orc_lidar_feature_array(const float *in, float *out, size_t n, int threads) {
    enum { MAX_THREADS = 256 };
    if (threads < 1) threads = 1;
    if (threads > MAX_THREADS) threads = MAX_THREADS;
    orc_map_job jobs[MAX_THREADS];
    pthread_t tids[MAX_THREADS];
    int joined[MAX_THREADS] = {0};
    for (int t = 0; t < threads; ++t) {
        jobs[t].in = in; jobs[t].out = out;
        jobs[t].begin = n * (size_t)t / (size_t)threads;
        jobs[t].end = n * (size_t)(t + 1) / (size_t)threads;
    }
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, orc_run_map, &jobs[t]) == 0) joined[t] = 1;
        else orc_run_map(&jobs[t]);
    }
    orc_run_map(&jobs[0]);
    for (int t = 1; t < threads; ++t)
        if (joined[t]) pthread_join(tids[t], NULL);
}

uint8_t orc_depth_to_luma(float depth_m) {
    /* Far plane (200 m) -> 0, near -> 255; round half to even. */
    float d = orc_clamp(orc_finite_or_zero(depth_m), 0.0f, 200.0f);
    float v = 255.0f * (1.0f - d / 200.0f);
    return (uint8_t)lrintf(v);
}

void orc_depth_to_luma_array(const float *depth, uint8_t *luma, size_t n) {
    for (size_t i = 0; i < n; ++i) luma[i] = orc_depth_to_luma(depth[i]);
}

void orc_diagnostics_env(const float *obs, const uint8_t *cameras, uint8_t *diag) {
    for (int head = 0; head < 2; ++head)
        for (int es = 0; es < 4; ++es)
            for (int as = 0; as < 8; ++as) {
                const int s = head * 32 + es * 8 + as;
                float best = 0.0f;
                int best_p = -1, n = 0;
                for (int el = 0; el < 4; ++el)
                    for (int az = 0; az < 16; ++az) {
                        const int bin = head * 2048 + (es * 4 + el) * 128 + as * 16 + az;
                        const float r = obs[48 + bin];
                        if (!isfinite(r) || r < 0.0f) continue;
                        ++n;
                        if (best_p < 0 || r < best) { best = r; best_p = el * 16 + az; }
                    }
                const float m = best_p < 0 ? -1.0f : best;
                const uint16_t word = (uint16_t)((best_p < 0 ? 0xff : best_p) | (n << 8));
                memcpy(diag + 4 * s, &m, 4);
                diag[256 + 2 * s] = (uint8_t)(word & 0xff);
                diag[256 + 2 * s + 1] = (uint8_t)(word >> 8);
            }
    for (int q = 0; q < 16; ++q) {
        const int cam = q / 4, qy = (q / 2) % 2, qx = q % 2;
        int lo = 0, n = 0;
        if (cameras) {
            lo = 255;
            const uint8_t *p = cameras + cam * 4096 + qy * 32 * 64 + qx * 32;
            for (int y = 0; y < 32; ++y)
                for (int x = 0; x < 32; ++x) {
                    const int v = p[y * 64 + x];
                    if (v < lo) lo = v;
                    n += v != 0;
                }
        }
        diag[384 + q] = (uint8_t)lo;
        diag[400 + 2 * q] = (uint8_t)(n & 0xff);
        diag[400 + 2 * q + 1] = (uint8_t)(n >> 8);
    }
}

typedef struct {
    const unsigned char *obs, *mission, *cameras;
    size_t obs_stride, mission_stride, camera_stride;
    float *out;
    size_t begin, end;
} orc_job;

static void *orc_run_job(void *arg) {
    const orc_job *j = (const orc_job *)arg;
    for (size_t e = j->begin; e < j->end; ++e) {
        const float *o = (const float *)(const void *)(j->obs + e * j->obs_stride);
        const float *m = (const float *)(const void *)(j->mission + e * j->mission_stride);
        const uint8_t *c = j->cameras ? j->cameras + e * j->camera_stride : NULL;
        orc_features_env(o, m, c, j->out + e * ORC_FEATURES);
    }
    return NULL;
}

void orc_features_batch(const unsigned char *obs, size_t obs_stride,
                        const unsigned char *mission, size_t mission_stride,
                        const unsigned char *cameras, size_t camera_stride,
                        float *out, size_t batch, int threads) {
    enum { MAX_THREADS = 256 };
    if (threads < 1) threads = 1;
    if (threads > MAX_THREADS) threads = MAX_THREADS;
    if ((size_t)threads > batch) threads = batch ? (int)batch : 1;
    orc_job jobs[MAX_THREADS];
    pthread_t tids[MAX_THREADS];
    for (int t = 0; t < threads; ++t) {
        jobs[t].obs = obs; jobs[t].mission = mission; jobs[t].cameras = cameras;
        jobs[t].obs_stride = obs_stride; jobs[t].mission_stride = mission_stride;
        jobs[t].camera_stride = camera_stride; jobs[t].out = out;
        jobs[t].begin = batch * (size_t)t / (size_t)threads;
        jobs[t].end = batch * (size_t)(t + 1) / (size_t)threads;
    }
    if (threads == 1) { orc_run_job(&jobs[0]); return; }
    int joined[MAX_THREADS] = {0};
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, orc_run_job, &jobs[t]) == 0)
            joined[t] = 1;
        else
            orc_run_job(&jobs[t]);   /* run inline if a thread cannot start */
    }
    orc_run_job(&jobs[0]);
    for (int t = 1; t < threads; ++t)
        if (joined[t]) pthread_join(tids[t], NULL);
}
