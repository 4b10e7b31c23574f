/*
 * Seeded synthetic sensor batches for the parity tests and the benchmark.
 *
 * Every environment draws from its own counter-keyed splitmix64 streams
 * (one per field), so any environment can be regenerated independently and
 * batches can be filled by several threads with identical results.  The
 * mixer is the splitmix64 finaliser the simulator uses for its own streams
 * (reference src/sim/physics.c:73-78).
 *
 * Distributions (per environment):
 *   obs[0..47], obs[4144..4147]   N(0,1), Box-Muller in double, rounded to float
 *   LiDAR obs[48..4143]           U[0.2, 300) m; 10% no-return sentinel -1
 *   mission[0..9]                 U[-1.5, 1.5); mission[6] in {0,1}, 12.5% arena
 *   camera depth                  U[0.5, 200) m; 15% far plane (200 m)
 *   camera luma (uint8)           255 * (1 - depth/200), round half to even
 *
 * Variants (edge-case quarters of the 4,096-env parity batch and more):
 *   1 every LiDAR bin is the no-return sentinel
 *   2 every camera pixel is at 37.5 m (luma 207)
 *   3 tied minimum ranges: three bins per sector share the sector minimum
 *   4 LiDAR values exactly at 0.2, 120 and 300 m; scalars exactly at +-scale
 *   5 non-finite and signed-zero values in every input field
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define SYN_OBS 4148
#define SYN_MISSION 10
#define SYN_CAMERA 16384

enum { FIELD_STATE = 1, FIELD_LIDAR = 2, FIELD_MISSION = 3, FIELD_CAMERA = 4, FIELD_EDGE = 5 };

static uint64_t syn_next(uint64_t *s) {
    uint64_t z = (*s += UINT64_C(0x9e3779b97f4a7c15));
    z = (z ^ (z >> 30)) * UINT64_C(0xbf58476d1ce4e5b9);
    z = (z ^ (z >> 27)) * UINT64_C(0x94d049bb133111eb);
    return z ^ (z >> 31);
}

static uint64_t syn_stream(uint64_t seed, uint64_t env, uint64_t field) {
    uint64_t s = seed ^ (field * UINT64_C(0xd1b54a32d192ed03));
    uint64_t k = syn_next(&s) ^ (env * UINT64_C(0x8cb92ba72f3d8dd7));
    return syn_next(&k);
}

/* 24 random bits as a float in [0, 1). */
static float syn_unit(uint64_t r) {
    return (float)(r >> 40) * (1.0f / 16777216.0f);
}

static double syn_unit_double(uint64_t *s) {
    return ((double)(syn_next(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

static float syn_normal(uint64_t *s) {
    const double u = syn_unit_double(s), v = syn_unit_double(s);
    return (float)(sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v));
}

static uint8_t syn_luma(float depth_m) {
    float d = depth_m < 0.0f ? 0.0f : (depth_m > 200.0f ? 200.0f : depth_m);
    return (uint8_t)lrintf(255.0f * (1.0f - d / 200.0f));
}

static const float syn_scale[48] = {
    300, 300, 100, 50, 50, 50, 1, 1, 1, 1, 5, 5, 5, 30, 30, 30,
    1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0,
    5, 5, 5, 5, 5, 5, 5, 5, 1, 1, 1, 1, 0, 0, 1, 1
};

static float syn_scale_of(int i) {
    const float pi = 3.14159265358979323846f;
    if (i >= 28 && i < 32) return pi / 4.0f;
    if (i == 44 || i == 45) return pi / 2.0f;
    return syn_scale[i];
}

void tb_synth_env(uint64_t seed, uint64_t env, int variant,
                  float *obs, float *mission, uint8_t *cameras, float *depth) {
    uint64_t s = syn_stream(seed, env, FIELD_STATE);
    for (int i = 0; i < 48; ++i) obs[i] = syn_normal(&s);
    for (int i = 0; i < 4; ++i) obs[4144 + i] = syn_normal(&s);

    float *lidar = obs + 48;
    s = syn_stream(seed, env, FIELD_LIDAR);
    const float lo = variant == 3 ? 1.0f : 0.2f;
    for (int b = 0; b < 4096; ++b) {
        const uint64_t r = syn_next(&s);
        const unsigned pick = (unsigned)(r & 0xffffu);
        if (variant == 1 || pick < 6554u) { lidar[b] = -1.0f; continue; }
        float v = lo + (300.0f - lo) * syn_unit(r);
        if (variant == 4) {
            const unsigned edge = (unsigned)((r >> 16) & 0xffu);
            if (edge < 13u) v = 0.2f;
            else if (edge < 26u) v = 300.0f;
            else if (edge < 39u) v = 120.0f;
        }
        lidar[b] = v;
    }
    if (variant == 3) {
        /* Three bins of every sector take the same value, below every other
         * bin of the sector; sectors alternate between two tie values so
         * ties also repeat across sectors. */
        uint64_t t = syn_stream(seed, env, FIELD_EDGE);
        for (int sector = 0; sector < 64; ++sector) {
            const int head = sector / 32, es = (sector / 8) % 4, as = sector % 8;
            const float tie = (sector & 1) ? 0.75f : 0.5f;
            for (int k = 0; k < 3; ++k) {
                const uint64_t r = syn_next(&t);
                const int el = (int)(r & 3u), az = (int)((r >> 2) & 15u);
                lidar[head * 2048 + (es * 4 + el) * 128 + as * 16 + az] = tie;
            }
        }
    }
    if (variant == 4) {
        uint64_t t = syn_stream(seed, env, FIELD_EDGE);
        for (int i = 0; i < 48; ++i) {
            const uint64_t r = syn_next(&t);
            if ((r & 3u) == 0) obs[i] = ((r >> 2) & 1u) ? syn_scale_of(i) : -syn_scale_of(i);
        }
        obs[4144] = 1.0f;
        obs[4145] = 0.0f;
    }

    s = syn_stream(seed, env, FIELD_MISSION);
    for (int i = 0; i < 10; ++i) mission[i] = -1.5f + 3.0f * syn_unit(syn_next(&s));
    mission[6] = (syn_next(&s) & 7u) == 0 ? 1.0f : 0.0f;
    if (variant == 4) {
        mission[0] = 1.0f;
        mission[1] = -1.0f;
        mission[6] = (env & 1u) ? 0.5f : 1.0f;
    }

    s = syn_stream(seed, env, FIELD_CAMERA);
    for (int p = 0; p < SYN_CAMERA; ++p) {
        float d;
        if (variant == 2) {
            d = 37.5f;
        } else {
            const uint64_t r = syn_next(&s);
            d = (r & 0xffffu) < 9830u ? 200.0f : 0.5f + 199.5f * syn_unit(r);
        }
        if (depth) depth[p] = d;
        if (cameras) cameras[p] = syn_luma(d);
    }

    if (variant == 5) {
        const float inf = INFINITY, nan = NAN;
        uint64_t t = syn_stream(seed, env, FIELD_EDGE);
        const float special[6] = {nan, inf, -inf, -0.0f, 0.0f, 3.0e38f};
        for (int i = 0; i < 48; ++i) {
            const uint64_t r = syn_next(&t);
            if ((r & 1u) == 0) obs[i] = special[(r >> 1) % 6u];
        }
        for (int i = 0; i < 4; ++i) obs[4144 + i] = special[(env + (uint64_t)i) % 6u];
        for (int b = 0; b < 4096; ++b) {
            const uint64_t r = syn_next(&t);
            if ((r & 7u) == 0) lidar[b] = special[(r >> 3) % 6u];
        }
        for (int i = 0; i < 10; ++i) {
            const uint64_t r = syn_next(&t);
            if ((r & 1u) == 0) mission[i] = special[(r >> 1) % 6u];
        }
        mission[6] = special[env % 6u];
    }
}

typedef struct {
    uint64_t seed;
    int variant;
    size_t batch, begin, end;
    unsigned char *obs, *mission, *cameras;
    size_t obs_stride, mission_stride, camera_stride;
    float *depth;
} syn_job;

static int syn_variant_for(const syn_job *j, size_t env) {
    if (j->variant >= 0) return j->variant;
    /* -1: four equal quarters, variants 1..4 in order. */
    return 1 + (int)((env * 4) / j->batch);
}

static void *syn_run(void *arg) {
    const syn_job *j = (const syn_job *)arg;
    float obs[SYN_OBS], mission[SYN_MISSION];
    for (size_t e = j->begin; e < j->end; ++e) {
        uint8_t *cam = j->cameras ? j->cameras + e * j->camera_stride : NULL;
        float *dep = j->depth ? j->depth + e * SYN_CAMERA : NULL;
        tb_synth_env(j->seed, e, syn_variant_for(j, e), obs, mission, cam, dep);
        memcpy(j->obs + e * j->obs_stride, obs, sizeof(obs));
        memcpy(j->mission + e * j->mission_stride, mission, sizeof(mission));
    }
    return NULL;
}

/* Fills `batch` environments at byte strides (records may interleave other
 * data).  variant -1 selects the four-quarter edge layout.  cameras and depth
 * may be NULL; depth rows are dense [batch, 16384] floats. */
void tb_synth_batch(uint64_t seed, int variant, size_t batch,
                    unsigned char *obs, size_t obs_stride,
                    unsigned char *mission, size_t mission_stride,
                    unsigned char *cameras, size_t camera_stride,
                    float *depth, int threads) {
    enum { MAX_THREADS = 128 };
    if (threads < 1) threads = 1;
    if (threads > MAX_THREADS) threads = MAX_THREADS;
    if ((size_t)threads > batch) threads = batch ? (int)batch : 1;
    syn_job jobs[MAX_THREADS];
    pthread_t tids[MAX_THREADS];
    int joined[MAX_THREADS] = {0};
    for (int t = 0; t < threads; ++t) {
        syn_job *j = &jobs[t];
        j->seed = seed; j->variant = variant; j->batch = batch;
        j->begin = batch * (size_t)t / (size_t)threads;
        j->end = batch * (size_t)(t + 1) / (size_t)threads;
        j->obs = obs; j->mission = mission; j->cameras = cameras; j->depth = depth;
        j->obs_stride = obs_stride; j->mission_stride = mission_stride;
        j->camera_stride = camera_stride;
    }
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, syn_run, &jobs[t]) == 0) joined[t] = 1;
        else syn_run(&jobs[t]);
    }
    syn_run(&jobs[0]);
    for (int t = 1; t < threads; ++t)
        if (joined[t]) pthread_join(tids[t], NULL);
}
