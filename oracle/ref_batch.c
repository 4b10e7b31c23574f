/*
 * TEST INFRASTRUCTURE ONLY (CPU baseline timing).  A threaded batch driver
 * around the reference's own CPU feature twin, tb_train_extract_features_cpu
 * (src/training/training.c:102-142, declared in
 * include/turbinator/training/training.h:55-58), which the Makefile compiles
 * from the reference source into the same library.  Environments are split
 * into contiguous ranges, one per thread; each call is the reference's
 * single-environment function, unchanged.
 */
#include <pthread.h>
#include <stddef.h>

void tb_train_extract_features_cpu(const float *obs, const float *mission,
                                   const unsigned char *cameras, float *out_features);

enum { RB_OBS = 4148, RB_MISSION = 10, RB_CAMERA = 16384, RB_FEATURES = 142, RB_MAX_THREADS = 256 };

typedef struct {
    const float *obs, *mission;
    const unsigned char *cameras;
    float *out;
    size_t begin, end;
} rb_job;

static void *rb_run(void *arg) {
    const rb_job *j = (const rb_job *)arg;
    for (size_t e = j->begin; e < j->end; ++e)
        tb_train_extract_features_cpu(j->obs + e * RB_OBS, j->mission + e * RB_MISSION,
                                      j->cameras ? j->cameras + e * RB_CAMERA : NULL,
                                      j->out + e * RB_FEATURES);
    return NULL;
}

/* Dense rows: obs [batch,4148], mission [batch,10], cameras [batch,16384]
 * (may be NULL), out [batch,142]. */
void ref_features_batch(const float *obs, const float *mission, const unsigned char *cameras,
                        float *out, size_t batch, int threads) {
    if (threads < 1) threads = 1;
    if (threads > RB_MAX_THREADS) threads = RB_MAX_THREADS;
    if ((size_t)threads > batch) threads = batch ? (int)batch : 1;
    rb_job jobs[RB_MAX_THREADS];
    pthread_t tids[RB_MAX_THREADS];
    int started[RB_MAX_THREADS] = {0};
    for (int t = 0; t < threads; ++t) {
        jobs[t].obs = obs;
        jobs[t].mission = mission;
        jobs[t].cameras = cameras;
        jobs[t].out = out;
        jobs[t].begin = batch * (size_t)t / (size_t)threads;
        jobs[t].end = batch * (size_t)(t + 1) / (size_t)threads;
    }
    for (int t = 1; t < threads; ++t) {
        if (pthread_create(&tids[t], NULL, rb_run, &jobs[t]) == 0)
            started[t] = 1;
        else
            rb_run(&jobs[t]);  /* run inline if a thread cannot start */
    }
    rb_run(&jobs[0]);
    for (int t = 1; t < threads; ++t)
        if (started[t]) pthread_join(tids[t], NULL);
}
