/*
 * Host helpers of the batched compact SAC actor (C11):
 *
 *  - tb_hip_sac_read_actor: the actor network of a checkpoint written by
 *    tb_sac_save (src/training/training.c:605-620).  The file holds an 8-byte
 *    magic "TBSAC01", the tb_train_config struct (LP64 layout, 64 bytes), the
 *    agent's rng state, the update count, three floats of the temperature
 *    optimiser, then each network as written by tb_net_write (:580-590): a
 *    step count, and per layer w, b, and the Adam moments mw, vw, mb, vb.
 *    Only the actor's w and b are returned, concatenated as
 *    w0[hidden][142] b0[hidden] w1[hidden][hidden] b1[hidden] w2[30][hidden]
 *    b2[30], the layout tb_hip_sac_actor_pack_device takes.
 *
 *  - tb_hip_sac_normals: the agent's normal draws (training.c:82-100:
 *    xorshift64* words, 24-bit uniforms, Box-Muller cosine branch).  Drawing
 *    15 per environment in order reproduces the stream that consecutive
 *    tb_sac_act_features(..., deterministic = 0, ...) calls consume.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "turbinator/training/hip_features.h"

enum { SAC_FEATURES = 142, SAC_RAW = 30, SAC_MIN_HIDDEN = 16, SAC_MAX_HIDDEN = 256 };

/* Mirrors the reference's tb_train_config (training.h:23-37) byte for byte. */
struct sac_config_image {
    uint64_t seed;
    size_t replay_capacity;
    int hidden_dim;
    float gamma, tau, actor_lr, critic_lr, alpha_lr, initial_alpha, target_entropy,
        reference_weight, max_grad_norm, reward_scale;
};

static int read_exact(FILE *f, void *dst, size_t bytes) {
    return fread(dst, 1, bytes, f) == bytes;
}

static int skip_bytes(FILE *f, size_t bytes) {
    return fseek(f, (long)bytes, SEEK_CUR) == 0;
}

size_t tb_hip_sac_read_actor(const char *path, float *weights, size_t capacity, int *hidden,
                             uint64_t *rng_state) {
    if (!path) return 0;
    FILE *f = fopen(path, "rb");
    if (!f) return 0;
    static const char magic_expected[8] = {'T', 'B', 'S', 'A', 'C', '0', '1', '\0'};
    char magic[8];
    struct sac_config_image cfg;
    uint64_t rng = 0, updates = 0, steps = 0;
    float alpha_state[3];
    size_t written = 0, need = 0;
    int ok = read_exact(f, magic, sizeof magic) && memcmp(magic, magic_expected, 8) == 0 &&
             read_exact(f, &cfg, sizeof cfg) && read_exact(f, &rng, sizeof rng) &&
             read_exact(f, &updates, sizeof updates) &&
             read_exact(f, alpha_state, sizeof alpha_state) && read_exact(f, &steps, sizeof steps);
    const int h = ok ? cfg.hidden_dim : 0;
    if (h < SAC_MIN_HIDDEN || h > SAC_MAX_HIDDEN) ok = 0;
    const int inputs[3] = {SAC_FEATURES, h, h};
    const int outputs[3] = {h, h, SAC_RAW};
    if (ok) {
        /* The actor with its Adam moments must lie inside the file: fseek past
         * the end would succeed, so check the length first. */
        for (int l = 0; l < 3; ++l) need += (size_t)inputs[l] * outputs[l] + outputs[l];
        const long here = ftell(f);
        ok = here >= 0 && fseek(f, 0, SEEK_END) == 0;
        const long end = ok ? ftell(f) : -1;
        ok = ok && end >= here && (size_t)(end - here) >= 3 * need * sizeof(float) &&
             fseek(f, here, SEEK_SET) == 0;
    }
    if (ok) {
        const int copy = weights && capacity >= need;
        for (int l = 0; ok && l < 3; ++l) {
            const size_t wc = (size_t)inputs[l] * outputs[l], bc = (size_t)outputs[l];
            if (copy) {
                ok = read_exact(f, weights + written, wc * sizeof(float)) &&
                     read_exact(f, weights + written + wc, bc * sizeof(float));
                written += wc + bc;
            } else {
                ok = skip_bytes(f, (wc + bc) * sizeof(float));
            }
            /* Adam moments mw, vw, mb, vb */
            ok = ok && skip_bytes(f, (2 * wc + 2 * bc) * sizeof(float));
        }
    }
    fclose(f);
    if (!ok) return 0;
    if (hidden) *hidden = h;
    if (rng_state) *rng_state = rng;
    return need;
}

static uint64_t sac_rand_u64(uint64_t *state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * UINT64_C(2685821657736338717);
}

static float sac_uniform(uint64_t *state) {
    return (float)((sac_rand_u64(state) >> 40) + 0.5) / 16777216.0f;
}

void tb_hip_sac_normals(uint64_t *state, float *out, size_t count) {
    if (!state || !out) return;
    const float two_pi = 2.0f * 3.14159265358979323846f;
    for (size_t i = 0; i < count; ++i) {
        const float u1 = fmaxf(sac_uniform(state), 1.0e-7f);
        const float u2 = sac_uniform(state);
        out[i] = sqrtf(-2.0f * logf(u1)) * cosf(two_pi * u2);
    }
}
