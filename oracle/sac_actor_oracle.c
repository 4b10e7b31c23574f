/*
 * TEST INFRASTRUCTURE ONLY: the CPU checker for the batched compact SAC
 * actor, restating for one environment
 *   tb_net_forward    src/training/training.c:219-233 (3 dense layers,
 *                     tanh on the hidden two, sequential float sums)
 *   tb_actor_sample   src/training/training.c:306-329 (clamped log-std,
 *                     tanh-squashed Gaussian, log-probability)
 *   tb_rand_u64 / tb_uniform / tb_normal  training.c:82-100 (the agent's
 *                     random stream, to reproduce the normals it draws)
 * compiled as the reference compiles training.c (ISO C11, no FMA
 * contraction), so each value matches tb_sac_act_features bit for bit.
 *
 * Weights use the reference's tb_dense layout: w[outputs][inputs], b[outputs].
 * normals (15 values or NULL = deterministic) are the draws tb_normal returns,
 * before the 0.15 scale of the last action.
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

#define ORC_PI 3.14159265358979323846f

static uint64_t orc_rand_u64(uint64_t *state) {          /* training.c:82-89 */
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * UINT64_C(2685821657736338717);
}

static float orc_uniform(uint64_t *state) {               /* training.c:91-93 */
    return (float)((orc_rand_u64(state) >> 40) + 0.5) / 16777216.0f;
}

void orc_sac_normals(uint64_t *state, float *out, size_t count) {   /* :95-99 */
    for (size_t i = 0; i < count; ++i) {
        const float u1 = fmaxf(orc_uniform(state), 1.0e-7f);
        const float u2 = orc_uniform(state);
        out[i] = sqrtf(-2.0f * logf(u1)) * cosf(2.0f * ORC_PI * u2);
    }
}

static float orc_finite(float x) { return isfinite(x) ? x : 0.0f; }
static float orc_clamp(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

static void orc_dense(const float *w, const float *b, int inputs, int outputs, const float *x,
                      float *y, int activate) {
    for (int o = 0; o < outputs; ++o) {
        const float *row = w + (size_t)o * (size_t)inputs;
        float value = b[o];
        for (int i = 0; i < inputs; ++i) value += row[i] * x[i];
        y[o] = activate ? tanhf(value) : value;
    }
}

void orc_sac_actor_env(const float *w0, const float *b0, const float *w1, const float *b1,
                       const float *w2, const float *b2, int hidden, const float *feature,
                       const float *normals, float *action, float *log_prob, float *raw_out) {
    float h0[256], h1[256], raw[30];
    orc_dense(w0, b0, 142, hidden, feature, h0, 1);
    orc_dense(w1, b1, hidden, hidden, h0, h1, 1);
    orc_dense(w2, b2, hidden, 30, h1, raw, 0);
    if (raw_out) memcpy(raw_out, raw, sizeof(raw));
    float lp = 0.0f;
    for (int i = 0; i < 15; ++i) {
        const float raw_ls = orc_finite(raw[15 + i]);
        const float log_std = orc_clamp(raw_ls, -3.5f, -1.6f);
        const float std = expf(log_std);
        const float eps = normals ? normals[i] * (i == 14 ? 0.15f : 1.0f) : 0.0f;
        const float z = orc_clamp(orc_finite(raw[i]) + std * eps, -8.0f, 8.0f);
        const float a = tanhf(z);
        action[i] = a;
        if (normals) {
            const float gaussian = -0.5f * eps * eps - log_std - 0.5f * logf(2.0f * ORC_PI);
            lp += gaussian - logf(1.0f - a * a + 1.0e-6f);
        }
    }
    if (log_prob) *log_prob = lp;
}
