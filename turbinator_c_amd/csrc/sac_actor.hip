// Batched compact SAC actor on gfx950: tb_sac_act_features
// (src/training/training.c:382-392) for a whole batch of feature rows in one
// launch, so the 142-value features never leave HBM.
//
//   tb_net_forward   training.c:219-233  142 -> hidden (tanh) -> hidden (tanh)
//                                        -> 30 (15 means, 15 raw log-std)
//   tb_actor_sample  training.c:306-329  clamped log-std, tanh-squashed
//                                        Gaussian action, log-probability
//
// The three dense layers run on the matrix cores (v_mfma_f32_16x16x4f32,
// fp32 in and out).  Each wave owns 16 environments and computes the
// transposed products  H^T = W * X^T : the weights are the A operand and the
// environments the columns of B.  With that orientation the 16x16 output
// fragment a lane holds (outputs 16t+4g..16t+4g+3 of environment lane%16,
// g = lane/16) is exactly the B-operand fragment the next layer needs for
// input chunk t, so activations stay in registers from layer to layer.
//
// Weights are first packed (tb_hip_sac_actor_pack_device) into that operand
// order: for output tile nt, input chunk s (16 inputs) and lane l, one float4
// holds W[16nt + l%16][16s + 4(l/16) + 0..3], so every weight load of a wave
// is one contiguous 1 KiB read.  Padding rows / columns hold zeros.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "turbinator/training/hip_features.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kFeatures = 142;
constexpr int kActions = 15;
constexpr int kRaw = 2 * kActions;
constexpr int kFeatureChunks = 9;  // 142 inputs padded to 144
constexpr int kRounds = 4;         // 16 x 15 (environment, action) slots over 64 lanes
constexpr int kMinHidden = 16, kMaxHidden = 256;
constexpr float kPi = 3.14159265358979323846f;
constexpr size_t kMaxBatch = 0x7fffffffu;

// Float offsets of the packed sections; every section starts on 256 bytes.
struct Packed {
    int ht;                 // hidden tiles (hidden padded to 16)
    size_t w[3], b[3];      // section offsets (floats)
    size_t total;           // floats
};

__host__ __device__ inline size_t align64(size_t x) { return (x + 63) & ~(size_t)63; }

__host__ __device__ inline Packed packed_layout(int hidden) {
    Packed p;
    p.ht = (hidden + 15) / 16;
    const int kc[3] = {kFeatureChunks, p.ht, p.ht};
    const int nt[3] = {p.ht, p.ht, 2};
    size_t off = 0;
    for (int l = 0; l < 3; ++l) {
        p.w[l] = off;
        off = align64(off + (size_t)nt[l] * kc[l] * 256);
        p.b[l] = off;
        off = align64(off + (size_t)nt[l] * 16);
    }
    p.total = off;
    return p;
}

struct PackArgs {
    const float *w[3], *b[3];
    int k[3], n[3], kc[3], nt[3];
    Packed layout;
    float *out;
};

// One thread per packed float.
__global__ __launch_bounds__(256) void sac_pack_kernel(PackArgs a) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.layout.total;
         i += (size_t)gridDim.x * blockDim.x) {
        float v = 0.0f;
        for (int l = 0; l < 3; ++l) {
            const size_t wsize = (size_t)a.nt[l] * a.kc[l] * 256;
            if (i >= a.layout.w[l] && i < a.layout.w[l] + wsize) {
                const size_t e = i - a.layout.w[l];
                const int t = (int)(e & 3);
                const size_t q = e >> 2;
                const int lane = (int)(q & 63);
                const int s = (int)((q >> 6) % a.kc[l]);
                const int tile = (int)((q >> 6) / a.kc[l]);
                const int n = 16 * tile + (lane & 15);
                const int k = 16 * s + 4 * (lane >> 4) + t;
                if (n < a.n[l] && k < a.k[l]) v = a.w[l][(size_t)n * a.k[l] + k];
            } else if (i >= a.layout.b[l] && i < a.layout.b[l] + (size_t)a.nt[l] * 16) {
                const size_t e = i - a.layout.b[l];
                if (e < (size_t)a.n[l]) v = a.b[l][e];
            }
        }
        a.out[i] = v;
    }
}

struct ActArgs {
    const float *packed;
    unsigned packed_bytes;
    unsigned w_off[3], b_off[3];  // section offsets in bytes
    const float *features, *normals;
    float *actions, *log_prob, *raw;
    size_t batch;
};

// Buffer resources (gfx9 word 3): loads address with one lane-offset VGPR and
// a uniform scalar offset, and read zero past num_records instead of faulting.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             kBufferWord3);
}

// Hidden-layer tanh from tanh(x) = 1 - 2 / (e^{2x} + 1) with the hardware
// exp2 and reciprocal: absolute error ~2e-7 (the reference's tanhf is within
// an ulp), infinities give +-1 and NaN stays NaN.  The next layer only sums
// these values, so an absolute bound is what matters; the action's own tanh
// uses the device library's tanhf.
__device__ __forceinline__ float tanh_hidden(float x) {
    const float e = __builtin_amdgcn_exp2f(x * 2.88539008177792681f);  // 2 / ln 2
    return __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
}

// One dense layer for the wave's 16 environments: out tile nt = W[tile nt] *
// in^T + b, fragments as described at the top of the file.  Output tiles are
// done in groups of up to 8.  The weight chunk of the step after the current
// one is always in flight while the current chunk runs on the matrix cores
// (>= 32 MFMAs of 32 cycles, longer than an L2 hit): within a group, into the
// next group, and from a layer's last step into the next layer's first chunk,
// which is handed over in `first`.  The bias is loaded when a group starts and
// added when it ends.  The scheduling barriers keep the compiler from hoisting
// every load of the layer into registers at once.
constexpr int kGroup = 8;

template <int KC, int NT, bool TANH, int KCN, int NTN>
__device__ __forceinline__ void dense_layer(__amdgpu_buffer_rsrc_t rsrc, unsigned w_off,
                                            unsigned b_off, unsigned next_w_off,
                                            const f32x4 (&in)[KC], f32x4 (&out)[NT],
                                            f32x4 (&first)[kGroup], int lane) {
    constexpr int G = NT < kGroup ? NT : kGroup;
    const int g = lane >> 4;
    const unsigned wlane = 16u * lane;
    f32x4 wc[kGroup], wn[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) wc[i] = first[i];
#pragma unroll
    for (int g0 = 0; g0 < NT; g0 += G) {
        f32x4 acc[G], bias[G];
#pragma unroll
        for (int i = 0; i < G; ++i)
            if (g0 + i < NT) {
                acc[i] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
                bias[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16u * g,
                                                                b_off + 64u * (g0 + i), 0);
            }
#pragma unroll
        for (int s = 0; s < KC; ++s) {
            if (s + 1 < KC) {  // next chunk of this group
#pragma unroll
                for (int i = 0; i < G; ++i)
                    if (g0 + i < NT)
                        wn[i] = __builtin_amdgcn_raw_buffer_load_b128(
                            rsrc, wlane, w_off + 1024u * ((g0 + i) * KC + s + 1), 0);
            } else if (g0 + G < NT) {  // first chunk of the next group
#pragma unroll
                for (int i = 0; i < G; ++i)
                    if (g0 + G + i < NT)
                        wn[i] = __builtin_amdgcn_raw_buffer_load_b128(
                            rsrc, wlane, w_off + 1024u * ((g0 + G + i) * KC), 0);
            } else if (NTN > 0) {  // first chunk of the next layer
#pragma unroll
                for (int i = 0; i < kGroup; ++i)
                    if (i < NTN)
                        wn[i] = __builtin_amdgcn_raw_buffer_load_b128(
                            rsrc, wlane, next_w_off + 1024u * (i * KCN), 0);
            }
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < G; ++i)
                    if (g0 + i < NT)
                        acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(wc[i][t], in[s][t], acc[i],
                                                                      0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < kGroup; ++i) wc[i] = wn[i];
        }
#pragma unroll
        for (int i = 0; i < G; ++i)
            if (g0 + i < NT) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float y = acc[i][v] + bias[i][v];
                    out[g0 + i][v] = TANH ? tanh_hidden(y) : y;
                }
            }
    }
#pragma unroll
    for (int i = 0; i < kGroup; ++i) first[i] = wc[i];
}

__device__ __forceinline__ float finite_or_zero(float x) {  // training.c:61-63
    return __builtin_isfinite(x) ? x : 0.0f;
}
__device__ __forceinline__ float clampf(float x, float lo, float hi) {  // training.c:57-59
    return x < lo ? lo : (x > hi ? hi : x);
}

template <int HT>
__global__ __launch_bounds__(256) void sac_actor_kernel(ActArgs a) {
    __shared__ float raw_s[4][16][33];
    __shared__ float term_s[4][16][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, j = lane & 15;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.packed, a.packed_bytes);
    // Layer 0's first weight chunk; each pass through the layers leaves the
    // next pass's first chunk here (the last layer prefetches layer 0).
    f32x4 first[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i)
        if (i < HT)
            first[i] = __builtin_amdgcn_raw_buffer_load_b128(
                wrs, 16u * lane, a.w_off[0] + 1024u * (i * kFeatureChunks), 0);
    // The loop bound is uniform over the block, so every wave meets the
    // barriers; waves past the batch end compute on zeros and store nothing.
    for (size_t gbase = (size_t)blockIdx.x * 64; gbase < a.batch;
         gbase += (size_t)gridDim.x * 64) {
        const size_t base = gbase + 16 * wave;
        const size_t env = base + j;
        const bool live = env < a.batch;
        // This group's feature rows; rows past the batch end read as zero.
        const size_t rows = a.batch - gbase < 64 ? a.batch - gbase : 64;
        const __amdgpu_buffer_rsrc_t frs =
            make_rsrc(a.features + gbase * kFeatures, (unsigned)(rows * kFeatures * 4));
        const unsigned frow = (unsigned)(16 * wave + j) * kFeatures * 4;
        f32x4 x[kFeatureChunks];
#pragma unroll
        for (int s = 0; s < kFeatureChunks; ++s) {
            // Inputs 16s+4g .. +3; rows are 568 bytes, so 8-byte loads stay aligned.
            const unsigned off = frow + (unsigned)(16 * s + 4 * g) * 4;
            typedef float f32x2 __attribute__((ext_vector_type(2)));
            const f32x2 lo = __builtin_bit_cast(
                f32x2, __builtin_amdgcn_raw_buffer_load_b64(frs, off, 0, 0));
            f32x2 hi = {0.0f, 0.0f};
            if (s + 1 < kFeatureChunks || g < 3)  // inputs 142, 143 are padding
                hi = __builtin_bit_cast(f32x2,
                                        __builtin_amdgcn_raw_buffer_load_b64(frs, off + 8, 0, 0));
            x[s] = (f32x4){lo[0], lo[1], hi[0], hi[1]};
        }
        // The group's normals (slot p = 15 e + i of environment base + e),
        // loaded now and used after the three layers.
        float drawn[kRounds];
#pragma unroll
        for (int round = 0; round < kRounds; ++round) {
            const int p = lane + 64 * round;
            drawn[round] = 0.0f;
            if (a.normals && p < 16 * kActions && base + p / kActions < a.batch)
                drawn[round] = a.normals[base * kActions + p];
        }
        f32x4 h0[HT], h1[HT], r[2];
        dense_layer<kFeatureChunks, HT, true, HT, HT>(wrs, a.w_off[0], a.b_off[0], a.w_off[1], x,
                                                      h0, first, lane);
        dense_layer<HT, HT, true, HT, 2>(wrs, a.w_off[1], a.b_off[1], a.w_off[2], h0, h1, first,
                                         lane);
        dense_layer<HT, 2, false, kFeatureChunks, (HT < kGroup ? HT : kGroup)>(
            wrs, a.w_off[2], a.b_off[2], a.w_off[0], h1, r, first, lane);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = 16 * nt + 4 * g + v;
                raw_s[wave][j][n] = r[nt][v];
                if (a.raw && live && n < kRaw) a.raw[env * kRaw + n] = r[nt][v];
            }
        __syncthreads();
        // training.c:310-327 for the wave's 16 x 15 (environment, action)
        // pairs, consecutive lanes on consecutive action slots.
#pragma unroll
        for (int round = 0; round < kRounds; ++round) {
            const int p = lane + 64 * round;
            const int e = p / kActions, i = p - kActions * e;
            const size_t ge = base + e;
            if (p >= 16 * kActions || ge >= a.batch) continue;
            const float raw_ls = finite_or_zero(raw_s[wave][e][kActions + i]);
            const float log_std = clampf(raw_ls, -3.5f, -1.6f);
            const float sd = expf(log_std);
            const float eps = a.normals ? drawn[round] * (i == 14 ? 0.15f : 1.0f) : 0.0f;
            const float z = clampf(finite_or_zero(raw_s[wave][e][i]) + sd * eps, -8.0f, 8.0f);
            const float act = tanhf(z);
            a.actions[ge * kActions + i] = act;
            const float gaussian = -0.5f * eps * eps - log_std - 0.5f * logf(2.0f * kPi);
            term_s[wave][e][i] = gaussian - logf(1.0f - act * act + 1.0e-6f);
        }
        __syncthreads();
        if (a.log_prob && lane < 16 && base + lane < a.batch) {
            float lp = 0.0f;  // summed in action order, as the reference does
            if (a.normals)
                for (int i = 0; i < kActions; ++i) lp += term_s[wave][lane][i];
            a.log_prob[base + lane] = lp;
        }
    }
}

template <int HT>
void launch_act(const ActArgs &a, unsigned blocks, hipStream_t s) {
    sac_actor_kernel<HT><<<blocks, 256, 0, s>>>(a);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t tb_hip_sac_actor_packed_bytes(int hidden) {
    if (hidden < kMinHidden || hidden > kMaxHidden) return 0;
    return packed_layout(hidden).total * sizeof(float);
}

extern "C" int tb_hip_sac_actor_pack_device(const float *w0, const float *b0, const float *w1,
                                            const float *b1, const float *w2, const float *b2,
                                            int hidden, void *packed, void *stream) {
    if (!w0 || !b0 || !w1 || !b1 || !w2 || !b2 || !packed || hidden < kMinHidden ||
        hidden > kMaxHidden || !aligned16(packed))
        return 0;
    PackArgs a;
    a.layout = packed_layout(hidden);
    const float *w[3] = {w0, w1, w2}, *b[3] = {b0, b1, b2};
    const int k[3] = {kFeatures, hidden, hidden}, n[3] = {hidden, hidden, kRaw};
    const int kc[3] = {kFeatureChunks, a.layout.ht, a.layout.ht};
    const int nt[3] = {a.layout.ht, a.layout.ht, 2};
    for (int l = 0; l < 3; ++l) {
        a.w[l] = w[l];
        a.b[l] = b[l];
        a.k[l] = k[l];
        a.n[l] = n[l];
        a.kc[l] = kc[l];
        a.nt[l] = nt[l];
    }
    a.out = static_cast<float *>(packed);
    (void)hipGetLastError();
    const size_t blocks = (a.layout.total + 255) / 256;
    sac_pack_kernel<<<(unsigned)blocks, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(a);
    return hipGetLastError() == hipSuccess;
}

extern "C" int tb_hip_sac_actor_act_device(const void *packed, int hidden, const float *features,
                                           const float *normals, float *actions,
                                           float *log_prob, float *raw, size_t batch_size,
                                           void *stream) {
    if (!packed || !features || !actions || hidden < kMinHidden || hidden > kMaxHidden ||
        !aligned16(packed) || batch_size == 0 || batch_size > kMaxBatch)
        return 0;
    const Packed p = packed_layout(hidden);
    ActArgs a;
    a.packed = static_cast<const float *>(packed);
    a.packed_bytes = (unsigned)(p.total * sizeof(float));
    for (int l = 0; l < 3; ++l) {
        a.w_off[l] = (unsigned)(p.w[l] * sizeof(float));
        a.b_off[l] = (unsigned)(p.b[l] * sizeof(float));
    }
    a.features = features;
    a.normals = normals;
    a.actions = actions;
    a.log_prob = log_prob;
    a.raw = raw;
    a.batch = batch_size;
    const size_t want = (batch_size + 63) / 64;
    const unsigned blocks = want > 65536 ? 65536u : (unsigned)want;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    (void)hipGetLastError();
    switch (p.ht) {
        case 1: launch_act<1>(a, blocks, s); break;
        case 2: launch_act<2>(a, blocks, s); break;
        case 3: launch_act<3>(a, blocks, s); break;
        case 4: launch_act<4>(a, blocks, s); break;
        case 5: launch_act<5>(a, blocks, s); break;
        case 6: launch_act<6>(a, blocks, s); break;
        case 7: launch_act<7>(a, blocks, s); break;
        case 8: launch_act<8>(a, blocks, s); break;
        case 9: launch_act<9>(a, blocks, s); break;
        case 10: launch_act<10>(a, blocks, s); break;
        case 11: launch_act<11>(a, blocks, s); break;
        case 12: launch_act<12>(a, blocks, s); break;
        case 13: launch_act<13>(a, blocks, s); break;
        case 14: launch_act<14>(a, blocks, s); break;
        case 15: launch_act<15>(a, blocks, s); break;
        default: launch_act<16>(a, blocks, s); break;
    }
    return hipGetLastError() == hipSuccess;
}
