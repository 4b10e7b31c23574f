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
// fp32 in and out) as transposed products  H^T = W * X^T  over groups of 16
// environments: the weights are the A operand and the environments the
// columns of B.  With that orientation the 16x16 output fragment a lane
// holds (outputs 16t+4g..16t+4g+3 of environment lane%16, g = lane/16) is
// exactly the B-operand fragment of input chunk t of the next layer.  A
// workgroup's four waves split every layer's output tiles between them and
// pass the finished tiles to each other through LDS in that fragment layout.
//
// Weights are first packed (tb_hip_sac_actor_pack_device) into that operand
// order: for output tile nt, input chunk s (16 inputs) and lane l, one float4
// holds W[16nt + l%16][16s + 4(l/16) + 0..3], so every weight load of a wave
// is one contiguous 1 KiB read.  Padding rows / columns hold zeros.  The
// last layer's rows are interleaved (mean, log-std, mean, ...), so a lane's
// output fragment holds two whole actions and the sampling runs on it in
// registers.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "turbinator/training/hip_features.h"
#include "xcd_order.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kFeatures = 142;
constexpr int kActions = 15;
constexpr int kRaw = 2 * kActions;
constexpr int kFeatureChunks = 9;  // 142 inputs padded to 144
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

// The hidden -> 30 layer's outputs are packed interleaved: packed row p holds
// the reference's output p / 2 (a mean) for even p and 15 + p / 2 (its
// log-std) for odd p, so the four outputs a lane holds are the (mean,
// log-std) pairs of two consecutive actions.
__host__ __device__ inline int raw_row(int p) { return (p & 1) ? kActions + (p >> 1) : (p >> 1); }

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
                if (n < a.n[l] && k < a.k[l])
                    v = a.w[l][(size_t)(l == 2 ? raw_row(n) : n) * a.k[l] + k];
            } else if (i >= a.layout.b[l] && i < a.layout.b[l] + (size_t)a.nt[l] * 16) {
                const int e = (int)(i - a.layout.b[l]);
                if (e < a.n[l]) v = a.b[l][l == 2 ? raw_row(e) : e];
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

// A workgroup's four waves share two groups of 16 environments: in the
// 142 -> hidden and hidden -> hidden layers wave w computes output tiles
// w, w + 4, w + 8, ... for both groups; in the hidden -> 30 layer (two tiles
// per group) wave w computes tile w % 2 of group w / 2.  The finished tiles
// go through LDS to all four waves as the next layer's input fragments.  A
// 16,384-row batch is 512 workgroups, two per CU, so every SIMD holds two
// waves with the same matrix-core work.
constexpr int kWaves = 4;
constexpr int kGroups = 2;  // groups of 16 environments per workgroup pass

// This wave's tiles nt = w + 4j (j < TPW, nt < NT) of one dense layer over
// KC input chunks, for the workgroup's G groups of 16 environments:
// out tile = W[tile] * in^T + b.  The layer's input rows are in LDS (`rows`,
// S floats per environment): lane l reads the B-operand fragment of chunk s,
// inputs 16s + 4g .. +3 of environment l % 16 of each group, as one float4.
// Every weight fragment a wave loads feeds 4 G matrix-core steps, one per
// group, so L2 delivers 1 KiB of weights per 4 G MFMAs.  Weight chunks
// stream through a ring of kDepth register slots: the chunk of step
// s + kDepth - 1 is requested while step s runs.  The loop has no branches:
// a slot j past the layer's tiles (when NT is not a multiple of 4) reads its
// weights and bias at an offset past the buffer end, which the buffer
// resource returns as zeros, computes a zero tile and is never stored.  The
// scheduling barrier keeps the compiler from hoisting every load of the
// layer.  The per-tile accumulation order (chunk s outer, k-step t inner)
// does not depend on how tiles or environments are spread over waves.
constexpr int kDepth = 4;
constexpr unsigned kPastEnd = 0x80000000u;  // lane offset beyond any packed buffer

// The first kDepth - 1 weight chunks and the bias of this wave's tiles of one
// layer, requested ahead of the layer (layer_prefetch) so that their round
// trip overlaps the previous phase of the pass.
template <int TPW>
struct LayerWeights {
    f32x4 ring[kDepth][TPW];
    f32x4 bias[TPW];
};

// Lane offsets of this wave's tile slots: a slot past the layer's NT tiles
// reads at kPastEnd (zeros through the buffer resource).
template <int NT, int TPW>
__device__ __forceinline__ void tile_slots(int w, int lane, unsigned (&wl)[TPW],
                                           unsigned (&bl)[TPW], int (&nt)[TPW]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        nt[j] = w + kWaves * j;
        const bool valid = nt[j] < NT;
        wl[j] = valid ? 16u * lane : kPastEnd;
        bl[j] = valid ? 16u * (lane >> 4) : kPastEnd;
        if (!valid) nt[j] = 0;
    }
}

template <int KC, int NT, int TPW>
__device__ __forceinline__ void layer_prefetch(__amdgpu_buffer_rsrc_t rsrc, unsigned w_off,
                                               unsigned b_off, int w, int lane,
                                               LayerWeights<TPW> &lw) {
    unsigned wl[TPW], bl[TPW];
    int nt[TPW];
    tile_slots<NT, TPW>(w, lane, wl, bl, nt);
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        lw.bias[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, bl[j], b_off + 64u * nt[j], 0);
#pragma unroll
        for (int d = 0; d < kDepth - 1; ++d)
            if (d < KC)
                lw.ring[d][j] = __builtin_amdgcn_raw_buffer_load_b128(
                    rsrc, wl[j], w_off + 1024u * (nt[j] * KC + d), 0);
    }
}

template <int KC, int NT, int TPW, int G, bool TANH, int S>
__device__ __forceinline__ void layer_tiles(__amdgpu_buffer_rsrc_t rsrc, unsigned w_off,
                                            const f32x4 *rows, LayerWeights<TPW> &lw,
                                            f32x4 (&out)[TPW][G], int w, int lane) {
    const int g = lane >> 4;
    const f32x4 *in = rows + ((lane & 15) * S) / 4 + g;  // group q, chunk s: in[q 4S + 4 s]
    unsigned wl[TPW], bl[TPW];
    int nt[TPW];
    tile_slots<NT, TPW>(w, lane, wl, bl, nt);
    f32x4 acc[TPW][G];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int q = 0; q < G; ++q) acc[j][q] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 xc[G], xn[G];
#pragma unroll
    for (int q = 0; q < G; ++q) xn[q] = xc[q] = in[q * 4 * S];
#pragma unroll
    for (int s = 0; s < KC; ++s) {
        if (s + kDepth - 1 < KC) {
#pragma unroll
            for (int j = 0; j < TPW; ++j)
                lw.ring[(s + kDepth - 1) % kDepth][j] = __builtin_amdgcn_raw_buffer_load_b128(
                    rsrc, wl[j], w_off + 1024u * (nt[j] * KC + s + kDepth - 1), 0);
        }
        if (s + 1 < KC) {
#pragma unroll
            for (int q = 0; q < G; ++q) xn[q] = in[q * 4 * S + 4 * (s + 1)];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int j = 0; j < TPW; ++j)
#pragma unroll
                for (int q = 0; q < G; ++q)
                    acc[j][q] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        lw.ring[s % kDepth][j][t], xc[q][t], acc[j][q], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < G; ++q) xc[q] = xn[q];
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int q = 0; q < G; ++q)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float y = acc[j][q][v] + lw.bias[j][v];
                out[j][q][v] = TANH ? tanh_hidden(y) : y;
            }
}

__device__ __forceinline__ float finite_or_zero(float x) {  // training.c:61-63
    return __builtin_isfinite(x) ? x : 0.0f;
}
__device__ __forceinline__ float clampf(float x, float lo, float hi) {  // training.c:57-59
    return x < lo ? lo : (x > hi ? hi : x);
}

// Writes this wave's hidden tiles into the workgroup's activation rows: lane
// l holds outputs 16nt + 4g .. +3 of environment l % 16 of each group, which
// is exactly the B-operand fragment of input chunk nt of the next layer.
template <int TPW, int G, int NT, int S>
__device__ __forceinline__ void store_tiles(f32x4 *rows, const f32x4 (&h)[TPW][G], int w,
                                            int lane) {
    const int g = lane >> 4, e = lane & 15;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        const int nt = w + kWaves * j;
        if (nt < NT) {
#pragma unroll
            for (int q = 0; q < G; ++q) rows[((16 * q + e) * S) / 4 + 4 * nt + g] = h[j][q];
        }
    }
}

template <int HT, int G>
__global__ __launch_bounds__(kWaves * 64) void sac_actor_kernel(ActArgs a) {
    constexpr int TPW = (HT + kWaves - 1) / kWaves;  // hidden tiles per wave
    static_assert(kWaves == 2 * G, "the hidden -> 30 layer gives each wave one (tile, group)");
    constexpr int E = 16 * G;                        // environments per workgroup pass
    // Row stride of the workgroup's LDS rows (floats): the 144 padded
    // features or the padded hidden activations, plus 4 so rows start on
    // different banks.  Buffer 1 holds the features during layer 0 and the
    // second hidden layer afterwards; buffer 0 the first hidden layer.
    constexpr int S = (16 * HT > 16 * kFeatureChunks ? 16 * HT : 16 * kFeatureChunks) + 4;
    __shared__ f32x4 buf[2][E * S / 4];
    __shared__ float term_s[E][16];
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, j = lane & 15;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.packed, a.packed_bytes);
    // The loop bound is uniform over the block, so every wave meets the
    // barriers; rows past the batch end compute on zeros and store nothing.
    // Groups go to workgroups in XCD-contiguous order, the order in which the
    // feature kernel writes its rows, so that behind it a workgroup reads
    // rows its own XCD wrote (14.9 -> 14.5 us at 16,384 rows).
    for (size_t base = xcd_contiguous(blockIdx.x, gridDim.x) * E; base < a.batch;
         base += (size_t)gridDim.x * E) {
        // Stage the feature rows in buffer 1 (rows are 568 bytes, 8-byte
        // aligned): every 8-byte load of the pass is issued before any LDS
        // store, so the rows arrive in one round trip.  Rows past the batch
        // end read as zero; inputs 142 and 143 are zero padding.
        constexpr int kPairs = E * 72;  // 72 float pairs per padded row
        constexpr int kPerThread = (kPairs + kWaves * 64 - 1) / (kWaves * 64);
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        f32x2 pairs[kPerThread];
        {
            const size_t rows = a.batch - base < (size_t)E ? a.batch - base : (size_t)E;
            const __amdgpu_buffer_rsrc_t frs =
                make_rsrc(a.features + base * kFeatures, (unsigned)(rows * kFeatures * 4));
#pragma unroll
            for (int it = 0; it < kPerThread; ++it) {
                const int q = tid + kWaves * 64 * it;
                const int e = q / 72, k = 2 * (q - 72 * e);
                pairs[it] = (f32x2){0.0f, 0.0f};
                if (q < kPairs && k < kFeatures)
                    pairs[it] = __builtin_bit_cast(
                        f32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                   frs, (unsigned)(e * kFeatures + k) * 4, 0, 0));
            }
        }
        // Layer 0's first weight chunks and bias, requested with the
        // features so that both round trips overlap.
        LayerWeights<TPW> lw0;
        layer_prefetch<kFeatureChunks, HT, TPW>(wrs, a.w_off[0], a.b_off[0], w, lane, lw0);
        // The hidden -> 30 layer gives wave w tile w % 2 of group w / 2:
        // lane (g, j) then holds the (mean, log-std) pairs of actions
        // 8 (w % 2) + 2 g and + 1 of environment j of that group.  Their
        // normal draws are loaded now and used after the three layers.
        const int tile2 = w & 1, group2 = w >> 1;
        const size_t env2 = base + 16 * group2 + j;
        float drawn[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int act = 8 * tile2 + 2 * g + h;
            drawn[h] = 0.0f;
            if (a.normals && act < kActions && env2 < a.batch)
                drawn[h] = a.normals[env2 * kActions + act];
        }
        {
            float *xs = reinterpret_cast<float *>(buf[1]);
#pragma unroll
            for (int it = 0; it < kPerThread; ++it) {
                const int q = tid + kWaves * 64 * it;
                const int e = q / 72, k = 2 * (q - 72 * e);
                if (q < kPairs) {
                    xs[e * S + k] = pairs[it][0];
                    xs[e * S + k + 1] = pairs[it][1];
                }
            }
        }
        __syncthreads();

        // Each layer's first weight chunks are requested before the
        // barrier that ends the previous layer.
        LayerWeights<TPW> lw1;
        {
            f32x4 h[TPW][G];
            layer_tiles<kFeatureChunks, HT, TPW, G, true, S>(wrs, a.w_off[0], buf[1], lw0, h, w,
                                                             lane);
            layer_prefetch<HT, HT, TPW>(wrs, a.w_off[1], a.b_off[1], w, lane, lw1);
            store_tiles<TPW, G, HT, S>(buf[0], h, w, lane);
        }
        __syncthreads();
        LayerWeights<1> lw2;
        {
            f32x4 h[TPW][G];
            layer_tiles<HT, HT, TPW, G, true, S>(wrs, a.w_off[1], buf[0], lw1, h, w, lane);
            layer_prefetch<HT, 2, 1>(wrs, a.w_off[2], a.b_off[2], tile2, lane, lw2);
            store_tiles<TPW, G, HT, S>(buf[1], h, w, lane);
        }
        __syncthreads();
        {
            f32x4 r[1][1];
            layer_tiles<HT, 2, 1, 1, false, S>(wrs, a.w_off[2], buf[1] + group2 * 4 * S, lw2, r,
                                               tile2, lane);
            // training.c:310-327 on this lane's two actions (the last lane
            // group of tile 1 holds one action and the padding).
            const bool live = env2 < a.batch;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int act_i = 8 * tile2 + 2 * g + h;
                if (act_i >= kActions) continue;
                const float mean_raw = r[0][0][2 * h], ls_raw = r[0][0][2 * h + 1];
                if (a.raw && live) {
                    a.raw[env2 * kRaw + act_i] = mean_raw;
                    a.raw[env2 * kRaw + kActions + act_i] = ls_raw;
                }
                const float log_std = clampf(finite_or_zero(ls_raw), -3.5f, -1.6f);
                const float sd = expf(log_std);
                const float eps = a.normals ? drawn[h] * (act_i == 14 ? 0.15f : 1.0f) : 0.0f;
                const float z = clampf(finite_or_zero(mean_raw) + sd * eps, -8.0f, 8.0f);
                const float act = tanhf(z);
                if (live) a.actions[env2 * kActions + act_i] = act;
                const float gaussian = -0.5f * eps * eps - log_std - 0.5f * logf(2.0f * kPi);
                term_s[16 * group2 + j][act_i] = gaussian - logf(1.0f - act * act + 1.0e-6f);
            }
        }
        __syncthreads();
        if (a.log_prob && tid < E && base + tid < a.batch) {
            float lp = 0.0f;  // summed in action order, as the reference does
            if (a.normals)
                for (int i = 0; i < kActions; ++i) lp += term_s[tid][i];
            a.log_prob[base + tid] = lp;
        }
    }
}

template <int HT>
void launch_act(const ActArgs &a, unsigned blocks, hipStream_t s) {
    sac_actor_kernel<HT, kGroups><<<blocks, kWaves * 64, 0, s>>>(a);
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
    const size_t want = (batch_size + 16 * kGroups - 1) / (16 * kGroups);
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
