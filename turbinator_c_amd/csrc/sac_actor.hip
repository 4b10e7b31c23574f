// Batched compact SAC actor on gfx950: tb_sac_act_features
// (src/training/training.c:382-392) for a whole batch of feature rows in one
// launch, so the 142-value features never leave HBM.
//
//   tb_net_forward   training.c:219-233  142 -> hidden (tanh) -> hidden (tanh)
//                                        -> 30 (15 means, 15 raw log-std)
//   tb_actor_sample  training.c:306-329  clamped log-std, tanh-squashed
//                                        Gaussian action, log-probability
//
// The three dense layers run on the fp16 matrix cores
// (v_mfma_f32_16x16x32_f16) with each fp32 operand split into two fp16
// pieces, x = hi + lo + err:  hi = fp16(x), lo = fp16(x - hi), both rounded
// to nearest even.  The subtraction is exact (Sterbenz), so while lo is a
// normal fp16, |err| <= 2^-22 |x|.  A product is summed as the three cross
// terms hi·hi, hi·lo and lo·hi: the dropped lo·lo and the two operands'
// errors come to at most 3·2^-22 |w x| (about 7e-7), and each cross product
// of two fp16 values is exact.  The instruction's block sum is not the
// correctly rounded sum, though: the bits of a product that lie more than
// 2^-24 below the largest product of its group of eight are dropped before
// the sum is rounded (tests/csrc/check_mfma_sum.hip; over 262,144 random
// outputs the error is at most 3.8 u sum|p|, 0.4 u on average, u = 2^-24).
// A layer's error is therefore a small multiple of u sum|w x|, the form of
// the reference's sequential fp32 sum too, and a hidden unit whose summands
// cancel passes it on to the outputs as the reference's does.  Three fp16
// steps take 3/16 of the fp32 matrix-core time of the same product.  (The
// two-piece fp16 split with three products is the scheme of Ootomo and
// Yokota, "Recovering single precision accuracy from Tensor Cores while
// surpassing the FP32 theoretical peak performance", IJHPCA 36(4), 2022;
// the range handling below is this kernel's.)
//
// Range.  fp16 is normal from 2^-14 to 65504, so every operand row is
// scaled by a power of two that brings its largest magnitude into
// [2^14, 2^15): each weight row when it is packed, each environment's
// features while they are staged, and the hidden activations (tanh, at
// most 1) by 2^14.  A piece more than 2^28 below its row's largest
// magnitude is an fp16 subnormal, whose rounding (at most 2^-25 at that
// scale) is up to 2^-39 of the row's largest magnitude, and no more than the
// operand.  That error follows the row's largest magnitude, not the
// product: where a row's largest weight meets a zero feature and a weight
// 2^30 below it meets a large one, it reaches about 1e-3 of the sum.  So a
// sum's error is a few u sum|w x| plus sum_k |x_k| min(|w_k|, 2^-39 max|w|)
// + |w_k| min(|x_k|, 2^-39 max|x|) (max|x| = 1 for hidden activations).
// The sums are unscaled with ldexp before the bias is added (exact: powers
// of two).
//
// The products are transposed, H^T = W * X^T, over groups of 16
// environments: the weights are the A operand and the environments the
// columns of B.  The 16x16 output fragment a lane holds (outputs
// 16t+4g..16t+4g+3 of environment lane%16, g = lane/16) is split and written
// to LDS as the next layer's B operand: a 32-input chunk c holds hidden
// tiles 2c and 2c+1, position 8g + 4h + v of the chunk being output
// 16(2c+h) + 4g + v, so a lane's four outputs of tile 2c+h land in its own
// 8-byte slot.  A workgroup's eight waves split every layer's output tiles
// between them and pass the finished tiles to each other through LDS.
//
// Weights are first packed (tb_hip_sac_actor_pack_device) into that operand
// order: for output tile nt, input chunk c, piece p and lane l, one 16-byte
// vector holds the piece of the scaled W[16nt + l%16][k] for the eight
// chunk positions 8(l/16) .. +7, so every weight load of a wave is one
// contiguous 1 KiB read; each tile's biases and unscale exponents follow
// its layer.  Padding rows / columns hold zeros.  The last layer's rows are
// interleaved (mean, log-std, mean, ...), so a lane's output fragment holds
// two whole actions and the sampling runs on it in registers.
//
// Infinite features have no split (their pieces would multiply zeros into
// NaN).  Such a feature is zeroed in the split operand and its product
// x * W[n][k] is added in fp32 by the lanes of its environment, from an
// fp32 copy of the first layer's weights kept in the packed buffer, which
// gives the reference's +-inf (or NaN where the reference's sum is NaN).
// NaN inputs need nothing: both pieces of a NaN are NaN.  Weights have no
// such path: a non-finite weight makes its row's output NaN for every
// environment, where the reference's would be +-inf or NaN.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "turbinator/training/hip_features.h"
#include "xcd_order.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kFeatures = 142;
constexpr int kActions = 15;
constexpr int kRaw = 2 * kActions;
constexpr int kFeatureChunks = 5;  // 142 inputs padded to 160 = 5 chunks of 32
constexpr int kPieces = 2;         // hi, lo
constexpr int kChunkBytes = 64;    // one piece of one 32-input chunk (32 fp16)
constexpr int kBlockBytes = kPieces * 1024;  // one (tile, chunk) of a packed layer
constexpr int kTileScaleBytes = 128;          // per tile: 16 fp32 biases, 16 int exponents
constexpr int kHiddenScale = 14;              // tanh outputs enter a layer times 2^14
constexpr int kMinHidden = 16, kMaxHidden = 256;
constexpr float kPi = 3.14159265358979323846f;
constexpr size_t kMaxBatch = 0x7fffffffu;

// Byte offsets of the packed sections; every section starts on 256 bytes.
struct Packed {
    int ht, hc;             // hidden tiles (16 outputs), hidden chunks (32 inputs)
    size_t w[3], b[3];      // weight pieces; fp32 biases and unscale exponents
    size_t w0;              // fp32 copy of the first layer's weights, [hidden][142]
    size_t total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline Packed packed_layout(int hidden) {
    Packed p;
    p.ht = (hidden + 15) / 16;
    p.hc = (p.ht + 1) / 2;
    const int kc[3] = {kFeatureChunks, p.hc, p.hc};
    const int nt[3] = {p.ht, p.ht, 2};
    size_t off = 0;
    for (int l = 0; l < 3; ++l) {
        p.w[l] = off;
        off = align256(off + (size_t)nt[l] * kc[l] * kBlockBytes);
        p.b[l] = off;
        off = align256(off + (size_t)nt[l] * kTileScaleBytes);
    }
    p.w0 = off;
    off = align256(off + (size_t)hidden * kFeatures * sizeof(float));
    p.total = off;
    return p;
}

// The hidden -> 30 layer's outputs are packed interleaved: packed row p holds
// the reference's output p / 2 (a mean) for even p and 15 + p / 2 (its
// log-std) for odd p, so the four outputs a lane holds are the (mean,
// log-std) pairs of two consecutive actions.
__host__ __device__ inline int raw_row(int p) { return (p & 1) ? kActions + (p >> 1) : (p >> 1); }

// The layer input that chunk c, position s (0..31) of layer `layer` carries:
// the features in order for the first layer; for the hidden layers the
// position order of the tile exchange (position 8g + 4h + v of chunk c is
// output 16(2c + h) + 4g + v of the previous layer).
__host__ __device__ inline int chunk_input(int layer, int c, int s) {
    if (layer == 0) return 32 * c + s;
    const int g = s >> 3, i = s & 7;
    return 16 * (2 * c + (i >> 2)) + 4 * g + (i & 3);
}

__device__ __forceinline__ bool infinite(float x) {
    return (__float_as_uint(x) & 0x7fffffffu) == 0x7f800000u;
}

// The exponent t that brings a row whose largest magnitude has the bits
// `max_bits` to [2^14, 2^15): 2^14 <= |max| 2^t < 2^15 for a normal max
// (all zero or subnormal rows get t = 141; a NaN max gives -114, and the
// row is NaN anyway).
__host__ __device__ inline int row_exponent(unsigned max_bits) {
    return 141 - (int)(max_bits >> 23);
}

// The split of two scaled values (|x| < 2^15), as packed fp16 pairs per
// piece.
__device__ __forceinline__ void split_pair(f32x2 x, unsigned &hi, unsigned &lo) {
    const f16x2 h = __builtin_convertvector(x, f16x2);
    const f32x2 hf = __builtin_convertvector(h, f32x2);
    const f32x2 r = {x[0] - hf[0], x[1] - hf[1]};
    hi = __builtin_bit_cast(unsigned, h);
    lo = __builtin_bit_cast(unsigned, __builtin_convertvector(r, f16x2));
}

struct PackArgs {
    const float *w[3], *b[3];
    int k[3], n[3], kc[3], nt[3];
    int hidden;
    Packed layout;
    unsigned *out;  // the packed buffer as 32-bit words
};

// The scale exponent of packed row n of layer l: the row's weights times
// 2^s lie below 2^15 in magnitude.
__device__ int row_scale(const PackArgs &a, int l, int n) {
    if (n >= a.n[l]) return 0;
    const float *row = a.w[l] + (size_t)(l == 2 ? raw_row(n) : n) * a.k[l];
    unsigned m = 0;
    for (int k = 0; k < a.k[l]; ++k) {
        const unsigned b = __float_as_uint(row[k]) & 0x7fffffffu;
        m = b > m ? b : m;
    }
    return row_exponent(m);
}

// The packed weight piece pair at byte offset `e` of layer l's weight
// section: two fp16 values of one piece, chunk positions i0 and i0 + 1.
__device__ unsigned packed_weight_pair(const PackArgs &a, int l, size_t e) {
    const size_t block = e / kBlockBytes;
    const int within = (int)(e % kBlockBytes);
    const int piece = within / 1024, lane = (within % 1024) / 16, i0 = (within % 16) / 2;
    const int tile = (int)(block / a.kc[l]), c = (int)(block % a.kc[l]);
    const int n = 16 * tile + (lane & 15);
    const int scale = row_scale(a, l, n);
    f32x2 v = {0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int k = chunk_input(l, c, 8 * (lane >> 4) + i0 + h);
        if (n < a.n[l] && k < a.k[l])
            v[h] = __builtin_amdgcn_ldexpf(
                a.w[l][(size_t)(l == 2 ? raw_row(n) : n) * a.k[l] + k], scale);
    }
    unsigned p[kPieces];
    split_pair(v, p[0], p[1]);
    return p[piece];
}

// One thread per packed 32-bit word.
__global__ __launch_bounds__(256) void sac_pack_kernel(PackArgs a) {
    const size_t words = a.layout.total / 4;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t byte = 4 * i;
        unsigned v = 0;
        for (int l = 0; l < 3; ++l) {
            const size_t wsize = (size_t)a.nt[l] * a.kc[l] * kBlockBytes;
            if (byte >= a.layout.w[l] && byte < a.layout.w[l] + wsize) {
                v = packed_weight_pair(a, l, byte - a.layout.w[l]);
            } else if (byte >= a.layout.b[l] &&
                       byte < a.layout.b[l] + (size_t)a.nt[l] * kTileScaleBytes) {
                // Tile block: biases of rows 16 t .. +15, then the exponents
                // that undo the row scale (and the hidden inputs' 2^14).
                const int e = (int)((byte - a.layout.b[l]) / 4);
                const int n = 16 * (e / 32) + (e % 16);
                if (n < a.n[l]) {
                    if (e % 32 < 16)
                        v = __float_as_uint(a.b[l][l == 2 ? raw_row(n) : n]);
                    else
                        v = (unsigned)(-row_scale(a, l, n) - (l == 0 ? 0 : kHiddenScale));
                }
            }
        }
        if (byte >= a.layout.w0 && byte < a.layout.w0 + (size_t)a.hidden * kFeatures * 4)
            v = __float_as_uint(a.w[0][(byte - a.layout.w0) / 4]);
        a.out[i] = v;
    }
}

struct ActArgs {
    const void *packed;
    unsigned packed_bytes;
    unsigned w_off[3], b_off[3], w0_off;  // section offsets in bytes
    int hidden;
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
// Returned times 2^14, the scale at which hidden activations enter the
// next layer (the same rounding: a power of two commutes with it).
__device__ __forceinline__ float tanh_hidden_scaled(float x) {
    const float e = __builtin_amdgcn_exp2f(x * 2.88539008177792681f);  // 2 / ln 2
    return __builtin_fmaf(-32768.0f, __builtin_amdgcn_rcpf(e + 1.0f), 16384.0f);
}

// A workgroup's NW waves share NW / 2 groups of 16 environments: in the
// 142 -> hidden and hidden -> hidden layers wave w computes output tiles
// w, w + NW, ... for all groups; in the hidden -> 30 layer (two tiles per
// group) wave w computes tile w % 2 of group w / 2.  The finished tiles go
// through LDS to all the waves as the next layer's input fragments.  Above
// 4 hidden tiles NW = 8: a 16,384-row batch is 256 workgroups, one per CU,
// every SIMD holds two waves with the same matrix-core work, and a CU reads
// each weight once (NW = 4, two workgroups per CU, reads each weight twice
// per CU: 9.4 against 9.1 us at hidden 128; four groups on four waves, one
// wave per SIMD: 11.7 us).  Up to 4 hidden tiles NW = 4, so that waves do
// not compute empty tiles (hidden 16: 6.4 against 7.3 us).
template <int HT>
struct Shape {
    static constexpr int waves = HT <= 4 ? 4 : 8;
    static constexpr int groups = waves / 2;  // groups of 16 environments per workgroup pass
};

// LDS rows of the workgroup: one per environment, KC chunks of 128 bytes
// (the hi and lo pieces of 32 inputs, 64 bytes each), plus 16 bytes so that
// the rows of a 16-byte read start on different banks.
__host__ __device__ constexpr int row_bytes(int kc) { return kc * kPieces * kChunkBytes + 16; }

// This wave's tiles nt = w + NW j (j < TPW, nt < NT) of one dense layer over
// KC input chunks, for the workgroup's G groups of 16 environments:
// out tile = W[tile] * in^T + b.  Lane l reads the B-operand fragment of
// chunk s, pieces of positions 8g .. +7 of environment l % 16 of each group,
// as two 16-byte LDS reads.  Every weight fragment a wave loads feeds
// 3 G matrix-core steps, so L2 delivers 2 KiB of weights per 3 G MFMAs.
// Weight chunks stream through a ring of ring_depth register slots: the
// chunk of step s + D - 1 is requested while step s runs.  The loop has no
// branches: a slot j past the layer's tiles (when NT is not a multiple of
// NW) reads its weights and bias at an offset past the buffer end, which the
// buffer resource returns as zeros, computes a zero tile and is never
// stored except as the zero padding tile.  The scheduling barrier keeps the
// compiler from hoisting every load of the layer.  The per-tile
// accumulation order (chunk s outer, cross term inner) does not depend on
// how tiles or environments are spread over waves.
constexpr unsigned kPastEnd = 0x80000000u;  // lane offset beyond any packed buffer

template <int TPW>
constexpr int ring_depth() { return TPW <= 2 ? 4 : 2; }

// The first weight chunks and the bias of this wave's tiles of one layer,
// requested ahead of the layer (layer_prefetch) so that their round trip
// overlaps the previous phase of the pass.
template <int TPW>
struct LayerWeights {
    u32x4 ring[ring_depth<TPW>()][TPW][kPieces];
    f32x4 bias[TPW];
    i32x4 unscale[TPW];
};

// Lane offsets of this wave's tile slots: a slot past the layer's NT tiles
// reads at kPastEnd (zeros through the buffer resource).
template <int NT, int TPW, int NW>
__device__ __forceinline__ void tile_slots(int w, int lane, unsigned (&wl)[TPW],
                                           unsigned (&bl)[TPW], int (&nt)[TPW]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        nt[j] = w + NW * j;
        const bool valid = nt[j] < NT;
        wl[j] = valid ? 16u * lane : kPastEnd;
        bl[j] = valid ? 16u * (lane >> 4) : kPastEnd;  // + 64 for the exponents
        if (!valid) nt[j] = 0;
    }
}

template <int KC, int TPW>
__device__ __forceinline__ void load_chunk(__amdgpu_buffer_rsrc_t rsrc, unsigned w_off,
                                           const unsigned (&wl)[TPW], const int (&nt)[TPW],
                                           int s, u32x4 (&slot)[TPW][kPieces]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int p = 0; p < kPieces; ++p)
            slot[j][p] = __builtin_amdgcn_raw_buffer_load_b128(
                rsrc, wl[j], w_off + kBlockBytes * (nt[j] * KC + s) + 1024u * p, 0);
}

template <int KC, int NT, int TPW, int NW>
__device__ __forceinline__ void layer_prefetch(__amdgpu_buffer_rsrc_t rsrc, unsigned w_off,
                                               unsigned b_off, int w, int lane,
                                               LayerWeights<TPW> &lw) {
    constexpr int D = ring_depth<TPW>();
    unsigned wl[TPW], bl[TPW];
    int nt[TPW];
    tile_slots<NT, TPW, NW>(w, lane, wl, bl, nt);
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        lw.bias[j] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, bl[j],
                                                         b_off + kTileScaleBytes * nt[j], 0));
        lw.unscale[j] = __builtin_bit_cast(
            i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rsrc, bl[j], b_off + kTileScaleBytes * nt[j] + 64u, 0));
    }
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
        if (d < KC) load_chunk<KC, TPW>(rsrc, w_off, wl, nt, d, lw.ring[d]);
}

__device__ __forceinline__ f32x4 mfma_f16(u32x4 w, u32x4 x, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, w),
                                                  __builtin_bit_cast(f16x8, x), acc, 0, 0, 0);
}

// The three cross terms, small ones first: (weight piece, input piece).
constexpr int kTerms = 3;
constexpr int kTermW[kTerms] = {1, 0, 0};
constexpr int kTermX[kTerms] = {0, 1, 0};

// Returns W * in^T + b for this wave's tiles (no activation): the scaled
// sums times 2^(row exponent - shift[q]), plus the bias.  `rows` are the
// layer's input rows in LDS, RS bytes apart; shift[q] is the scale exponent
// of group q's inputs beyond the one the packed exponents already undo.
template <int KC, int NT, int TPW, int G, int RS, int NW>
__device__ __forceinline__ void layer_tiles(__amdgpu_buffer_rsrc_t rsrc, unsigned w_off,
                                            const u32x4 *rows, LayerWeights<TPW> &lw,
                                            const int (&shift)[G], f32x4 (&out)[TPW][G], int w,
                                            int lane) {
    constexpr int D = ring_depth<TPW>();
    constexpr int RS16 = RS / 16;
    const int g = lane >> 4;
    const u32x4 *in = rows + (lane & 15) * RS16 + g;  // group q, chunk s, piece p:
                                                      // in[16 q RS16 + 8 s + 4 p]
    unsigned wl[TPW], bl[TPW];
    int nt[TPW];
    tile_slots<NT, TPW, NW>(w, lane, wl, bl, nt);
    f32x4 acc[TPW][G];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int q = 0; q < G; ++q) acc[j][q] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 xc[G][kPieces], xn[G][kPieces];
#pragma unroll
    for (int q = 0; q < G; ++q)
#pragma unroll
        for (int p = 0; p < kPieces; ++p) xn[q][p] = xc[q][p] = in[16 * q * RS16 + 4 * p];
#pragma unroll
    for (int s = 0; s < KC; ++s) {
        if (s + D - 1 < KC) load_chunk<KC, TPW>(rsrc, w_off, wl, nt, s + D - 1,
                                                lw.ring[(s + D - 1) % D]);
        if (s + 1 < KC) {
#pragma unroll
            for (int q = 0; q < G; ++q)
#pragma unroll
                for (int p = 0; p < kPieces; ++p)
                    xn[q][p] = in[16 * q * RS16 + 8 * (s + 1) + 4 * p];
        }
#pragma unroll
        for (int t = 0; t < kTerms; ++t)
#pragma unroll
            for (int j = 0; j < TPW; ++j)
#pragma unroll
                for (int q = 0; q < G; ++q)
                    acc[j][q] = mfma_f16(lw.ring[s % D][j][kTermW[t]], xc[q][kTermX[t]],
                                         acc[j][q]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < G; ++q)
#pragma unroll
            for (int p = 0; p < kPieces; ++p) xc[q][p] = xn[q][p];
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int q = 0; q < G; ++q)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                out[j][q][v] = __builtin_amdgcn_ldexpf(acc[j][q][v], lw.unscale[j][v] - shift[q]) +
                               lw.bias[j][v];
}

__device__ __forceinline__ float finite_or_zero(float x) {  // training.c:61-63
    return __builtin_isfinite(x) ? x : 0.0f;
}
__device__ __forceinline__ float clampf(float x, float lo, float hi) {  // training.c:57-59
    return x < lo ? lo : (x > hi ? hi : x);
}

// Writes this wave's hidden tiles, after tanh, into the workgroup's
// activation rows as split pieces: lane l's outputs 16nt + 4g .. +3 of
// environment l % 16 go to chunk nt / 2, positions 8g + 4(nt % 2) .. +3.
// NH is the number of tiles the next layer reads (the hidden tiles rounded
// up to whole chunks): a slot past the hidden tiles computed a zero tile,
// whose tanh is zero, and writes the padding.
template <int TPW, int G, int NH, int RS, int NW>
__device__ __forceinline__ void store_tiles(unsigned char *rows, f32x4 (&h)[TPW][G], int w,
                                            int lane) {
    const int g = lane >> 4, e = lane & 15;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        const int nt = w + NW * j;
        if (nt < NH) {
#pragma unroll
            for (int q = 0; q < G; ++q) {
                u32x2 pc[kPieces];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const f32x2 x = {tanh_hidden_scaled(h[j][q][2 * hh]),
                                     tanh_hidden_scaled(h[j][q][2 * hh + 1])};
                    unsigned hi, lo;
                    split_pair(x, hi, lo);
                    pc[0][hh] = hi;
                    pc[1][hh] = lo;
                }
                unsigned char *base = rows + (16 * q + e) * RS + (nt >> 1) * kPieces * kChunkBytes +
                                      16 * g + 8 * (nt & 1);
#pragma unroll
                for (int p = 0; p < kPieces; ++p)
                    *reinterpret_cast<u32x2 *>(base + kChunkBytes * p) = pc[p];
            }
        }
    }
}

template <int HT, int G, int NW>
__global__ __launch_bounds__(NW * 64) void sac_actor_kernel(ActArgs a) {
    constexpr int TPW = (HT + NW - 1) / NW;  // hidden tiles per wave
    constexpr int HC = (HT + 1) / 2;                 // hidden chunks of 32 inputs
    // The hidden -> 30 layer's 2 G (tile, group) pairs, G2 groups per wave.
    static_assert(2 * G % NW == 0, "whole groups per wave in the hidden -> 30 layer");
    constexpr int G2 = 2 * G / NW;
    constexpr int E = 16 * G;                        // environments per workgroup pass
    // Buffer 1 holds the features during layer 0 and the second hidden layer
    // afterwards; buffer 0 the first hidden layer.
    constexpr int RS = row_bytes(kFeatureChunks > HC ? kFeatureChunks : HC);
    __shared__ u32x4 buf[2][E * RS / 16];
    __shared__ float term_s[E][16];
    // Per environment of the pass: nonzero when its feature row holds an
    // infinity, and the largest magnitude of its other features (as bits),
    // both written while staging and read by layer 0.
    __shared__ int special[E];
    __shared__ unsigned row_max[E];
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, j = lane & 15;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.packed, a.packed_bytes);

    // The loop bound is uniform over the block, so every wave meets the
    // barriers; rows past the batch end compute on zeros and store nothing.
    // Groups go to workgroups in XCD-contiguous order, the order in which the
    // feature kernel writes its rows, so that behind it a workgroup reads
    // rows its own XCD wrote.
    for (size_t base = xcd_contiguous(blockIdx.x, gridDim.x) * E; base < a.batch;
         base += (size_t)gridDim.x * E) {
        // Stage the feature rows in buffer 1 (rows are 568 bytes, 8-byte
        // aligned): kRowThreads consecutive threads share an environment,
        // each loading kRowPairs consecutive float pairs, every load of the
        // pass issued before any LDS store so that the rows arrive in one
        // round trip.  Rows past the batch end read as zero; inputs 142 to
        // 159 are zero padding.
        constexpr int kRowThreads = NW * 64 / E;                 // 8
        constexpr int kRowPairs = 16 * kFeatureChunks / kRowThreads;  // 10
        static_assert(kRowThreads * kRowPairs == 16 * kFeatureChunks, "row split");
        const int se = tid / kRowThreads, sr = tid % kRowThreads;
        f32x2 pairs[kRowPairs];
        {
            const size_t rows = a.batch - base < (size_t)E ? a.batch - base : (size_t)E;
            const __amdgpu_buffer_rsrc_t frs =
                make_rsrc(a.features + base * kFeatures, (unsigned)(rows * kFeatures * 4));
#pragma unroll
            for (int it = 0; it < kRowPairs; ++it) {
                const int k = 2 * (kRowPairs * sr + it);
                pairs[it] = (f32x2){0.0f, 0.0f};
                if (k < kFeatures)
                    pairs[it] = __builtin_bit_cast(
                        f32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                   frs, (unsigned)(se * kFeatures + k) * 4, 0, 0));
            }
        }
        // Layer 0's first weight chunks and bias, requested with the
        // features so that both round trips overlap.
        LayerWeights<TPW> lw0;
        layer_prefetch<kFeatureChunks, HT, TPW, NW>(wrs, a.w_off[0], a.b_off[0], w, lane, lw0);
        // The hidden -> 30 layer gives wave w tile w % 2 of the G2 groups
        // from group2 = G2 (w / 2) on: lane (g, j) then holds the (mean,
        // log-std) pairs of actions 8 (w % 2) + 2 g and + 1 of environment j
        // of each.  Their normal draws are loaded now and used after the
        // three layers.
        const int tile2 = w & 1, group2 = G2 * (w >> 1);
        float drawn[G2][2];
#pragma unroll
        for (int i = 0; i < G2; ++i) {
            const size_t env2 = base + 16 * (group2 + i) + j;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int act = 8 * tile2 + 2 * g + h;
                drawn[i][h] = 0.0f;
                if (a.normals && act < kActions && env2 < a.batch)
                    drawn[i][h] = a.normals[env2 * kActions + act];
            }
        }
        // Infinite features go to the exact path (zero in the split operand);
        // the row's largest other magnitude sets its scale.  The row's
        // threads are kRowThreads consecutive lanes: both reduce by xor
        // shuffles, and the first thread records them for layer 0.
        {
            unsigned m = 0;
            int inf = 0;
#pragma unroll
            for (int it = 0; it < kRowPairs; ++it) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    if (infinite(pairs[it][h])) {
                        pairs[it][h] = 0.0f;
                        inf = 1;
                    }
                    const unsigned b = __float_as_uint(pairs[it][h]) & 0x7fffffffu;
                    m = b > m ? b : m;
                }
            }
#pragma unroll
            for (int d = 1; d < kRowThreads; d <<= 1) {
                const unsigned o = (unsigned)__shfl_xor((int)m, d);
                m = o > m ? o : m;
                inf |= __shfl_xor(inf, d);
            }
            if (sr == 0) {
                row_max[se] = m;
                special[se] = inf;
            }
            const int t = row_exponent(m);
            unsigned char *xs = reinterpret_cast<unsigned char *>(buf[1]);
#pragma unroll
            for (int it = 0; it < kRowPairs; ++it) {
                const int k = 2 * (kRowPairs * sr + it);
                const f32x2 x = {__builtin_amdgcn_ldexpf(pairs[it][0], t),
                                 __builtin_amdgcn_ldexpf(pairs[it][1], t)};
                unsigned pc[kPieces];
                split_pair(x, pc[0], pc[1]);
                unsigned char *at = xs + se * RS + (k >> 5) * kPieces * kChunkBytes + 2 * (k & 31);
#pragma unroll
                for (int p = 0; p < kPieces; ++p)
                    *reinterpret_cast<unsigned *>(at + kChunkBytes * p) = pc[p];
            }
        }
        __syncthreads();

        // Each layer's first weight chunks are requested before the
        // barrier that ends the previous layer.
        LayerWeights<TPW> lw1;
        {
            f32x4 h[TPW][G];
            int shift[G];
#pragma unroll
            for (int q = 0; q < G; ++q) shift[q] = row_exponent(row_max[16 * q + j]);
            layer_tiles<kFeatureChunks, HT, TPW, G, RS, NW>(wrs, a.w_off[0], buf[1], lw0, shift, h,
                                                            w, lane);
            // The exact products of the infinite features, added by the
            // lanes of their environment (rare).
            bool mine[G];
            bool any = false;
#pragma unroll
            for (int q = 0; q < G; ++q) {
                mine[q] = special[16 * q + j] != 0;
                any |= mine[q];
            }
            if (__builtin_amdgcn_ballot_w64(any)) {
                const float *w0 = reinterpret_cast<const float *>(
                    static_cast<const unsigned char *>(a.packed) + a.w0_off);
#pragma unroll
                for (int q = 0; q < G; ++q) {
                    if (!mine[q]) continue;
                    const float *row = a.features + (base + 16 * q + j) * kFeatures;
                    for (int k = 0; k < kFeatures; ++k) {
                        const float x = row[k];
                        if (!infinite(x)) continue;
#pragma unroll
                        for (int jj = 0; jj < TPW; ++jj)
#pragma unroll
                            for (int v = 0; v < 4; ++v) {
                                const int n = 16 * (w + NW * jj) + 4 * g + v;
                                if (n < a.hidden) h[jj][q][v] += x * w0[(size_t)n * kFeatures + k];
                            }
                    }
                }
            }
            layer_prefetch<HC, HT, TPW, NW>(wrs, a.w_off[1], a.b_off[1], w, lane, lw1);
            store_tiles<TPW, G, 2 * HC, RS, NW>(reinterpret_cast<unsigned char *>(buf[0]), h, w,
                                                lane);
        }
        __syncthreads();
        LayerWeights<1> lw2;
        {
            f32x4 h[TPW][G];
            int shift[G] = {};
            layer_tiles<HC, HT, TPW, G, RS, NW>(wrs, a.w_off[1], buf[0], lw1, shift, h, w, lane);
            layer_prefetch<HC, 2, 1, NW>(wrs, a.w_off[2], a.b_off[2], tile2, lane, lw2);
            store_tiles<TPW, G, 2 * HC, RS, NW>(reinterpret_cast<unsigned char *>(buf[1]), h, w,
                                                lane);
        }
        __syncthreads();
        {
            f32x4 r[1][G2];
            const int shift[G2] = {};
            layer_tiles<HC, 2, 1, G2, RS, NW>(wrs, a.w_off[2], buf[1] + group2 * 16 * (RS / 16), lw2,
                                          shift, r, tile2, lane);
            // training.c:310-327 on this lane's two actions of each group
            // (the last lane group of tile 1 holds one action and the
            // padding).
#pragma unroll
            for (int i = 0; i < G2; ++i) {
                const size_t env2 = base + 16 * (group2 + i) + j;
                const bool live = env2 < a.batch;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int act_i = 8 * tile2 + 2 * g + h;
                    if (act_i >= kActions) continue;
                    const float mean_raw = r[0][i][2 * h], ls_raw = r[0][i][2 * h + 1];
                    if (a.raw && live) {
                        a.raw[env2 * kRaw + act_i] = mean_raw;
                        a.raw[env2 * kRaw + kActions + act_i] = ls_raw;
                    }
                    const float log_std = clampf(finite_or_zero(ls_raw), -3.5f, -1.6f);
                    const float sd = expf(log_std);
                    const float eps =
                        a.normals ? drawn[i][h] * (act_i == 14 ? 0.15f : 1.0f) : 0.0f;
                    const float z = clampf(finite_or_zero(mean_raw) + sd * eps, -8.0f, 8.0f);
                    const float act = tanhf(z);
                    if (live) a.actions[env2 * kActions + act_i] = act;
                    const float gaussian = -0.5f * eps * eps - log_std - 0.5f * logf(2.0f * kPi);
                    term_s[16 * (group2 + i) + j][act_i] =
                        gaussian - logf(1.0f - act * act + 1.0e-6f);
                }
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
void launch_act(const ActArgs &a, hipStream_t s) {
    constexpr int NW = Shape<HT>::waves, G = Shape<HT>::groups;
    const size_t want = (a.batch + 16 * G - 1) / (16 * G);
    const unsigned blocks = want > 65536 ? 65536u : (unsigned)want;
    sac_actor_kernel<HT, G, NW><<<blocks, NW * 64, 0, s>>>(a);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" size_t tb_hip_sac_actor_packed_bytes(int hidden) {
    if (hidden < kMinHidden || hidden > kMaxHidden) return 0;
    return packed_layout(hidden).total;
}

extern "C" int tb_hip_sac_actor_pack_device(const float *w0, const float *b0, const float *w1,
                                            const float *b1, const float *w2, const float *b2,
                                            int hidden, void *packed, void *stream) {
    if (!w0 || !b0 || !w1 || !b1 || !w2 || !b2 || !packed || hidden < kMinHidden ||
        hidden > kMaxHidden || !aligned16(packed))
        return 0;
    PackArgs a;
    a.layout = packed_layout(hidden);
    a.hidden = hidden;
    const float *w[3] = {w0, w1, w2}, *b[3] = {b0, b1, b2};
    const int k[3] = {kFeatures, hidden, hidden}, n[3] = {hidden, hidden, kRaw};
    const int kc[3] = {kFeatureChunks, a.layout.hc, a.layout.hc};
    const int nt[3] = {a.layout.ht, a.layout.ht, 2};
    for (int l = 0; l < 3; ++l) {
        a.w[l] = w[l];
        a.b[l] = b[l];
        a.k[l] = k[l];
        a.n[l] = n[l];
        a.kc[l] = kc[l];
        a.nt[l] = nt[l];
    }
    a.out = static_cast<unsigned *>(packed);
    (void)hipGetLastError();
    const size_t blocks = (a.layout.total / 4 + 255) / 256;
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
    a.packed = packed;
    a.packed_bytes = (unsigned)p.total;
    for (int l = 0; l < 3; ++l) {
        a.w_off[l] = (unsigned)p.w[l];
        a.b_off[l] = (unsigned)p.b[l];
    }
    a.w0_off = (unsigned)p.w0;
    a.hidden = hidden;
    a.features = features;
    a.normals = normals;
    a.actions = actions;
    a.log_prob = log_prob;
    a.raw = raw;
    a.batch = batch_size;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    (void)hipGetLastError();
    switch (p.ht) {
        case 1: launch_act<1>(a, s); break;
        case 2: launch_act<2>(a, s); break;
        case 3: launch_act<3>(a, s); break;
        case 4: launch_act<4>(a, s); break;
        case 5: launch_act<5>(a, s); break;
        case 6: launch_act<6>(a, s); break;
        case 7: launch_act<7>(a, s); break;
        case 8: launch_act<8>(a, s); break;
        case 9: launch_act<9>(a, s); break;
        case 10: launch_act<10>(a, s); break;
        case 11: launch_act<11>(a, s); break;
        case 12: launch_act<12>(a, s); break;
        case 13: launch_act<13>(a, s); break;
        case 14: launch_act<14>(a, s); break;
        case 15: launch_act<15>(a, s); break;
        default: launch_act<16>(a, s); break;
    }
    return hipGetLastError() == hipSuccess;
}
