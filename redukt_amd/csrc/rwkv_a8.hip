// rwkv_a8.hip — the W8A8 tier of the RWKV-7 token step: the reference's own int8
// arithmetic (src/domain/tensor.rs:105-143, 1791-1866: every quantized projection takes
// its input vector to int8 with one scale, sums exact int32 products and rescales once per
// row), with everything else in the reference's operation order, sums included
// (src/infrastructure/rwkv7/model.rs:643-925), so a stream's logits are the CPU path's
// bit for bit.
//
// Per layer, in stream order (one graph):
//   k_shift_a8<6>  ln1 LayerNorm (sequential sums), token shift: x_r, x_k, x_v as int8
//                  (+ scale), x_w, x_a, x_g, x_v as f32 for the LoRAs
//   k_proj_a8      receptance, key, value (v_mfma_i32_16x16x64_i8 on the int8 weight
//                  tiles); first LoRA stages w1 (tanh), a1, g1 (sigmoid), v1 in the lane
//                  order of dot_avx2_order (tensor.rs:1676-1693)
//   k_proj_a8      second LoRA stages w2, a2, g2, v2
//   k_wkv_a8       one wave per (head, stream): decay, a, l2-normalised key, modified key,
//                  value mix, WKV-7, GroupNorm, bonus (sequential sums), gate; the gated
//                  vector as f32 with each head's largest magnitude
//   k_proj_a8      output projection + residual, quantizing the gated vector as it loads it
//   k_shift_a8<1>  ln2 + channel-mix token shift -> int8
//   k_proj_a8      FFN key, squared ReLU (f32)
//   k_quant_a8     those activations -> int8
//   k_proj_a8      FFN value + residual
// then k_shift_a8<0> (ln_out -> int8), k_head_a8 and optionally the softmax.
//
// A vector that one workgroup produces whole (the LayerNorm outputs) is quantized there.  The
// gated vector comes from one wave per head: it is written as f32 with each head's largest
// magnitude, and every workgroup of the output projection takes the stream's scale from
// those maxima (exact: a maximum does not depend on the order) and rounds the values it
// loads.  The FFN activations (d_ffn long, from many workgroups) are rounded once by a pass
// of their own, since the FFN value product would round them again in every row tile.
//
// The reference-order tier (F32 weights, profile bit 6) runs the same element-wise kernels
// with every projection an F32 GEMV in the reference's dot_avx2_order (mat_vec_mul_into,
// tensor.rs:1602-1693; exact_gemv_launch, eight lanes per output; receptance, key and value
// in one launch): k_shift_a8 hands all six
// token-shift inputs over as f32, and the receptance, key, value, output, FFN and head
// products replace the int8 ones (the FFN key's squared ReLU in its epilogue), so the
// logits are the CPU path's F32 logits bit for bit.
//
// Integer products are exact, so the k-order of the int8 matrix products is free: the
// weight tiles of the int8 matrix-core tiers serve unchanged (the 16 bytes a lane holds for
// k-pair p are row r's columns 64p + 8g + [0, 8) and 64p + 32 + 8g + [0, 8), g = lane / 16)
// and the activation operand is loaded with the same column map.  Every output element
// depends on its own stream only.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <utility>

#include "mfma_common.h"
#include "model.h"
#include "portable_math.h"
#include "rwkv_common.h"
#include "step.h"

#pragma clang fp contract(off)

namespace rdk {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;
constexpr int kPer = 4;                    // LayerNorm channels per thread: d <= 1024
constexpr int kMaxD = kBlock * kPer;
constexpr int kMix = 6;
constexpr int kSegs = 8;
constexpr int kHead = 64;
constexpr int kWaves = kBlock / kWave;
constexpr int kWavePairs = 12;                   // int8 products: k-pairs a wave requests at once
constexpr int kWavePairsF = 4;                   // the same with f32 activations (16 floats a pair)
constexpr int kLoraBatch = 48;                   // LoRA steps whose loads are requested at once
constexpr int kHeadMaxPairs = kMaxD / 64;
constexpr int kHeadTiles = 2;                    // head: row tiles per wave
constexpr int kHeadRowPad = 32;                  // head: LDS row padding of the staged activations (bytes)

// ---------------------------------------------------------------- int8 activations

// quantize_vec_i8_into (tensor.rs:1791-1800): scale = amax / 127 (1 without a nonzero
// magnitude; NaNs never raise amax), q = round(v * (1 / scale)) with Rust's round (half
// away from zero, as roundf), clamped to +-127 (a NaN passes the clamp) and converted by
// the saturating `as i8` (NaN -> 0).
__device__ __forceinline__ float q8_scale(float amax) { return amax > 0.0f ? amax / 127.0f : 1.0f; }

__device__ __forceinline__ int8_t q8_of(float v, float inv) {
    float t = roundf(v * inv);
    if (t < -127.0f) t = -127.0f;
    if (t > 127.0f) t = 127.0f;
    return t != t ? (int8_t)0 : (int8_t)(int)t;
}

// |v| folded into a running maximum the way the reference folds it (`if a > max`): a NaN
// never enters, and the maximum of the rest does not depend on the order.
__device__ __forceinline__ float fold_abs(float m, float v) {
    const float a = fabsf(v);
    return a > m ? a : m;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float t = __shfl_xor(v, o, kWave);
        v = t > v ? t : v;
    }
    return v;
}

// Iterator::sum over f32, as the reference's layer_norm_into, group_norm_into,
// l2_normalize_per_head_inplace and bonus take it (tensor.rs:1390-1424, model.rs:899-909):
// ((0 + sh[0]) + sh[1]) + ..., each partial sum rounded in turn.  Every lane walks the whole
// row (broadcast LDS reads, each block of 32 requested while the previous one is added), so
// every lane ends with the sum.
__device__ __forceinline__ void add32(float& s, const float4 (&v)[8]) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        s += v[j].x;
        s += v[j].y;
        s += v[j].z;
        s += v[j].w;
    }
}

__device__ __forceinline__ void load32(float4 (&v)[8], const float* p) {
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = *(const float4*)(p + 4 * j);
}

__device__ __forceinline__ float seq_sum(const float* sh, int n) {
    float s = 0.0f;
    // Pairs of 32-element blocks through two buffers: the next block is requested before the
    // current one is added (the last request re-reads a block, unused).
    const int n64 = n / 64 * 64;
    float4 a[8], b[8];
    if (n64 > 0) load32(a, sh);
    for (int i = 0; i < n64; i += 64) {
        load32(b, sh + i + 32);
        add32(s, a);
        load32(a, sh + min(i + 64, n64 - 32));
        add32(s, b);
    }
    int i = n64;
    if (i + 32 <= n) {
        load32(a, sh + i);
        add32(s, a);
        i += 32;
    }
    for (; i < n; i++) s += sh[i];
    return s;
}

// Two such sums over two rows of 64, walked together (independent chains).
__device__ __forceinline__ void seq_sum2_64(const float* a, const float* b, float& sa, float& sb) {
    float s = 0.0f, t = 0.0f;
#pragma unroll
    for (int i = 0; i < kHead; i += 4) {
        const float4 u = *(const float4*)(a + i);
        const float4 w = *(const float4*)(b + i);
        s += u.x; t += w.x; s += u.y; t += w.y; s += u.z; t += w.z; s += u.w; t += w.w;
    }
    sa = s;
    sb = t;
}

// ---------------------------------------------------------------- LayerNorm + token shift

struct ShiftA8Args {
    const float* x;              // [n][d]
    const float* ln_w;
    const float* ln_b;
    float* prev;                 // slot s's previous ln output at prev + s * prev_stride (NMIX > 0)
    size_t prev_stride;
    const uint32_t* slots;
    uint32_t cap;                // state slots of the pool (the clamp bound)
    const float* mix[kMix];
    float* outf[kMix];           // output m as f32 [n][d] (null: not wanted)
    int8_t* outq[kMix];          // output m as int8 [rows16][dp] (null: not wanted)
    float* outs[kMix];           // the int8 output's scale per stream
    int d, dp;
};

// layer_norm_into (tensor.rs:1390-1398) with both sums sequential: mean = sum(x) / d,
// var = sum((x - mean)^2) / d, ln = (x - mean) * (1 / sqrt(var + 1e-5)) * w + b; then the
// token shift of time_mixing_scratch (model.rs:811-820) / channel_mixing_scratch
// (:920-921): input_m = ln + (prev - ln) * mix_m, and the slot's prev becomes ln.  NMIX = 0:
// the ln output itself is output 0.  One workgroup per stream.
template <int NMIX>
__global__ __launch_bounds__(kBlock) void k_shift_a8(ShiftA8Args a) {
    __shared__ __align__(16) float row[kMaxD];
    __shared__ float wmax[kMix][kBlock / kWave];
    constexpr int kOut = NMIX ? NMIX : 1;
    const uint32_t b = blockIdx.x;
    const int d = a.d;
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const uint32_t slot = NMIX ? clamp_slot(a.slots[b], a.cap) : 0u;
    int cc[kPer];
    bool in[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int c = (int)threadIdx.x + kBlock * q;
        in[q] = c < d;
        cc[q] = c < d ? c : d - 1;
    }
    float xv[kPer], wv[kPer], bv[kPer], mv[kOut][kPer], pv[kPer];
    const float* xb = a.x + (size_t)b * d;
    float* const pp = NMIX ? a.prev + slot * a.prev_stride : nullptr;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        xv[q] = xb[cc[q]];
        wv[q] = a.ln_w[cc[q]];
        bv[q] = a.ln_b[cc[q]];
        pv[q] = NMIX ? pp[cc[q]] : 0.0f;
    }
#pragma unroll
    for (int m = 0; m < NMIX; m++)
#pragma unroll
        for (int q = 0; q < kPer; q++) mv[m][q] = a.mix[m][cc[q]];
#pragma unroll
    for (int q = 0; q < kPer; q++)
        if (in[q]) row[cc[q]] = xv[q];
    __syncthreads();
    const float mean = seq_sum(row, d) / (float)d;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPer; q++)
        if (in[q]) row[cc[q]] = (xv[q] - mean) * (xv[q] - mean);
    __syncthreads();
    const float inv = 1.0f / sqrtf(seq_sum(row, d) / (float)d + 1e-5f);
    float val[kOut][kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const float ln = (xv[q] - mean) * inv * wv[q] + bv[q];
        if (NMIX == 0) {
            val[0][q] = ln;
            continue;
        }
        const float xx = pv[q] - ln;
#pragma unroll
        for (int m = 0; m < NMIX; m++) val[m][q] = ln + xx * mv[m][q];
        if (in[q]) pp[cc[q]] = ln;
    }
#pragma unroll
    for (int m = 0; m < kOut; m++) {
        if (a.outf[m] != nullptr) {
#pragma unroll
            for (int q = 0; q < kPer; q++)
                if (in[q]) a.outf[m][(size_t)b * d + cc[q]] = val[m][q];
        }
        if (a.outq[m] != nullptr) {
            float mx = 0.0f;
#pragma unroll
            for (int q = 0; q < kPer; q++)
                if (in[q]) mx = fold_abs(mx, val[m][q]);
            mx = wave_max(mx);
            if (lane == 0) wmax[m][wave] = mx;
        }
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < kOut; m++) {
        if (a.outq[m] == nullptr) continue;
        float amax = 0.0f;
#pragma unroll
        for (int w = 0; w < kBlock / kWave; w++) amax = wmax[m][w] > amax ? wmax[m][w] : amax;
        const float scale = q8_scale(amax);
        const float qinv = 1.0f / scale;
#pragma unroll
        for (int q = 0; q < kPer; q++)
            if (in[q]) a.outq[m][(size_t)b * a.dp + cc[q]] = q8_of(val[m][q], qinv);
        if (threadIdx.x == 0) a.outs[m][b] = scale;
    }
}

const void* shift_a8_fn(int nmix) {
    if (nmix == 6) return (const void*)k_shift_a8<6>;
    if (nmix == 1) return (const void*)k_shift_a8<1>;
    return (const void*)k_shift_a8<0>;
}

// ---------------------------------------------------------------- projections

enum { SEG_A8 = 0, SEG_LORA = 1 };
enum { MODE_STORE = 0, MODE_RESID = 1 };

struct SegA8 {
    int kind, mode, act;
    TMat w;                  // SEG_A8: per-row int8 weight tiles
    const int8_t* q;         // SEG_A8: int8 activations, stream b at q + b * kp, scales qs
    const float* qs;
    int kp;
    const float* qf;         // or f32 activations, stream b at qf + b * kp (q null), with the
    const float* pmax;       // largest magnitude of each of their `nparts` pieces at pmax + b * nparts
    int nparts;
    int wpt;                 // SEG_A8: waves per tile (1, 2 or 4), each a contiguous share of the k-pairs
    LMat l;                  // SEG_LORA
    const float* xf;         // SEG_LORA: f32 activations, stream b at xf + b * ldx
    int ldx;
    float* out;              // row r of stream b at out[b * ld + r]
    int ld;
    uint32_t blk0;           // first workgroup of this segment
};

struct ProjA8Args {
    SegA8 seg[kSegs];
    int nseg;
    uint32_t n, groups;
};

__device__ __forceinline__ i32x4 mma8(const int4& w, const int2& lo, const int2& hi, const i32x4& c) {
    const i32x4 a = {w.x, w.y, w.z, w.w};
    const i32x4 v = {lo.x, lo.y, hi.x, hi.y};
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, v, c, 0, 0, 0);
}

// acc += the products of k-pairs [p0, p1) of one tile (weights at A, the lane's int8
// activations at qb), requested kWavePairs at a time before the first product.
__device__ __forceinline__ i32x4 a8_pairs(const int4* A, const int8_t* qb, int p0, int p1, i32x4 acc) {
    for (int c = p0; c < p1; c += kWavePairs) {
        int4 w[kWavePairs];
        int2 lo[kWavePairs], hi[kWavePairs];
#pragma unroll
        for (int j = 0; j < kWavePairs; j++) {
            const int p = c + j;
            if (p < p1) {
                w[j] = A[(size_t)p * 64];
                lo[j] = *(const int2*)(qb + 64 * p);
                hi[j] = *(const int2*)(qb + 64 * p + 32);
            }
        }
#pragma unroll
        for (int j = 0; j < kWavePairs; j++)
            if (c + j < p1) acc = mma8(w[j], lo[j], hi[j], acc);
    }
    return acc;
}

__device__ __forceinline__ int pack4(float a, float b, float c, float d, float inv) {
    return (int)((uint32_t)(uint8_t)q8_of(a, inv) | (uint32_t)(uint8_t)q8_of(b, inv) << 8 |
                 (uint32_t)(uint8_t)q8_of(c, inv) << 16 | (uint32_t)(uint8_t)q8_of(d, inv) << 24);
}

// The same from f32 activations at fb, each rounded to int8 with the stream's 1 / scale as
// it arrives (quantize_vec_i8_into's rule).
__device__ __forceinline__ i32x4 a8_pairs_f(const int4* A, const float* fb, float inv, int p0, int p1, i32x4 acc) {
    for (int c = p0; c < p1; c += kWavePairsF) {
        int4 w[kWavePairsF];
        float4 v[kWavePairsF][4];
#pragma unroll
        for (int j = 0; j < kWavePairsF; j++) {
            const int p = c + j;
            if (p < p1) {
                w[j] = A[(size_t)p * 64];
                v[j][0] = *(const float4*)(fb + 64 * p);
                v[j][1] = *(const float4*)(fb + 64 * p + 4);
                v[j][2] = *(const float4*)(fb + 64 * p + 32);
                v[j][3] = *(const float4*)(fb + 64 * p + 36);
            }
        }
#pragma unroll
        for (int j = 0; j < kWavePairsF; j++) {
            if (c + j >= p1) continue;
            int2 lo, hi;
            lo.x = pack4(v[j][0].x, v[j][0].y, v[j][0].z, v[j][0].w, inv);
            lo.y = pack4(v[j][1].x, v[j][1].y, v[j][1].z, v[j][1].w, inv);
            hi.x = pack4(v[j][2].x, v[j][2].y, v[j][2].z, v[j][2].w, inv);
            hi.y = pack4(v[j][3].x, v[j][3].y, v[j][3].z, v[j][3].w, inv);
            acc = mma8(w[j], lo, hi, acc);
        }
    }
    return acc;
}

// The scale of stream b's f32 activations: q8_scale of the largest of its pieces' maxima.
// The four lanes of the stream (kg = 0..3) each take a quarter of the pieces, then meet.
__device__ __forceinline__ float pieces_scale(const float* pmax, int nparts, uint32_t b, int kg) {
    const float* pm = pmax + (size_t)b * nparts;
    float m = 0.0f;
    for (int i = kg; i < nparts; i += 4) m = pm[i] > m ? pm[i] : m;
    float t = __shfl_xor(m, 16, kWave);
    m = t > m ? t : m;
    t = __shfl_xor(m, 32, kWave);
    m = t > m ? t : m;
    return q8_scale(m);
}

// q8_mat_vec_mul_into (tensor.rs:1819-1866) for one 16-row tile x 16 streams: `wpt` waves
// take contiguous shares of the k-pairs, their int32 partial sums meet in LDS (exact, so in
// any order), and wave 0 of the tile writes out = (float)acc * (scale_row * scale_stream).
__device__ __forceinline__ void a8_tile(const SegA8& s, int t, int part, uint32_t g, uint32_t n,
                                        i32x4 (*red)[kWave]) {
    const int lane = threadIdx.x % kWave, kg = lane / 16, wave = wave_index();
    const uint32_t b = g * kRowTile + lane % 16;          // < rows16: the activation rows exist
    const int np = s.w.ks / 2;
    const bool live = t < s.w.rt;
    const float sb = s.q != nullptr ? (b < n ? s.qs[b] : 1.0f) : pieces_scale(s.pmax, s.nparts, b, kg);
    // The epilogue's operands are requested with the products' (they do not depend on them).
    const int r0 = min(t, s.w.rt - 1) * kRowTile + kg * 4;
    float sw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sw[i] = s.w.scales[r0 + i];
    float* o = s.out + (size_t)b * s.ld + r0;
    const bool vec = r0 + 3 < s.w.rows && ((s.ld | r0) & 3) == 0 && ((uintptr_t)s.out & 15) == 0;
    f32x4 y = {0, 0, 0, 0};
    if (live && part == 0 && vec && b < n && s.mode == MODE_RESID) y = *(f32x4*)o;
    i32x4 acc = {0, 0, 0, 0};
    if (live) {
        const int share = (np + s.wpt - 1) / s.wpt;
        const int p0 = part * share, p1 = min(np, p0 + share);
        const int4* A = (const int4*)s.w.w + (size_t)t * np * 64 + lane;
        if (s.q != nullptr) acc = a8_pairs(A, s.q + (size_t)b * s.kp + 8 * kg, p0, p1, acc);
        else acc = a8_pairs_f(A, s.qf + (size_t)b * s.kp + 8 * kg, 1.0f / sb, p0, p1, acc);
    }
    if (s.wpt > 1) {
        if (part > 0) red[wave][lane] = acc;
        __syncthreads();
        if (part > 0) return;
        for (int j = 1; j < s.wpt; j++) acc += red[wave + j][lane];
    }
    if (!live || b >= n) return;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = activate(s.act, (float)acc[i] * (sw[i] * sb), 0, 0);
    if (vec) {
#pragma unroll
        for (int i = 0; i < 4; i++) y[i] = s.mode == MODE_RESID ? y[i] + v[i] : v[i];
        *(f32x4*)o = y;
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (r0 + i >= s.w.rows) continue;
        o[i] = s.mode == MODE_RESID ? o[i] + v[i] : v[i];
    }
}

// mat_vec_mul_into over f32 (tensor.rs:1602-1693, dot_avx2_order) for rows of one stream:
// chain l of a row accumulates the columns c = l (mod 8) from +0 with one multiply and one
// add each; then hsum_f32_scalar ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) (each
// pairing one commutative add, so every lane that forms it gets the same bits) and the
// activation of the LoRA stage.  Long rows (the first stages, K = d) take a lane per chain
// (eight rows a wave, kLoraBatch steps requested at once); short rows (the second stages,
// K = rank) take two lanes, chains 4h .. 4h + 3 on lane h, with 16-byte loads (32 rows a
// wave, every step requested at once).
template <int LPR>
__device__ __forceinline__ void lora_rows(const SegA8& s, int rb, uint32_t b) {
    constexpr int kRowsPerWave = kWave / LPR, kCh = 8 / LPR;
    const int lane = threadIdx.x % kWave, h = lane % LPR;
    const int r = rb * (kWaves * kRowsPerWave) + wave_index() * kRowsPerWave + lane / LPR;
    const int rr = r < s.l.rows8 ? r : s.l.rows8 - 1;
    const int steps = s.l.cols / 8;
    const size_t wstep = (size_t)s.l.rows8 * 8;
    const float* w = s.l.w + (size_t)rr * 8 + kCh * h;
    const float* x = s.xf + (size_t)b * s.ldx + kCh * h;
    float acc[kCh];
#pragma unroll
    for (int j = 0; j < kCh; j++) acc[j] = 0.0f;
    if (LPR == 8) {
        int i = 0;
        for (; i + kLoraBatch <= steps; i += kLoraBatch) {
            float wv[kLoraBatch], xv[kLoraBatch];
#pragma unroll
            for (int u = 0; u < kLoraBatch; u++) {
                wv[u] = w[(i + u) * wstep];
                xv[u] = x[8 * (i + u)];
            }
#pragma unroll
            for (int u = 0; u < kLoraBatch; u++) acc[0] += wv[u] * xv[u];
        }
        for (; i < steps; i++) acc[0] += w[i * wstep] * x[8 * i];
    } else {
        constexpr int kB = kLoraBatch / 4;
        for (int i0 = 0; i0 < steps; i0 += kB) {
            float4 wv[kB], xv[kB];
#pragma unroll
            for (int u = 0; u < kB; u++) {
                const int i = i0 + u;
                if (i < steps) {
                    wv[u] = *(const float4*)(w + i * wstep);
                    xv[u] = *(const float4*)(x + 8 * i);
                }
            }
#pragma unroll
            for (int u = 0; u < kB; u++) {
                if (i0 + u < steps) {
                    acc[0] += wv[u].x * xv[u].x;
                    acc[1] += wv[u].y * xv[u].y;
                    acc[2] += wv[u].z * xv[u].z;
                    acc[3] += wv[u].w * xv[u].w;
                }
            }
        }
    }
    // complete in lane h = 0 of the row, the lane that stores
    float sum;
    if (LPR == 8) {
        sum = hsum8_lane0(acc[0]);
    } else {
        float s4[4];
#pragma unroll
        for (int j = 0; j < 4; j++) s4[j] = acc[j] + dpp_move<kDppQuadXor1>(acc[j]);
        sum = (s4[0] + s4[2]) + (s4[1] + s4[3]);
    }
    if (h == 0 && r < s.l.rows) s.out[(size_t)b * s.ld + r] = activate(s.act, sum, r, s.l.rows);
}

// Lanes per row of a LoRA segment with `cols` columns.
constexpr int lora_lpr(int cols) { return cols >= 256 ? 8 : 2; }

__global__ __launch_bounds__(kBlock) void k_proj_a8(ProjA8Args a) {
    __shared__ i32x4 red[kWaves][kWave];
    int si = 0;
    for (int i = 1; i < a.nseg; i++)
        if (blockIdx.x >= a.seg[i].blk0) si = i;
    const SegA8& s = a.seg[si];
    const uint32_t local = blockIdx.x - s.blk0;
    if (s.kind == SEG_A8) {
        const int wave = wave_index(), tpb = kWaves / s.wpt;
        const int t = (int)(local / a.groups) * tpb + wave / s.wpt;
        a8_tile(s, t, wave % s.wpt, local % a.groups, a.n, red);
    } else if (lora_lpr(s.l.cols) == 8) {
        lora_rows<8>(s, (int)(local / a.n), local % a.n);
    } else {
        lora_rows<2>(s, (int)(local / a.n), local % a.n);
    }
}

// ---------------------------------------------------------------- WKV-7

struct WkvA8Args {
    const float* rkv;        // [n][3d]: r, k, v
    const float* lorad;      // [n][4d]: decay, a, g, v second LoRA stages
    const float *w0, *a0, *v0, *k_k, *k_a, *r_k, *ln_x_w, *ln_x_b;
    float* wkv;              // this layer's state of slot s at wkv + s * slot_stride
    size_t slot_stride;
    float* vfirst;           // [n][d]
    const uint32_t* slots;
    uint32_t cap;            // state slots of the pool (the clamp bound)
    float* gated;            // the gated vector, stream b at gated + b * ldg
    int ldg;
    float* gmax;             // the largest |gated| of head h at gmax + b * heads + h
    int heads, d, layer, g1k;
};

// time_mixing_scratch steps 3-12 after the projections (model.rs:827-912) for one head of
// one stream; lane i owns channel c = 64 h + i and row i of the head's state.  The sums over
// the head (l2 norm, GroupNorm mean and variance, bonus) are sequential; the state products
// t = S·(-kk) and out = S·r already run over j in order per lane.
__global__ __launch_bounds__(kHead) void k_wkv_a8(WkvA8Args a) {
    __shared__ __align__(16) float sw[kHead], skka[kHead], snegkk[kHead], skmod[kHead], sr[kHead];
    __shared__ __align__(16) float sa[kHead], sb[kHead];
    const int i = threadIdx.x, h = blockIdx.x;
    const uint32_t b = blockIdx.y;
    const int d = a.d, c = h * kHead + i;
    const uint32_t slot = clamp_slot(a.slots[b], a.cap);
    const float* rkv = a.rkv + (size_t)b * 3 * d;
    const float* ld = a.lorad + (size_t)b * 4 * d;
    const float r = rkv[c], k = rkv[d + c], v = rkv[2 * d + c];
    const float lw = ld[c], la = ld[d + c], g = ld[2 * d + c], lv = ld[3 * d + c];
    const float vf = a.layer != 0 ? a.vfirst[(size_t)b * d + c] : 0.0f;
    // The head's state is stored [j / 4][i][4]: lane i's float4 q holds S[i][4q .. 4q + 3].
    float4* sbase = (float4*)(a.wkv + slot * a.slot_stride + (size_t)h * kHead * kHead);
    float S[kHead];
#pragma unroll
    for (int q = 0; q < kHead / 4; q++) {
        const float4 t4 = sbase[q * kHead + i];
        S[4 * q] = t4.x; S[4 * q + 1] = t4.y; S[4 * q + 2] = t4.z; S[4 * q + 3] = t4.w;
    }
    // Step 3: exp(-0.606531 * sigmoid(w0 + lora)) (decay_sigmoid_into, tensor.rs:1082-1101)
    const float w = lane_exp_f(-0.606531f * lane_sigmoid_f(a.w0[c] + lw));
    // Step 4 (sigmoid_add_into :1040-1056)
    const float aa = lane_sigmoid_f(a.a0[c] + la);
    // Step 6: kk = (k * k_k) / sqrt(sum over the head of (k * k_k)^2), 0 when the norm is
    // <= 1e-12 (l2_normalize_per_head_inplace :1416-1424)
    const float kk0 = k * a.k_k[c];
    sa[i] = kk0 * kk0;
    __syncthreads();
    const float norm = sqrtf(seq_sum(sa, kHead));
    const float kk = kk0 * (norm > 1e-12f ? 1.0f / norm : 0.0f);
    // Step 7
    const float kmod = k * (1.0f + (aa - 1.0f) * a.k_a[c]);
    // Step 8: v_out, mixed towards the layer-0 value from the second layer on (:1128-1147)
    float vout = v;
    if (a.layer != 0) {
        const float mix = lane_sigmoid_f(a.v0[c] + lv);
        vout += (vf - vout) * mix;
    } else {
        a.vfirst[(size_t)b * d + c] = v;
    }
    // Step 9: t = S·(-kk); S[i][j] = S[i][j] w[j] + t[i] (kk a)[j] + v_out[i] kmod[j]; out = S·r
    sw[i] = w;
    skka[i] = kk * aa;
    snegkk[i] = -kk;
    skmod[i] = kmod;
    sr[i] = r;
    __syncthreads();
    float tt = 0.0f;
#pragma unroll
    for (int j = 0; j < kHead; j++) tt += S[j] * snegkk[j];
#pragma unroll
    for (int j = 0; j < kHead; j++) S[j] = S[j] * sw[j] + tt * skka[j] + vout * skmod[j];
    float o = 0.0f;
#pragma unroll
    for (int j = 0; j < kHead; j++) o += S[j] * sr[j];
#pragma unroll
    for (int q = 0; q < kHead / 4; q++) sbase[q * kHead + i] = make_float4(S[4 * q], S[4 * q + 1], S[4 * q + 2], S[4 * q + 3]);
    // Step 10: GroupNorm over the head, eps 64e-5 (group_norm_into :1400-1414); step 11:
    // bonus = sum over the head of r * k * r_k (k_mod for g1k models), times v_out
    const float ksrc = a.g1k ? kmod : k;
    sa[i] = o;
    sb[i] = r * ksrc * a.r_k[c];
    __syncthreads();
    float osum, bonus;
    seq_sum2_64(sa, sb, osum, bonus);
    const float mean = osum / (float)kHead;
    __syncthreads();
    sa[i] = (o - mean) * (o - mean);
    __syncthreads();
    const float var = seq_sum(sa, kHead) / (float)kHead;
    float on = (o - mean) * (1.0f / sqrtf(var + 64e-5f)) * a.ln_x_w[c] + a.ln_x_b[c];
    on += bonus * vout;
    // Step 12: gate; the output projection quantizes it
    const float gated = on * g;
    a.gated[(size_t)b * a.ldg + c] = gated;
    const float mx = wave_max(fold_abs(0.0f, gated));
    if (i == 0) a.gmax[(size_t)b * a.heads + h] = mx;
}

// ---------------------------------------------------------------- activations -> int8

struct QuantA8Args {
    const float* x;          // stream b at x + b * ld, K values (K a multiple of 4)
    int ld, K;
    int8_t* q;               // [rows16][kp]
    int kp;
    float* qs;
};

// quantize_vec_i8_into (tensor.rs:1791-1800) of one stream's FFN activations: the vector
// arrives from many workgroups of the FFN key product, so it is taken to int8 here, once,
// for every row tile of the FFN value product.
__global__ __launch_bounds__(kBlock) void k_quant_a8(QuantA8Args a) {
    __shared__ float wm[kWaves];
    const uint32_t b = blockIdx.x;
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const float4* xb = (const float4*)(a.x + (size_t)b * a.ld);
    const int k4 = a.K / 4;
    float mx = 0.0f;
    for (int c = threadIdx.x; c < k4; c += kBlock) {
        const float4 v = xb[c];
        mx = fold_abs(fold_abs(fold_abs(fold_abs(mx, v.x), v.y), v.z), v.w);
    }
    mx = wave_max(mx);
    if (lane == 0) wm[wave] = mx;
    __syncthreads();
    float amax = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) amax = wm[w] > amax ? wm[w] : amax;
    const float scale = q8_scale(amax);
    const float inv = 1.0f / scale;
    int* qb = (int*)(a.q + (size_t)b * a.kp);
    for (int c = threadIdx.x; c < k4; c += kBlock) {
        const float4 v = xb[c];
        qb[c] = pack4(v.x, v.y, v.z, v.w, inv);
    }
    if (threadIdx.x == 0) a.qs[b] = scale;
}

// ---------------------------------------------------------------- head

struct HeadA8Args {
    TMat w;                  // [vocab][d] per-row int8 tiles
    const int8_t* q;         // ln_out as int8 [rows16][kp], scales qs
    const float* qs;
    int kp;
    float* out;              // logits, stream b at out + b * ld
    int ld;
    uint32_t n, groups;
};

// 16-byte chunk ch of stream group g's int8 activations (zero past the group's chunks).
template <int NP>
__device__ __forceinline__ int4 head_chunk(const HeadA8Args& a, uint32_t g, int ch) {
    if (ch >= kRowTile * NP * 4) return make_int4(0, 0, 0, 0);
    const int row = ch / (NP * 4), col = ch % (NP * 4);
    return *(const int4*)(a.q + (size_t)(g * kRowTile + row) * a.kp + 16 * col);
}

// The head as q8_mat_vec_mul_into: each wave keeps kHeadTiles row tiles' weights (NP k-pairs
// each) in registers and walks every stream group; a group's int8 activations are staged in
// LDS once for the workgroup (the next group's requested while this one is multiplied).
template <int NP>
__global__ __launch_bounds__(kBlock) void k_head_a8(HeadA8Args a) {
    constexpr int kRow = NP * 64 + kHeadRowPad;   // LDS row stride: row j starts 8j banks apart
    constexpr int kChunks = kRowTile * NP * 4;    // 16-byte chunks of a group's activations
    constexpr int kPer = (kChunks + kBlock - 1) / kBlock;
    __shared__ __align__(16) int8_t sq[kRowTile * kRow];
    const int lane = threadIdx.x % kWave, kg = lane / 16, wave = wave_index();
    const int t0 = ((int)blockIdx.x * kWaves + wave) * kHeadTiles;
    int4 W[kHeadTiles][NP];
    float sw[kHeadTiles][4];
#pragma unroll
    for (int j = 0; j < kHeadTiles; j++) {
        const int t = min(t0 + j, a.w.rt - 1);
        const int4* A = (const int4*)a.w.w + (size_t)t * NP * 64 + lane;
#pragma unroll
        for (int p = 0; p < NP; p++) W[j][p] = A[(size_t)p * 64];
#pragma unroll
        for (int i = 0; i < 4; i++) sw[j][i] = a.w.scales[t * kRowTile + kg * 4 + i];
    }
    int4 stage[kPer];
#pragma unroll
    for (int u = 0; u < kPer; u++) stage[u] = head_chunk<NP>(a, 0, (int)threadIdx.x + kBlock * u);
    for (uint32_t g = 0; g < a.groups; g++) {
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kPer; u++) {
            const int ch = (int)threadIdx.x + kBlock * u;
            if (ch < kChunks) *(int4*)(sq + (ch / (NP * 4)) * kRow + 16 * (ch % (NP * 4))) = stage[u];
        }
        __syncthreads();
        if (g + 1 < a.groups) {
#pragma unroll
            for (int u = 0; u < kPer; u++) stage[u] = head_chunk<NP>(a, g + 1, (int)threadIdx.x + kBlock * u);
        }
        i32x4 acc[kHeadTiles];
#pragma unroll
        for (int j = 0; j < kHeadTiles; j++) acc[j] = i32x4{0, 0, 0, 0};
        const int8_t* qb = sq + (lane % 16) * kRow + 8 * kg;
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int2 lo = *(const int2*)(qb + 64 * p), hi = *(const int2*)(qb + 64 * p + 32);
#pragma unroll
            for (int j = 0; j < kHeadTiles; j++) acc[j] = mma8(W[j][p], lo, hi, acc[j]);
        }
        const uint32_t b = g * kRowTile + lane % 16;
        if (b >= a.n) continue;
        const float sb = a.qs[b];
#pragma unroll
        for (int j = 0; j < kHeadTiles; j++) {
            const int t = t0 + j;
            if (t >= a.w.rt) continue;
            const int r0 = t * kRowTile + kg * 4;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = (float)acc[j][i] * (sw[j][i] * sb);
            float* o = a.out + (size_t)b * a.ld + r0;
            if (r0 + 3 < a.w.rows && ((a.ld | r0) & 3) == 0 && ((uintptr_t)a.out & 15) == 0) {
                *(f32x4*)o = f32x4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (r0 + i < a.w.rows) o[i] = v[i];
            }
        }
    }
}

template <int... P>
const void* head_a8_pick(int np, std::integer_sequence<int, P...>) {
    const void* fns[] = {(const void*)k_head_a8<P + 1>...};
    return np >= 1 && np <= (int)sizeof...(P) ? fns[np - 1] : nullptr;
}
const void* head_a8_fn(int np) { return head_a8_pick(np, std::make_integer_sequence<int, kHeadMaxPairs>{}); }

// ---------------------------------------------------------------- step assembly

struct ProjA8Builder {
    ProjA8Args a{};
    uint32_t blocks = 0;
    uint32_t n = 0, groups = 0;
    ProjA8Builder(uint32_t n_, uint32_t groups_) : n(n_), groups(groups_) {}
    // An int8 product on int8 activations q (row kp bytes, scales qs), or on f32 activations
    // qf (row kp floats) whose pieces' maxima are pmax.
    SegA8& a8(const TMat& w, const int8_t* q, const float* qs, const float* qf, const float* pmax, int nparts, int kp,
              int mode, int act, float* out, int ld) {
        SegA8& s = a.seg[a.nseg++];
        s.kind = SEG_A8;
        s.mode = mode;
        s.act = act;
        s.w = w;
        s.q = q;
        s.qs = qs;
        s.qf = qf;
        s.pmax = pmax;
        s.nparts = nparts;
        s.kp = kp;
        // Waves per tile: as many as keep at least three k-pairs a wave (at 64 streams a
        // 768-column tile over four waves takes half the time it takes over two).
        const int np = w.ks / 2;
        int wpt = 1;
        while (wpt < kWaves && np / (2 * wpt) >= 3) wpt *= 2;
        s.wpt = wpt;
        s.out = out;
        s.ld = ld;
        s.blk0 = blocks;
        const int tpb = kWaves / wpt;
        blocks += (uint32_t)((w.rt + tpb - 1) / tpb) * groups;
        return s;
    }
    void lora(const LMat& l, const float* xf, int ldx, int act, float* out, int ld) {
        SegA8& s = a.seg[a.nseg++];
        s.kind = SEG_LORA;
        s.mode = MODE_STORE;
        s.act = act;
        s.l = l;
        s.xf = xf;
        s.ldx = ldx;
        s.out = out;
        s.ld = ld;
        s.blk0 = blocks;
        const int rows_per_block = kBlock / lora_lpr(l.cols);
        blocks += (uint32_t)((l.rows8 + rows_per_block - 1) / rows_per_block) * n;
    }
    Launch launch() {
        a.n = n;
        a.groups = groups;
        return Launch::make((const void*)k_proj_a8, dim3(blocks), dim3(kBlock), 0, KC_PROJ, a);
    }
};

}  // namespace

void RwkvStep::build_a8(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i,
                        int& sm_i) const {
    const RDims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d;
    const RwkvSizes z = rwkv_sizes(D, p.cap, true);
    const uint32_t groups = (n + kRowTile - 1) / kRowTile;
    const int dp = (int)z.dp, fp = (int)z.fp;
    int8_t* aq[kAqVecs];
    for (int k = 0; k < kAqVecs; k++) aq[k] = p.aq + (size_t)k * z.rows16 * z.dp;   // act: the last, rows fp
    float* as[kAqVecs];
    for (int k = 0; k < kAqVecs; k++) as[k] = p.as + (size_t)k * p.cap;
    float* mixf[4];
    for (int k = 0; k < 4; k++) mixf[k] = p.mixf + (size_t)k * p.cap * d;
    float* lh[4];
    for (int k = 0; k < 4; k++) lh[k] = p.lorah + z.lh_off[k];
    float* gmax = p.pmax;                                  // [rows16][heads]
    const int lsum = (int)z.lora_sum;
    const size_t state_stride = (size_t)D.nl * D.d;
    const size_t wkv_layer = (size_t)D.h * D.n * D.n;
    out.clear();
    io_i = (int)out.size();
    out.push_back(embed_launch(*m.emb, p, io, nullptr, nullptr, nullptr, 0, 0));
    for (uint32_t l = 0; l < D.nl; l++) {
        const RLayer& L = m.layers[l];
        // x_r, x_w, x_k, x_v, x_a, x_g: r, k, v -> int8; w, a, g, v -> f32 (mixf order w, a, g, v)
        ShiftA8Args s1{p.x, L.ln1_w, L.ln1_b, p.x_att + (size_t)l * d, state_stride, p.slots, p.scap, {}, {}, {}, {},
                       d, dp};
        for (int k = 0; k < kMix; k++) s1.mix[k] = L.mix[k];
        s1.outq[0] = aq[kAqR];
        s1.outs[0] = as[kAqR];
        s1.outq[2] = aq[kAqK];
        s1.outs[2] = as[kAqK];
        s1.outq[3] = aq[kAqV];
        s1.outs[3] = as[kAqV];
        s1.outf[1] = mixf[kLoraW];
        s1.outf[4] = mixf[kLoraA];
        s1.outf[5] = mixf[kLoraG];
        s1.outf[3] = mixf[kLoraV];
        out.push_back(Launch::make(shift_a8_fn(6), dim3(n), dim3(kBlock), 0, KC_SHIFT, s1));
        ProjA8Builder p1(n, groups);
        p1.a8(L.r, aq[kAqR], as[kAqR], nullptr, nullptr, 0, dp, MODE_STORE, ACT_NONE, p.rkv, 3 * d);
        p1.a8(L.k, aq[kAqK], as[kAqK], nullptr, nullptr, 0, dp, MODE_STORE, ACT_NONE, p.rkv + d, 3 * d);
        p1.a8(L.v, aq[kAqV], as[kAqV], nullptr, nullptr, 0, dp, MODE_STORE, ACT_NONE, p.rkv + 2 * d, 3 * d);
        p1.lora(L.x1[kLoraW], mixf[kLoraW], d, ACT_TANH, lh[kLoraW], lsum);
        p1.lora(L.x1[kLoraA], mixf[kLoraA], d, ACT_NONE, lh[kLoraA], lsum);
        p1.lora(L.x1[kLoraG], mixf[kLoraG], d, ACT_SIGMOID, lh[kLoraG], lsum);
        if (l != 0) p1.lora(L.x1[kLoraV], mixf[kLoraV], d, ACT_NONE, lh[kLoraV], lsum);
        out.push_back(p1.launch());
        ProjA8Builder p2(n, groups);
        for (int k = 0; k < 4; k++)
            if (k != kLoraV || l != 0) p2.lora(L.x2[k], lh[k], lsum, ACT_NONE, p.lorad + k * d, 4 * d);
        out.push_back(p2.launch());
        WkvA8Args wa{p.rkv, p.lorad, L.w0, L.a0, L.v0, L.k_k, L.k_a, L.r_k, L.ln_x_w, L.ln_x_b,
                     p.wkv + l * wkv_layer, (size_t)D.nl * wkv_layer, p.vfirst, p.slots, p.scap, p.gatedf, dp, gmax,
                     (int)D.h, d, (int)l, (int)D.g1k};
        out.push_back(Launch::make((const void*)k_wkv_a8, dim3(D.h, n), dim3(kHead), 0, KC_WKV, wa));
        ProjA8Builder po(n, groups);
        po.a8(L.o, nullptr, nullptr, p.gatedf, gmax, (int)D.h, dp, MODE_RESID, ACT_NONE, p.x, d);
        out.push_back(po.launch());
        ShiftA8Args s2{p.x, L.ln2_w, L.ln2_b, p.x_ffn + (size_t)l * d, state_stride, p.slots, p.scap, {}, {}, {}, {},
                       d, dp};
        s2.mix[0] = L.ffn_x_k;
        s2.outq[0] = aq[kAqFfn];
        s2.outs[0] = as[kAqFfn];
        out.push_back(Launch::make(shift_a8_fn(1), dim3(n), dim3(kBlock), 0, KC_SHIFT, s2));
        ProjA8Builder pk(n, groups);
        pk.a8(L.fk, aq[kAqFfn], as[kAqFfn], nullptr, nullptr, 0, dp, MODE_STORE, ACT_RELU2, p.actf, fp);
        out.push_back(pk.launch());
        QuantA8Args qa{p.actf, fp, (int)D.f, aq[kAqAct], fp, as[kAqAct]};
        out.push_back(Launch::make((const void*)k_quant_a8, dim3(n), dim3(kBlock), 0, KC_PROJ, qa));
        ProjA8Builder pv(n, groups);
        pv.a8(L.fv, aq[kAqAct], as[kAqAct], nullptr, nullptr, 0, fp, MODE_RESID, ACT_NONE, p.x, d);
        out.push_back(pv.launch());
    }
    ShiftA8Args sf{p.x, m.ln_out_w, m.ln_out_b, nullptr, 0, p.slots, p.scap, {}, {}, {}, {}, d, dp};
    sf.outq[0] = aq[kAqHead];
    sf.outs[0] = as[kAqHead];
    out.push_back(Launch::make(shift_a8_fn(0), dim3(n), dim3(kBlock), 0, KC_SHIFT, sf));
    const TMat& H = *m.head;
    head_i = (int)out.size();
    HeadA8Args ha{H, aq[kAqHead], as[kAqHead], dp, io.out + (size_t)io.b0 * D.vocab, (int)D.vocab, n, groups};
    const int per_block = kWaves * kHeadTiles;
    out.push_back(Launch::make(head_a8_fn(H.ks / 2), dim3((H.rt + per_block - 1) / per_block), dim3(kBlock), 0,
                               KC_HEAD, ha));
    sm_i = -1;
    if (io.probs) {
        sm_i = (int)out.size();
        out.push_back(softmax_launch(io.out, (int)D.vocab, n));
    }
}

void RwkvStep::build_ref(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i,
                         int& sm_i) const {
    const RDims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d, f = (int)D.f;
    const RwkvSizes z = rwkv_sizes(D, p.cap, true, true);
    // mixf: x_w, x_a, x_g, x_v (the LoRA inputs, x_v also the value input), then x_r, x_k;
    // the channel mix's input and ln_out reuse x_r's buffer once the receptance has read it
    float* mixf[6];
    for (int k = 0; k < 6; k++) mixf[k] = p.mixf + (size_t)k * p.cap * d;
    float* const xr = mixf[4];
    float* const xk = mixf[5];
    float* lh[4];
    for (int k = 0; k < 4; k++) lh[k] = p.lorah + z.lh_off[k];
    const int lsum = (int)z.lora_sum;
    const size_t state_stride = (size_t)D.nl * D.d;
    const size_t wkv_layer = (size_t)D.h * D.n * D.n;
    out.clear();
    io_i = (int)out.size();
    out.push_back(embed_launch(*m.emb, p, io, nullptr, nullptr, nullptr, 0, 0));
    for (uint32_t l = 0; l < D.nl; l++) {
        const RLayer& L = m.layers[l];
        ShiftA8Args s1{p.x, L.ln1_w, L.ln1_b, p.x_att + (size_t)l * d, state_stride, p.slots, p.scap, {}, {}, {}, {},
                       d, d};
        for (int k = 0; k < kMix; k++) s1.mix[k] = L.mix[k];
        s1.outf[0] = xr;
        s1.outf[1] = mixf[kLoraW];
        s1.outf[2] = xk;
        s1.outf[3] = mixf[kLoraV];
        s1.outf[4] = mixf[kLoraA];
        s1.outf[5] = mixf[kLoraG];
        out.push_back(Launch::make(shift_a8_fn(6), dim3(n), dim3(kBlock), 0, KC_SHIFT, s1));
        // receptance, key and value in one launch
        const RowMat* const rkv_w[3] = {&L.e_r, &L.e_k, &L.e_v};
        const float* const rkv_in[3] = {xr, xk, mixf[kLoraV]};
        const uint32_t rkv_off[3] = {0u, (uint32_t)d, 2u * d};
        out.push_back(exact_gemv3_launch(rkv_w, rkv_in, n, p.rkv, rkv_off, 3u * d, KC_PROJ));
        ProjA8Builder p1(n, 0);
        p1.lora(L.x1[kLoraW], mixf[kLoraW], d, ACT_TANH, lh[kLoraW], lsum);
        p1.lora(L.x1[kLoraA], mixf[kLoraA], d, ACT_NONE, lh[kLoraA], lsum);
        p1.lora(L.x1[kLoraG], mixf[kLoraG], d, ACT_SIGMOID, lh[kLoraG], lsum);
        if (l != 0) p1.lora(L.x1[kLoraV], mixf[kLoraV], d, ACT_NONE, lh[kLoraV], lsum);
        out.push_back(p1.launch());
        ProjA8Builder p2(n, 0);
        for (int k = 0; k < 4; k++)
            if (k != kLoraV || l != 0) p2.lora(L.x2[k], lh[k], lsum, ACT_NONE, p.lorad + k * d, 4 * d);
        out.push_back(p2.launch());
        // the gated vector in f32 rows of d (its per-head maxima are not used here)
        WkvA8Args wa{p.rkv, p.lorad, L.w0, L.a0, L.v0, L.k_k, L.k_a, L.r_k, L.ln_x_w, L.ln_x_b,
                     p.wkv + l * wkv_layer, (size_t)D.nl * wkv_layer, p.vfirst, p.slots, p.scap, p.gatedf, d, p.pmax,
                     (int)D.h, d, (int)l, (int)D.g1k};
        out.push_back(Launch::make((const void*)k_wkv_a8, dim3(D.h, n), dim3(kHead), 0, KC_WKV, wa));
        out.push_back(exact_gemv_launch(L.e_o, p.gatedf, n, p.x, (uint32_t)d, EXACT_RESID, KC_PROJ));
        ShiftA8Args s2{p.x, L.ln2_w, L.ln2_b, p.x_ffn + (size_t)l * d, state_stride, p.slots, p.scap, {}, {}, {}, {},
                       d, d};
        s2.mix[0] = L.ffn_x_k;
        s2.outf[0] = xr;
        out.push_back(Launch::make(shift_a8_fn(1), dim3(n), dim3(kBlock), 0, KC_SHIFT, s2));
        out.push_back(exact_gemv_launch(L.e_fk, xr, n, p.actf, (uint32_t)f, EXACT_RELU2, KC_PROJ));
        out.push_back(exact_gemv_launch(L.e_fv, p.actf, n, p.x, (uint32_t)d, EXACT_RESID, KC_PROJ));
    }
    ShiftA8Args sf{p.x, m.ln_out_w, m.ln_out_b, nullptr, 0, p.slots, p.scap, {}, {}, {}, {}, d, d};
    sf.outf[0] = xr;
    out.push_back(Launch::make(shift_a8_fn(0), dim3(n), dim3(kBlock), 0, KC_SHIFT, sf));
    head_i = (int)out.size();
    out.push_back(exact_gemv_launch(*m.e_head, xr, n, io.out + (size_t)io.b0 * D.vocab, D.vocab, EXACT_STORE, KC_HEAD));
    sm_i = -1;
    if (io.probs) {
        sm_i = (int)out.size();
        out.push_back(softmax_launch(io.out, (int)D.vocab, n));
    }
}

}  // namespace rdk
