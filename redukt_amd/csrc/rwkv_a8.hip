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
//   k_wkv_a8       one workgroup per stream, a wave per head: decay, a, l2-normalised key,
//                  modified key, value mix, WKV-7, GroupNorm, bonus (sequential sums), gate;
//                  the gated vector as int8
//   k_proj_a8      output projection + residual
//   k_shift_a8<1>  ln2 + channel-mix token shift -> int8
//   k_proj_a8      FFN key, squared ReLU (f32)
//   k_quant_a8     those activations -> int8
//   k_proj_a8      FFN value + residual
// then k_shift_a8<0> (ln_out -> int8), k_head_a8 and optionally the softmax.
//
// Integer products are exact, so the k-order of the int8 matrix products is free: the
// weight tiles of the int8 matrix-core tiers serve unchanged (the 16 bytes a lane holds for
// k-pair p are row r's columns 64p + 8g + [0, 8) and 64p + 32 + 8g + [0, 8), g = lane / 16)
// and the activation operand is loaded with the same column map.  Every output element
// depends on its own stream only.
#include <hip/hip_runtime.h>

#include <algorithm>

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
constexpr int kMaxHeads = kMaxD / kHead;
constexpr int kWaves = kBlock / kWave;
constexpr int kWavePairs = 12;                   // int8 products: k-pairs a wave requests at once
constexpr int kLoraRows = kBlock / 8;            // LoRA products: eight rows per wave
constexpr int kHeadMaxPairs = kMaxD / 64;

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
// row (broadcast LDS reads), so every lane ends with the sum.
__device__ __forceinline__ float seq_sum(const float* sh, int n) {
    float s = 0.0f;
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        const float4 u = *(const float4*)(sh + i);
        const float4 w = *(const float4*)(sh + i + 4);
        s += u.x; s += u.y; s += u.z; s += u.w;
        s += w.x; s += w.y; s += w.z; s += w.w;
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
    const int8_t* q;         // SEG_A8: int8 activations, stream b at q + b * kp
    const float* qs;         // their scales
    int kp;
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

// acc += the products of k-pairs [p0, p1) of one tile (weights at A, the lane's
// activations at qb), requested kWavePairs at a time before the first product.
__device__ __forceinline__ i32x4 a8_pairs(const int4* A, const int8_t* qb, int p0, int p1, i32x4 acc) {
    for (int c = p0; c < p1; c += kWavePairs) {
        int4 w[kWavePairs];
        int2 lo[kWavePairs], hi[kWavePairs];
#pragma unroll
        for (int j = 0; j < kWavePairs; j++) {
            const int p = c + j < p1 ? c + j : p1 - 1;
            w[j] = A[(size_t)p * 64];
            lo[j] = *(const int2*)(qb + 64 * p);
            hi[j] = *(const int2*)(qb + 64 * p + 32);
        }
#pragma unroll
        for (int j = 0; j < kWavePairs; j++)
            if (c + j < p1) acc = mma8(w[j], lo[j], hi[j], acc);
    }
    return acc;
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
    i32x4 acc = {0, 0, 0, 0};
    if (live) {
        const int share = (np + s.wpt - 1) / s.wpt;
        const int p0 = part * share, p1 = min(np, p0 + share);
        acc = a8_pairs((const int4*)s.w.w + (size_t)t * np * 64 + lane, s.q + (size_t)b * s.kp + 8 * kg, p0, p1, acc);
    }
    if (s.wpt > 1) {
        if (part > 0) red[wave][lane] = acc;
        __syncthreads();
        if (part > 0) return;
        for (int j = 1; j < s.wpt; j++) acc += red[wave + j][lane];
    }
    if (!live || b >= n) return;
    const int r0 = t * kRowTile + kg * 4;
    const float sb = s.qs[b];
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = activate(s.act, (float)acc[i] * (s.w.scales[r0 + i] * sb), 0, 0);
    float* o = s.out + (size_t)b * s.ld + r0;
    if (r0 + 3 < s.w.rows && ((s.ld | r0) & 3) == 0 && ((uintptr_t)s.out & 15) == 0) {
        f32x4 y = s.mode == MODE_RESID ? *(f32x4*)o : f32x4{0, 0, 0, 0};
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

// mat_vec_mul_into over f32 (tensor.rs:1602-1693, dot_avx2_order) for eight rows of one
// stream (the wave): lane l of a row's eight accumulates the columns c = l (mod 8) from +0
// with one multiply and one add each, then hsum_f32_scalar ((a0 + a4) + (a2 + a6)) +
// ((a1 + a5) + (a3 + a7)) over the eight lanes (each pairing one commutative add), then
// the activation of the LoRA stage.
__device__ __forceinline__ void lora_rows(const SegA8& s, int rb, uint32_t b) {
    const int lane = threadIdx.x % kWave, l = lane % 8;
    const int r = rb * kLoraRows + wave_index() * 8 + lane / 8;
    const int rr = r < s.l.rows8 ? r : s.l.rows8 - 1;
    const int steps = s.l.cols / 8;
    const float* w = s.l.w + (size_t)rr * 8 + l;
    const size_t wstep = (size_t)s.l.rows8 * 8;
    const float* x = s.xf + (size_t)b * s.ldx + l;
    float acc = 0.0f;
    int i = 0;
    for (; i + 8 <= steps; i += 8) {
        float wv[8], xv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            wv[u] = w[(i + u) * wstep];
            xv[u] = x[8 * (i + u)];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) acc += wv[u] * xv[u];
    }
    for (; i < steps; i++) acc += w[i * wstep] * x[8 * i];
    float h = acc + __shfl_xor(acc, 4, kWave);
    h = h + __shfl_xor(h, 2, kWave);
    h = h + __shfl_xor(h, 1, kWave);
    if (l == 0 && r < s.l.rows) s.out[(size_t)b * s.ld + r] = activate(s.act, h, r, s.l.rows);
}

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
    } else {
        lora_rows(s, (int)(local / a.n), local % a.n);
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
    int8_t* q;               // the gated vector as int8 [rows16][dp], its scale per stream
    float* qs;
    int dp, d, layer, g1k;
};

// time_mixing_scratch steps 3-12 after the projections (model.rs:827-912) for one stream:
// wave h owns head h, lane i channel c = 64 h + i and row i of the head's state.  The sums
// over a head (l2 norm, GroupNorm mean and variance, bonus) are sequential; the state
// products t = S·(-kk) and out = S·r already run over j in order per lane.  Then the gated
// vector goes to int8 for the output projection (its amax over all heads).
__global__ __launch_bounds__(kMaxD) void k_wkv_a8(WkvA8Args a) {
    __shared__ __align__(16) float sw[kMaxHeads][kHead], skka[kMaxHeads][kHead], snegkk[kMaxHeads][kHead];
    __shared__ __align__(16) float skmod[kMaxHeads][kHead], sr[kMaxHeads][kHead];
    __shared__ __align__(16) float sa[kMaxHeads][kHead], sb[kMaxHeads][kHead];
    __shared__ float smax[kMaxHeads];
    const int i = threadIdx.x % kHead, h = threadIdx.x / kHead;
    const int heads = (int)blockDim.x / kHead;
    const uint32_t b = blockIdx.x;
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
    sa[h][i] = kk0 * kk0;
    __syncthreads();
    const float norm = sqrtf(seq_sum(sa[h], kHead));
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
    sw[h][i] = w;
    skka[h][i] = kk * aa;
    snegkk[h][i] = -kk;
    skmod[h][i] = kmod;
    sr[h][i] = r;
    __syncthreads();
    float tt = 0.0f;
#pragma unroll
    for (int j = 0; j < kHead; j++) tt += S[j] * snegkk[h][j];
#pragma unroll
    for (int j = 0; j < kHead; j++) S[j] = S[j] * sw[h][j] + tt * skka[h][j] + vout * skmod[h][j];
    float o = 0.0f;
#pragma unroll
    for (int j = 0; j < kHead; j++) o += S[j] * sr[h][j];
#pragma unroll
    for (int q = 0; q < kHead / 4; q++) sbase[q * kHead + i] = make_float4(S[4 * q], S[4 * q + 1], S[4 * q + 2], S[4 * q + 3]);
    // Step 10: GroupNorm over the head, eps 64e-5 (group_norm_into :1400-1414); step 11:
    // bonus = sum over the head of r * k * r_k (k_mod for g1k models), times v_out
    const float ksrc = a.g1k ? kmod : k;
    sa[h][i] = o;
    sb[h][i] = r * ksrc * a.r_k[c];
    __syncthreads();
    float osum, bonus;
    seq_sum2_64(sa[h], sb[h], osum, bonus);
    const float mean = osum / (float)kHead;
    __syncthreads();
    sa[h][i] = (o - mean) * (o - mean);
    __syncthreads();
    const float var = seq_sum(sa[h], kHead) / (float)kHead;
    float on = (o - mean) * (1.0f / sqrtf(var + 64e-5f)) * a.ln_x_w[c] + a.ln_x_b[c];
    on += bonus * vout;
    // Step 12: gate, then int8 for the output projection
    const float gated = on * g;
    const float mx = wave_max(fold_abs(0.0f, gated));
    if (i == 0) smax[h] = mx;
    __syncthreads();
    float amax = 0.0f;
    for (int hh = 0; hh < heads; hh++) amax = smax[hh] > amax ? smax[hh] : amax;
    const float scale = q8_scale(amax);
    a.q[(size_t)b * a.dp + c] = q8_of(gated, 1.0f / scale);
    if (threadIdx.x == 0) a.qs[b] = scale;
}

// ---------------------------------------------------------------- activations -> int8

struct QuantA8Args {
    const float* x;          // stream b at x + b * ld, K values
    int ld, K;
    int8_t* q;               // [rows16][kp]
    int kp;
    float* qs;
};

__global__ __launch_bounds__(kBlock) void k_quant_a8(QuantA8Args a) {
    __shared__ float wm[kBlock / kWave];
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
    for (int w = 0; w < kBlock / kWave; w++) amax = wm[w] > amax ? wm[w] : amax;
    const float scale = q8_scale(amax);
    const float inv = 1.0f / scale;
    uint32_t* qb = (uint32_t*)(a.q + (size_t)b * a.kp);
    for (int c = threadIdx.x; c < k4; c += kBlock) {
        const float4 v = xb[c];
        qb[c] = (uint32_t)(uint8_t)q8_of(v.x, inv) | (uint32_t)(uint8_t)q8_of(v.y, inv) << 8 |
                (uint32_t)(uint8_t)q8_of(v.z, inv) << 16 | (uint32_t)(uint8_t)q8_of(v.w, inv) << 24;
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

// The head as q8_mat_vec_mul_into: each wave keeps one 16-row tile's weights in registers
// and walks every stream group.
__global__ __launch_bounds__(kBlock) void k_head_a8(HeadA8Args a) {
    const int lane = threadIdx.x % kWave, kg = lane / 16;
    const int t = (int)blockIdx.x * kWaves + wave_index();
    if (t >= a.w.rt) return;
    const int np = a.w.ks / 2;
    int4 W[kHeadMaxPairs];
    const int4* A = (const int4*)a.w.w + (size_t)t * np * 64 + lane;
#pragma unroll
    for (int p = 0; p < kHeadMaxPairs; p++)
        if (p < np) W[p] = A[(size_t)p * 64];
    const int r0 = t * kRowTile + kg * 4;
    float sw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sw[i] = a.w.scales[r0 + i];
    const bool vec = r0 + 3 < a.w.rows && ((a.ld | r0) & 3) == 0 && ((uintptr_t)a.out & 15) == 0;
    for (uint32_t g = 0; g < a.groups; g++) {
        const uint32_t b = g * kRowTile + lane % 16;
        const int8_t* qb = a.q + (size_t)b * a.kp + 8 * kg;
        i32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < kHeadMaxPairs; p += 2) {
            if (p < np) acc0 = mma8(W[p], *(const int2*)(qb + 64 * p), *(const int2*)(qb + 64 * p + 32), acc0);
            if (p + 1 < np)
                acc1 = mma8(W[p + 1], *(const int2*)(qb + 64 * p + 64), *(const int2*)(qb + 64 * p + 96), acc1);
        }
        const i32x4 acc = acc0 + acc1;
        if (b >= a.n) continue;
        const float sb = a.qs[b];
        float* o = a.out + (size_t)b * a.ld + r0;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = (float)acc[i] * (sw[i] * sb);
        if (vec) {
            *(f32x4*)o = f32x4{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (r0 + i < a.w.rows) o[i] = v[i];
        }
    }
}

// ---------------------------------------------------------------- step assembly

struct ProjA8Builder {
    ProjA8Args a{};
    uint32_t blocks = 0;
    uint32_t n = 0, groups = 0;
    ProjA8Builder(uint32_t n_, uint32_t groups_) : n(n_), groups(groups_) {}
    void a8(const TMat& w, const int8_t* q, const float* qs, int kp, int mode, int act, float* out, int ld) {
        SegA8& s = a.seg[a.nseg++];
        s.kind = SEG_A8;
        s.mode = mode;
        s.act = act;
        s.w = w;
        s.q = q;
        s.qs = qs;
        s.kp = kp;
        // Waves per tile: enough that a wave's share fits one request of kWavePairs, more
        // while the launch has few tiles (each wave then waits on fewer requests in turn).
        const int np = w.ks / 2;
        int wpt = 1;
        while (wpt < kWaves && (np + wpt - 1) / wpt > kWavePairs) wpt *= 2;
        while (wpt < kWaves && (size_t)w.rt * groups * wpt < 1024 && np / (2 * wpt) >= 3) wpt *= 2;
        s.wpt = wpt;
        s.out = out;
        s.ld = ld;
        s.blk0 = blocks;
        const int tpb = kWaves / wpt;
        blocks += (uint32_t)((w.rt + tpb - 1) / tpb) * groups;
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
        blocks += (uint32_t)((l.rows8 + kLoraRows - 1) / kLoraRows) * n;
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
    const int d = (int)D.d, ff = (int)D.f;
    const RwkvSizes z = rwkv_sizes(D, p.cap, true);
    const uint32_t groups = (n + kRowTile - 1) / kRowTile;
    const int dp = (int)z.dp, fp = (int)z.fp;
    int8_t* aq[kAqVecs];
    for (int k = 0; k < kAqVecs; k++) aq[k] = p.aq + (size_t)k * z.rows16 * z.dp;
    float* as[kAqVecs];
    for (int k = 0; k < kAqVecs; k++) as[k] = p.as + (size_t)k * p.cap;
    float* mixf[4];
    for (int k = 0; k < 4; k++) mixf[k] = p.mixf + (size_t)k * p.cap * d;
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
        p1.a8(L.r, aq[kAqR], as[kAqR], dp, MODE_STORE, ACT_NONE, p.rkv, 3 * d);
        p1.a8(L.k, aq[kAqK], as[kAqK], dp, MODE_STORE, ACT_NONE, p.rkv + d, 3 * d);
        p1.a8(L.v, aq[kAqV], as[kAqV], dp, MODE_STORE, ACT_NONE, p.rkv + 2 * d, 3 * d);
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
                     p.wkv + l * wkv_layer, (size_t)D.nl * wkv_layer, p.vfirst, p.slots, p.scap, aq[kAqGated],
                     as[kAqGated], dp, d, (int)l, (int)D.g1k};
        out.push_back(Launch::make((const void*)k_wkv_a8, dim3(n), dim3(D.h * kHead), 0, KC_WKV, wa));
        ProjA8Builder po(n, groups);
        po.a8(L.o, aq[kAqGated], as[kAqGated], dp, MODE_RESID, ACT_NONE, p.x, d);
        out.push_back(po.launch());
        ShiftA8Args s2{p.x, L.ln2_w, L.ln2_b, p.x_ffn + (size_t)l * d, state_stride, p.slots, p.scap, {}, {}, {}, {},
                       d, dp};
        s2.mix[0] = L.ffn_x_k;
        s2.outq[0] = aq[kAqFfn];
        s2.outs[0] = as[kAqFfn];
        out.push_back(Launch::make(shift_a8_fn(1), dim3(n), dim3(kBlock), 0, KC_SHIFT, s2));
        ProjA8Builder pk(n, groups);
        pk.a8(L.fk, aq[kAqFfn], as[kAqFfn], dp, MODE_STORE, ACT_RELU2, p.actf, ff);
        out.push_back(pk.launch());
        QuantA8Args qa{p.actf, ff, ff, aq[kAqAct], fp, as[kAqAct]};
        out.push_back(Launch::make((const void*)k_quant_a8, dim3(n), dim3(kBlock), 0, KC_PROJ, qa));
        ProjA8Builder pv(n, groups);
        pv.a8(L.fv, aq[kAqAct], as[kAqAct], fp, MODE_RESID, ACT_NONE, p.x, d);
        out.push_back(pv.launch());
    }
    ShiftA8Args sf{p.x, m.ln_out_w, m.ln_out_b, nullptr, 0, p.slots, p.scap, {}, {}, {}, {}, d, dp};
    sf.outq[0] = aq[kAqHead];
    sf.outs[0] = as[kAqHead];
    out.push_back(Launch::make(shift_a8_fn(0), dim3(n), dim3(kBlock), 0, KC_SHIFT, sf));
    const TMat& H = *m.head;
    head_i = (int)out.size();
    HeadA8Args ha{H, aq[kAqHead], as[kAqHead], dp, io.out + (size_t)io.b0 * D.vocab, (int)D.vocab, n, groups};
    out.push_back(Launch::make((const void*)k_head_a8, dim3((H.rt + kWaves - 1) / kWaves),
                               dim3(kBlock), 0, KC_HEAD, ha));
    sm_i = -1;
    if (io.probs) {
        sm_i = (int)out.size();
        out.push_back(softmax_launch(io.out, (int)D.vocab, n));
    }
}

}  // namespace rdk
