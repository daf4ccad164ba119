// rwkv_step.hip — gfx950 kernels of one RWKV-7 token step for N lockstep streams
// (src/infrastructure/rwkv7/model.rs:643-925).
//
// Per layer, in stream order (all replayed from the step's hipGraph):
//   k_rwkv_shift  ln1 LayerNorm, token shift against the slot's previous ln1 output,
//                 the six mixed inputs x_r..x_g as bf16 limbs (B-fragment tiles)
//   k_proj        receptance, key, value (f32 out) and the first LoRA stages with their
//                 activation (tanh for decay, sigmoid for g) as limbs
//   k_proj        second LoRA stages (f32 out)
//   k_rwkv_wkv    decay, a, g, l2-normalised key, modified key, value mix, the WKV-7
//                 update of the 64x64 head state, GroupNorm, bonus, gate (limbs out)
//   k_proj        output projection + residual
//   k_rwkv_shift  ln2 LayerNorm + channel-mix token shift (limbs)
//   k_proj        FFN key + squared ReLU (limbs)
//   k_proj        FFN value + residual
// then the final LayerNorm and the head, and optionally the softmax.
//
// Projections use the three-limb bf16 split of mfma_common.h (exact int8 weights, F32
// weights in six limb products).  The element-wise code follows the reference's order
// and portable exp (lane forms on the 8-aligned body); sums over a head or a row that
// the reference takes sequentially (LayerNorm, GroupNorm, l2 norm, bonus) are fixed-order
// trees here, so those differ from the CPU path in the last bits only.  Every output
// element depends on its own stream only: results do not depend on n, position or slot.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "mfma_common.h"
#include "model.h"
#include "portable_math.h"
#include "rwkv_common.h"
#include "step.h"

#pragma clang fp contract(off)

namespace rdk {

RwkvSizes rwkv_sizes(const RDims& D, uint32_t cap, bool a8, bool exact) {
    RwkvSizes z{};
    const size_t gcap = (cap + 15) / 16;
    auto ks_of = [](uint32_t cols) { return (int)((cols + kKAlign - 1) / kKAlign * (kKAlign / kKStep)); };
    z.ks_d = ks_of(D.d);
    z.ks_f = ks_of(D.f);
    // Recurrent state over cap + 1 slots: slot cap is the pool's scratch slot.
    z.state_d = (size_t)(cap + 1) * D.nl * D.d;
    z.wkv = (size_t)(cap + 1) * D.nl * D.h * D.n * D.n;
    size_t off = 0, loff = 0;
    for (int i = 0; i < 4; i++) {
        z.ks_lora[i] = ks_of(D.lora[i]);
        z.lora_off[i] = off;
        off += gcap * z.ks_lora[i] * 3 * 512;
        z.lh_off[i] = loff;
        loff += D.lora[i];
    }
    z.lora_sum = loff;
    z.dp = (size_t)z.ks_d * kKStep;
    z.fp = (size_t)z.ks_f * kKStep;
    z.rows16 = gcap * 16;
    if (a8) {
        z.mixf = (exact ? 6 : 4) * (size_t)cap * D.d;
        z.lorah = (size_t)cap * z.lora_sum;
        z.aq = z.rows16 * (kAqAct * z.dp + z.fp);
        z.as = (size_t)kAqVecs * cap;
        z.gatedf = z.rows16 * z.dp;
        z.actf = z.rows16 * z.fp;
        z.pmax = z.rows16 * D.h;
    } else {
        z.mixl = gcap * z.ks_d * 3 * 512;
        z.gatedl = z.mixl;
        z.actl = gcap * z.ks_f * 3 * 512;
        z.loral = off;
    }
    return z;
}

namespace {

constexpr int kBlock = 256;
constexpr int kProjWaves = 8;
constexpr int kProjPairs = 3;    // k-pairs per wave and pass
constexpr int kMaxSegs = 8;
constexpr int kMaxShiftMix = 6;

// ---------------------------------------------------------------- LayerNorm + token shift

struct ShiftArgs {
    const float* x;              // [n][d]
    const float* ln_w;
    const float* ln_b;
    float* prev;                 // slot s's previous ln output at prev + s * prev_stride (null: none)
    size_t prev_stride;
    const uint32_t* slots;
    uint32_t cap;                // state slots of the pool (the clamp bound)
    int nmix;                    // 0: the ln output itself goes to out[0]
    const float* mix[kMaxShiftMix];
    __bf16* out[kMaxShiftMix];
    int ks, d;
};

// layer_norm_into (tensor.rs:1390-1398): mean, then the mean of squared deviations,
// (x - mean) * (1 / sqrt(var + 1e-5)) * w + b; the token shift of time_mixing_scratch
// (model.rs:811-820) / channel_mixing_scratch (:920-921): xx = prev - ln,
// input_m = ln + xx * mix_m; the slot's prev becomes ln (model.rs:663, 675).
// NMIX = a.nmix (0: the ln output itself goes to out[0], no previous value).  Every
// operand is requested before the first wait: the slot, x, the LayerNorm weights, the
// mixes, then the slot's previous ln once the slot is known.  Channels past d re-read
// channel d - 1 and are left out of the sums and the stores.
template <int NMIX>
__global__ __launch_bounds__(kBlock) void k_rwkv_shift(ShiftArgs a) {
    __shared__ float sh[2][kBlock / kWave];
    const uint32_t b = blockIdx.x;
    const int d = a.d;
    constexpr int kPer = 4;  // d <= 1024
    constexpr int kMix = NMIX ? NMIX : 1;
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const uint32_t slot = NMIX ? clamp_slot(a.slots[b], a.cap) : 0u;
    int cc[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) cc[q] = min((int)threadIdx.x + kBlock * q, d - 1);
    float xv[kPer], wv[kPer], bv[kPer], mv[kMix][kPer], pv[kPer];
    const float* xb = a.x + (size_t)b * d;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        xv[q] = xb[cc[q]];
        wv[q] = a.ln_w[cc[q]];
        bv[q] = a.ln_b[cc[q]];
    }
#pragma unroll
    for (int m = 0; m < NMIX; m++)
#pragma unroll
        for (int q = 0; q < kPer; q++) mv[m][q] = a.mix[m][cc[q]];
    float* const pp = NMIX ? a.prev + slot * a.prev_stride : nullptr;
#pragma unroll
    for (int q = 0; q < kPer; q++) pv[q] = NMIX ? pp[cc[q]] : 0.0f;
    bool in[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) in[q] = (int)threadIdx.x + kBlock * q < d;
    // Block sums: wave sums, then ((w0 + w1) + w2) + w3; each sum has its own LDS row, so
    // one barrier per sum.
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < kPer; q++) s += in[q] ? xv[q] : 0.0f;
    s = wave_sum(s);
    if (lane == 0) sh[0][wave] = s;
    __syncthreads();
    const float mean = (((sh[0][0] + sh[0][1]) + sh[0][2]) + sh[0][3]) / (float)d;
    float vs = 0.0f;
#pragma unroll
    for (int q = 0; q < kPer; q++)
        if (in[q]) vs += (xv[q] - mean) * (xv[q] - mean);
    vs = wave_sum(vs);
    if (lane == 0) sh[1][wave] = vs;
    __syncthreads();
    const float inv = 1.0f / sqrtf((((sh[1][0] + sh[1][1]) + sh[1][2]) + sh[1][3]) / (float)d + 1e-5f);
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        if (!in[q]) continue;
        const int c = cc[q];
        const float ln = (xv[q] - mean) * inv * wv[q] + bv[q];
        if (NMIX == 0) {
            write_limb1(a.out[0], a.ks, b, c, ln);
            continue;
        }
        const float xx = pv[q] - ln;
#pragma unroll
        for (int m = 0; m < NMIX; m++) write_limb1(a.out[m], a.ks, b, c, ln + xx * mv[m][q]);
        pp[c] = ln;
    }
}

const void* shift_fn(int nmix) {
    if (nmix == 6) return (const void*)k_rwkv_shift<6>;
    if (nmix == 1) return (const void*)k_rwkv_shift<1>;
    return (const void*)k_rwkv_shift<0>;
}

// ---------------------------------------------------------------- projections

enum { PROJ_STORE = 0, PROJ_RESID = 1, PROJ_LIMBS = 2 };

struct ProjSeg {
    TMat w;
    const __bf16* in;        // B-fragment limbs with w.ks k-steps
    int mode, act;
    float* out;              // STORE / RESID: out[b * ld + row]
    int ld;
    __bf16* lout;            // LIMBS: the rows of w become the k of lout (lks k-steps)
    int lks;
    int tile0;               // first blockIdx.x of this segment
};

struct ProjArgs {
    ProjSeg seg[kMaxSegs];
    int nseg;
    uint32_t n;
};

template <bool Q8>
__device__ __forceinline__ void proj_finish(const ProjSeg& sg, int t, f32x4 s, uint32_t n);

// One 16-row tile x 16 streams.  Eight waves each take an eighth of the k-pairs (limb
// orders in separate accumulators), with kProjPairs pairs of weight and activation
// fragments requested at once; the eighths are added in wave order, then the row scale.
template <bool Q8>
__device__ __forceinline__ void proj_tile(const ProjSeg& sg, int t, uint32_t n, f32x4 (*part)[kWave]) {
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const uint32_t b0 = blockIdx.y * kRowTile;
    const TMat& w = sg.w;
    const int np = w.ks / 2;
    const int p_lo = wave * np / kProjWaves, p_hi = (wave + 1) * np / kProjWaves;
    const bool grp = Q8 && w.group != w.cols;
    const int gpr = w.ks / 2;
    const uint32_t g0 = b0 / kRowTile;
    f32x4 acc3[3];
#pragma unroll
    for (int o = 0; o < 3; o++) acc3[o] = f32x4{0, 0, 0, 0};
#pragma unroll 1
    for (int pb = p_lo; pb < p_hi; pb += kProjPairs) {
        RawPair raw[kProjPairs];
        bf16x8 bfr[kProjPairs][2][3];
        float sc[kProjPairs][4];
#pragma unroll
        for (int q = 0; q < kProjPairs; q++) {
            const int p = pb + q;
            if (p >= p_hi) break;
            raw[q] = load_pair<Q8>(w, t, p, lane);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const __bf16* f = sg.in + (((size_t)g0 * w.ks + 2 * p + h) * 3) * 512 + lane * 8;
                bfr[q][h][0] = lds_frag(f);
                bfr[q][h][1] = lds_frag(f + 512);
                bfr[q][h][2] = lds_frag(f + 1024);
            }
            if (grp) {
#pragma unroll
                for (int i = 0; i < 4; i++) sc[q][i] = w.scales[(size_t)(t * kRowTile + (lane / 16) * 4 + i) * gpr + p];
            }
        }
#pragma unroll
        for (int q = 0; q < kProjPairs; q++) {
            const int p = pb + q;
            if (p >= p_hi) break;
            AFrag a0, a1;
            decode_pair<Q8>(raw[q], a0, a1);
            if (grp) {
                f32x4 pp{0, 0, 0, 0};
                pp = mma_step<Q8>(a0, bfr[q][0][0], bfr[q][0][1], bfr[q][0][2], pp);
                pp = mma_step<Q8>(a1, bfr[q][1][0], bfr[q][1][1], bfr[q][1][2], pp);
#pragma unroll
                for (int i = 0; i < 4; i++) acc3[0][i] = __builtin_fmaf(pp[i], sc[q][i], acc3[0][i]);
            } else {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const AFrag& af = h ? a1 : a0;
                    const bf16x8* bb = bfr[q][h];
                    if (Q8) {
                        acc3[0] = mma(af.h, bb[0], acc3[0]);
                        acc3[1] = mma(af.h, bb[1], acc3[1]);
                        acc3[2] = mma(af.h, bb[2], acc3[2]);
                    } else {
                        acc3[0] = mma(af.h, bb[0], acc3[0]);
                        acc3[1] = mma(af.h, bb[1], acc3[1]);
                        acc3[1] = mma(af.m, bb[0], acc3[1]);
                        acc3[2] = mma(af.h, bb[2], acc3[2]);
                        acc3[2] = mma(af.m, bb[1], acc3[2]);
                        acc3[2] = mma(af.l, bb[0], acc3[2]);
                    }
                }
            }
        }
    }
    const f32x4 acc = (acc3[0] + acc3[1]) + acc3[2];
    if (wave > 0) part[wave - 1][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    f32x4 s = acc;
    for (int q = 0; q < kProjWaves - 1; q++) s = s + part[q][lane];
    proj_finish<Q8>(sg, t, s, n);
}

// The epilogue of row tile t from its summed products s (one wave): the row scale, then
// the segment's output (limbs after the activation, a store, or a residual add).
template <bool Q8>
__device__ __forceinline__ void proj_finish(const ProjSeg& sg, int t, f32x4 s, uint32_t n) {
    const int lane = threadIdx.x % kWave;
    const uint32_t b0 = blockIdx.y * kRowTile;
    const TMat& w = sg.w;
    const bool grp = Q8 && w.group != w.cols;
    const int r0 = t * kRowTile + (lane / 16) * 4;
    const uint32_t b = b0 + lane % 16;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float rs = Q8 && !grp ? w.scales[r0 + i] : 1.0f;
        v[i] = s[i] * rs;
    }
    const bool ok = b < n;
    if (sg.mode == PROJ_LIMBS) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = r0 + i < w.rows ? activate(sg.act, v[i], r0 + i, w.rows) : 0.0f;
        if (ok) write_limbs4(sg.lout, sg.lks, t, b, v);
        return;
    }
    if (!ok) return;
    float* o = sg.out + (size_t)b * sg.ld + r0;
    if (r0 + 3 < w.rows && ((sg.ld | r0) & 3) == 0 && ((uintptr_t)sg.out & 15) == 0) {
        // The lane's four rows in one 16-byte access (row-major out, 16-byte aligned rows).
        f32x4 y = *(f32x4*)o;
#pragma unroll
        for (int i = 0; i < 4; i++) y[i] = sg.mode == PROJ_RESID ? y[i] + v[i] : v[i];
        *(f32x4*)o = y;
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (r0 + i >= w.rows) continue;
        o[i] = sg.mode == PROJ_RESID ? o[i] + v[i] : v[i];
    }
}

__global__ __launch_bounds__(kProjWaves * kWave) void k_proj(ProjArgs a) {
    __shared__ f32x4 part[kProjWaves - 1][kWave];
    int si = 0;
    for (int i = 1; i < a.nseg; i++)
        if ((int)blockIdx.x >= a.seg[i].tile0) si = i;
    const ProjSeg sg = a.seg[si];
    const int t = blockIdx.x - sg.tile0;
    if (sg.w.group) proj_tile<true>(sg, t, a.n, part);
    else proj_tile<false>(sg, t, a.n, part);
}

// TT row tiles x 16 streams per workgroup: each wave multiplies all TT tiles over its
// eighth of the k-pairs with one load of the activation fragments, every tile's products
// in proj_tile's order; the eight waves' sums go through LDS and wave i < TT adds tile i's
// in wave order (wave 0's first, as proj_tile does), so every output has proj_tile's bits.
// Tiles past the segment's last load its last tile's weights and store nothing.
template <bool Q8, int TT>
__device__ __forceinline__ void proj_tiles(const ProjSeg& sg, int tb, uint32_t n, f32x4 (*part)[TT][kWave]) {
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const uint32_t b0 = blockIdx.y * kRowTile;
    const TMat& w = sg.w;
    const int np = w.ks / 2;
    const int p_lo = wave * np / kProjWaves, p_hi = (wave + 1) * np / kProjWaves;
    const bool grp = Q8 && w.group != w.cols;
    const int gpr = w.ks / 2;
    const uint32_t g0 = b0 / kRowTile;
    const int t0 = tb * TT;
    // k-pairs requested per pass (batching only: the products' order is the same)
    constexpr int PP = TT >= 4 ? 1 : kProjPairs;
    int tl[TT];
#pragma unroll
    for (int i = 0; i < TT; i++) tl[i] = min(t0 + i, w.rt - 1);
    f32x4 acc3[TT][3];
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
        for (int o = 0; o < 3; o++) acc3[i][o] = f32x4{0, 0, 0, 0};
#pragma unroll 1
    for (int pb = p_lo; pb < p_hi; pb += PP) {
        RawPair raw[PP][TT];
        bf16x8 bfr[PP][2][3];
        float sc[PP][TT][4];
#pragma unroll
        for (int q = 0; q < PP; q++) {
            const int p = pb + q;
            if (p >= p_hi) break;
#pragma unroll
            for (int i = 0; i < TT; i++) raw[q][i] = load_pair<Q8>(w, tl[i], p, lane);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const __bf16* f = sg.in + (((size_t)g0 * w.ks + 2 * p + h) * 3) * 512 + lane * 8;
                bfr[q][h][0] = lds_frag(f);
                bfr[q][h][1] = lds_frag(f + 512);
                bfr[q][h][2] = lds_frag(f + 1024);
            }
            if (grp) {
#pragma unroll
                for (int i = 0; i < TT; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        sc[q][i][e] = w.scales[(size_t)(tl[i] * kRowTile + (lane / 16) * 4 + e) * gpr + p];
            }
        }
#pragma unroll
        for (int q = 0; q < PP; q++) {
            const int p = pb + q;
            if (p >= p_hi) break;
#pragma unroll
            for (int i = 0; i < TT; i++) {
                AFrag a0, a1;
                decode_pair<Q8>(raw[q][i], a0, a1);
                if (grp) {
                    f32x4 pp{0, 0, 0, 0};
                    pp = mma_step<Q8>(a0, bfr[q][0][0], bfr[q][0][1], bfr[q][0][2], pp);
                    pp = mma_step<Q8>(a1, bfr[q][1][0], bfr[q][1][1], bfr[q][1][2], pp);
#pragma unroll
                    for (int e = 0; e < 4; e++) acc3[i][0][e] = __builtin_fmaf(pp[e], sc[q][i][e], acc3[i][0][e]);
                } else {
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const AFrag& af = h ? a1 : a0;
                        const bf16x8* bb = bfr[q][h];
                        if (Q8) {
                            acc3[i][0] = mma(af.h, bb[0], acc3[i][0]);
                            acc3[i][1] = mma(af.h, bb[1], acc3[i][1]);
                            acc3[i][2] = mma(af.h, bb[2], acc3[i][2]);
                        } else {
                            acc3[i][0] = mma(af.h, bb[0], acc3[i][0]);
                            acc3[i][1] = mma(af.h, bb[1], acc3[i][1]);
                            acc3[i][1] = mma(af.m, bb[0], acc3[i][1]);
                            acc3[i][2] = mma(af.h, bb[2], acc3[i][2]);
                            acc3[i][2] = mma(af.m, bb[1], acc3[i][2]);
                            acc3[i][2] = mma(af.l, bb[0], acc3[i][2]);
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < TT; i++) part[wave][i][lane] = (acc3[i][0] + acc3[i][1]) + acc3[i][2];
    __syncthreads();
    if (wave >= TT || t0 + wave >= w.rt) return;
    f32x4 s = part[0][wave][lane];
    for (int q = 1; q < kProjWaves; q++) s = s + part[q][wave][lane];
    proj_finish<Q8>(sg, t0 + wave, s, n);
}

template <int TT>
__global__ __launch_bounds__(kProjWaves * kWave) void k_proj_t(ProjArgs a) {
    __shared__ f32x4 part[kProjWaves][TT][kWave];
    int si = 0;
    for (int i = 1; i < a.nseg; i++)
        if ((int)blockIdx.x >= a.seg[i].tile0) si = i;
    const ProjSeg sg = a.seg[si];
    const int tb = blockIdx.x - sg.tile0;
    if (sg.w.group) proj_tiles<true, TT>(sg, tb, a.n, part);
    else proj_tiles<false, TT>(sg, tb, a.n, part);
}

// Row tiles per projection workgroup (1: k_proj): four when the step runs as parts (n of
// n_all streams), whose launches share the device, one otherwise.  Measured at RWKV-7 0.1B,
// µs per step for one / two / four tiles, int8 per-row: 64 streams in one part 747 / 802 /
// 797, 128 streams in two parts 1042 / 1025 / 973, 256 streams 1571 / 1509 / 1303; F32:
// 64 streams 922 / 1012 / 1060, 128 1313 / 1304 / 1305, 256 2045 / 1988 / 1911.
// REDUKT_GPU_PROJ_TILES = 1, 2 or 4 forces a count.
int proj_tiles_for(uint32_t n, uint32_t n_all) {
    const char* e = getenv("REDUKT_GPU_PROJ_TILES");
    const int v = e && *e ? atoi(e) : 0;
    if (v == 1 || v == 2 || v == 4) return v;
    return n_all > n ? 4 : 1;
}

// ---------------------------------------------------------------- WKV-7

struct WkvArgs {
    const float* rkv;        // [n][3d]: r, k, v
    const float* lorad;      // [n][4d]: decay, a, g, v second LoRA stages
    const float *w0, *a0, *v0, *k_k, *k_a, *r_k, *ln_x_w, *ln_x_b;
    float* wkv;              // this layer's state of slot s at wkv + s * slot_stride
    size_t slot_stride;
    float* vfirst;           // [n][d]
    const uint32_t* slots;
    uint32_t cap;            // state slots of the pool (the clamp bound)
    __bf16* gated;           // B-fragment limbs with ks k-steps
    int ks, d, layer, g1k;
};

constexpr int kHead = 64;

// The sum of v over the 64 lanes of a wave, in every lane: lanes paired by DPP inside each
// row of 16 (i ^ 1, i ^ 2, then the mirrored quads and halves; each add pairs equal partial
// sums in both orders, which IEEE addition makes equal), then the four row sums
// (r0 + r1) + (r2 + r3).  Every lane must be active.  Four VALU moves and four lane reads,
// against six LDS permutes for a butterfly over __shfl_xor.
__device__ __forceinline__ float wave_sum_rows(float v) {
    v = v + dpp_move<kDppQuadXor1>(v);
    v = v + dpp_move<kDppQuadXor2>(v);
    v = v + dpp_move<0x141>(v);  // row_half_mirror: lane i reads lane 7 - i of its half-row
    v = v + dpp_move<0x140>(v);  // row_mirror: lane i reads lane 15 - i of its row
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

// time_mixing_scratch steps 3-12 after the projections (model.rs:827-912) for one head of
// one stream; lane i owns channel c = 64 h + i and row i of the head's state.
__global__ __launch_bounds__(kHead) void k_rwkv_wkv(WkvArgs a) {
    __shared__ float sw[kHead], skka[kHead], snegkk[kHead], skmod[kHead], sr[kHead];
    const int i = threadIdx.x, h = blockIdx.x;
    const uint32_t b = blockIdx.y;
    const int d = a.d, c = h * kHead + i;
    const uint32_t slot = clamp_slot(a.slots[b], a.cap);
    const float* rkv = a.rkv + (size_t)b * 3 * d;
    const float* ld = a.lorad + (size_t)b * 4 * d;
    const float r = rkv[c], k = rkv[d + c], v = rkv[2 * d + c];
    const float lw = ld[c], la = ld[d + c], g = ld[2 * d + c], lv = ld[3 * d + c];
    const float vf = a.layer != 0 ? a.vfirst[(size_t)b * d + c] : 0.0f;
    // The head's state is stored [j / 4][i][4]: lane i's float4 q holds S[i][4q .. 4q + 3],
    // so each load and store of the wave is one contiguous 1 KB run.
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
    // Step 6: kk = (k * k_k) / |k * k_k| per head, 0 when the norm is <= 1e-12 (:1416-1424)
    const float kk0 = k * a.k_k[c];
    const float norm = sqrtf(wave_sum_rows(kk0 * kk0));
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
    // The two state dot products with four partial sums (column j into sum j % 4), added
    // (p0 + p1) + (p2 + p3): four short chains instead of one of 64.
    float tp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kHead; j++) tp[j % 4] += S[j] * snegkk[j];
    const float tt = (tp[0] + tp[1]) + (tp[2] + tp[3]);
#pragma unroll
    for (int j = 0; j < kHead; j++) S[j] = S[j] * sw[j] + tt * skka[j] + vout * skmod[j];
    float op[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kHead; j++) op[j % 4] += S[j] * sr[j];
    const float o = (op[0] + op[1]) + (op[2] + op[3]);
#pragma unroll
    for (int q = 0; q < kHead / 4; q++) sbase[q * kHead + i] = make_float4(S[4 * q], S[4 * q + 1], S[4 * q + 2], S[4 * q + 3]);
    // Step 10: GroupNorm over the head, eps 64e-5 (group_norm_into :1400-1414)
    const float mean = wave_sum_rows(o) / (float)kHead;
    const float var = wave_sum_rows((o - mean) * (o - mean)) / (float)kHead;
    float on = (o - mean) * (1.0f / sqrtf(var + 64e-5f)) * a.ln_x_w[c] + a.ln_x_b[c];
    // Step 11: bonus = sum over the head of r * k * r_k (k_mod for g1k models), times v_out
    const float ksrc = a.g1k ? kmod : k;
    on += wave_sum_rows(r * ksrc * a.r_k[c]) * vout;
    // Step 12: gate; the output projection follows as a matrix-core product
    write_limb1(a.gated, a.ks, b, c, on * g);
}

// ---------------------------------------------------------------- step assembly

struct ProjBuilder {
    ProjArgs a{};
    int tiles = 0;   // workgroups along x
    int tt = 1;      // row tiles per workgroup
    explicit ProjBuilder(int tiles_per_wg = 1) : tt(tiles_per_wg) {}
    void add(const TMat& w, const __bf16* in, int mode, int act, float* out, int ld, __bf16* lout, int lks) {
        ProjSeg& s = a.seg[a.nseg++];
        s.w = w;
        s.in = in;
        s.mode = mode;
        s.act = act;
        s.out = out;
        s.ld = ld;
        s.lout = lout;
        s.lks = lks;
        s.tile0 = tiles;
        tiles += (w.rt + tt - 1) / tt;
    }
    Launch launch(uint32_t n) {
        a.n = n;
        const void* f = tt == 4 ? (const void*)k_proj_t<4> : tt == 2 ? (const void*)k_proj_t<2> : (const void*)k_proj;
        return Launch::make(f, dim3(tiles, (n + kRowTile - 1) / kRowTile), dim3(kProjWaves * kWave), 0, KC_PROJ, a);
    }
};

}  // namespace

void RwkvStep::build(Pool& pool, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const {
    if (m.exact) {
        build_ref(pool, io, out, io_i, head_i, sm_i);
        return;
    }
    if (m.a8) {
        build_a8(pool, io, out, io_i, head_i, sm_i);
        return;
    }
    const RDims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d;
    const RwkvSizes z = rwkv_sizes(D, pool.cap, false);
    // The scratch of this part of the step (rows from b0, a multiple of 16): every per-row
    // array offset by b0 rows, every limb buffer by b0 / 16 groups; the recurrent state is
    // indexed by slot and stays whole.
    const size_t b0 = io.b0, g0 = b0 / kRowTile, limb_group = 3 * 512;
    Pool p = pool;
    p.x = pool.x + b0 * d;
    p.rkv = pool.rkv + b0 * 3 * d;
    p.lorad = pool.lorad + b0 * 4 * d;
    p.vfirst = pool.vfirst + b0 * d;
    p.slots = pool.slots + b0;
    p.gatedl = pool.gatedl + g0 * z.ks_d * limb_group;
    p.ffnl = pool.ffnl + g0 * z.ks_d * limb_group;
    p.headl = pool.headl + g0 * z.ks_d * limb_group;
    p.actl = pool.actl + g0 * z.ks_f * limb_group;
    out.clear();
    io_i = (int)out.size();
    out.push_back(embed_launch(*m.emb, p, io, nullptr, nullptr, nullptr, 0, 0));
    __bf16* mixl[6];
    for (int k = 0; k < 6; k++) mixl[k] = pool.mixl + k * z.mixl + g0 * z.ks_d * limb_group;
    __bf16* loral[4];
    for (int k = 0; k < 4; k++) loral[k] = pool.loral + z.lora_off[k] + g0 * z.ks_lora[k] * limb_group;
    const size_t state_stride = (size_t)D.nl * D.d;
    const size_t wkv_layer = (size_t)D.h * D.n * D.n;
    const int tt = proj_tiles_for(n, io.n_all ? io.n_all : n);
    for (uint32_t l = 0; l < D.nl; l++) {
        const RLayer& L = m.layers[l];
        ShiftArgs s1{p.x, L.ln1_w, L.ln1_b, p.x_att + (size_t)l * d, state_stride, p.slots, p.scap, 6, {}, {}, z.ks_d, d};
        for (int k = 0; k < 6; k++) {
            s1.mix[k] = L.mix[k];
            s1.out[k] = mixl[k];
        }
        out.push_back(Launch::make(shift_fn(s1.nmix), dim3(n), dim3(kBlock), 0, KC_SHIFT, s1));
        // receptance <- x_r, key <- x_k, value <- x_v; LoRA inputs x_w, x_a, x_g, x_v
        ProjBuilder p1(tt);
        p1.add(L.r, mixl[0], PROJ_STORE, ACT_NONE, p.rkv, 3 * d, nullptr, 0);
        p1.add(L.k, mixl[2], PROJ_STORE, ACT_NONE, p.rkv + d, 3 * d, nullptr, 0);
        p1.add(L.v, mixl[3], PROJ_STORE, ACT_NONE, p.rkv + 2 * d, 3 * d, nullptr, 0);
        p1.add(L.l1[kLoraW], mixl[1], PROJ_LIMBS, ACT_TANH, nullptr, 0, loral[kLoraW], z.ks_lora[kLoraW]);
        p1.add(L.l1[kLoraA], mixl[4], PROJ_LIMBS, ACT_NONE, nullptr, 0, loral[kLoraA], z.ks_lora[kLoraA]);
        p1.add(L.l1[kLoraG], mixl[5], PROJ_LIMBS, ACT_SIGMOID, nullptr, 0, loral[kLoraG], z.ks_lora[kLoraG]);
        if (l != 0) p1.add(L.l1[kLoraV], mixl[3], PROJ_LIMBS, ACT_NONE, nullptr, 0, loral[kLoraV], z.ks_lora[kLoraV]);
        out.push_back(p1.launch(n));
        ProjBuilder p2(tt);
        for (int k = 0; k < 4; k++)
            if (k != kLoraV || l != 0) p2.add(L.l2[k], loral[k], PROJ_STORE, ACT_NONE, p.lorad + k * d, 4 * d, nullptr, 0);
        out.push_back(p2.launch(n));
        WkvArgs wa{p.rkv, p.lorad, L.w0, L.a0, L.v0, L.k_k, L.k_a, L.r_k, L.ln_x_w, L.ln_x_b,
                   p.wkv + l * wkv_layer, (size_t)D.nl * wkv_layer, p.vfirst, p.slots, p.scap, p.gatedl, z.ks_d, d,
                   (int)l, (int)D.g1k};
        out.push_back(Launch::make((const void*)k_rwkv_wkv, dim3(D.h, n), dim3(kHead), 0, KC_WKV, wa));
        ProjBuilder po(tt);
        po.add(L.o, p.gatedl, PROJ_RESID, ACT_NONE, p.x, d, nullptr, 0);
        out.push_back(po.launch(n));
        ShiftArgs s2{p.x, L.ln2_w, L.ln2_b, p.x_ffn + (size_t)l * d, state_stride, p.slots, p.scap, 1, {}, {}, z.ks_d, d};
        s2.mix[0] = L.ffn_x_k;
        s2.out[0] = p.ffnl;
        out.push_back(Launch::make(shift_fn(s2.nmix), dim3(n), dim3(kBlock), 0, KC_SHIFT, s2));
        ProjBuilder pk(tt);
        pk.add(L.fk, p.ffnl, PROJ_LIMBS, ACT_RELU2, nullptr, 0, p.actl, z.ks_f);
        out.push_back(pk.launch(n));
        ProjBuilder pv(tt);
        pv.add(L.fv, p.actl, PROJ_RESID, ACT_NONE, p.x, d, nullptr, 0);
        out.push_back(pv.launch(n));
    }
    const TMat& H = *m.head;
    const bool ws = H.group != 0 && H.group == H.cols && H.ks / 2 <= 12;
    if (ws) {
        ShiftArgs sf{p.x, m.ln_out_w, m.ln_out_b, nullptr, 0, p.slots, p.scap, 0, {}, {}, z.ks_d, d};
        sf.out[0] = p.headl;
        out.push_back(Launch::make(shift_fn(sf.nmix), dim3(n), dim3(kBlock), 0, KC_SHIFT, sf));
    }
    head_i = (int)out.size();
    out.push_back(head_launch(H, p, io, p.x, m.ln_out_w, m.ln_out_b, ws ? p.headl : nullptr, nullptr, d, 0, ws));
    sm_i = -1;
    if (io.probs) {
        sm_i = (int)out.size();
        out.push_back(softmax_launch(io.out + b0 * D.vocab, (int)D.vocab, n));
    }
}

}  // namespace rdk
