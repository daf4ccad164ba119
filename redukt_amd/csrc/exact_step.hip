// exact_step.hip — the Mamba step in the reference CPU path's own arithmetic: the
// reference-order tier.
//
// Weight profile bit 6 selects it with numeric contract 1 (the reference's "Plain" kernel
// family: every product and every sum rounded on its own), bit 7 with numeric contract 2
// (fma-v1, src/domain/gemv_fma.rs:1-26: every acc + w * x of a GEMV one fused
// multiply-add).  Every projection output (row r, stream b) is the reference GEMV of that
// row, f32_rows / q8w_rows (src/domain/gemv.rs:181-194, 459-502) or their contract-2
// twins (gemv_fma.rs:98-134): eight accumulators by column residue from +0 over the
// 8-aligned body in column order, the horizontal sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7))
// (the tail is empty: every matrix here has whole 32-column blocks); Q8 rows fold
// dot_g * scale_g over the column groups from +0.  Eight lanes compute one output, lane l
// holding the reference's accumulator l, so nothing depends on the launch shape, the batch
// or the slot.  The norms are the reference's sequential sums (rms_norm_into,
// layer_norm_into: src/domain/tensor.rs:900-908, 1390-1398), the scan takes the portable exp, and the
// element-wise code (conv, SiLU, softplus, the d16 recurrence, the gate, softmax) is the
// other tiers', already the CPU path's bit for bit; so the logits are the CPU path's
// logits.  Per layer:
//   k_norm_e  : the layer's RMSNorm (LayerNorm with a bias) of the residual stream;
//   k_gemv_e  : in_proj, then conv1d + SiLU (conv_silu_block order) on the conv-branch rows;
//   k_gemv_e  : x_proj, each stream's complete outputs;
//   k_scan    : shared with the other tiers (dt_proj in the contract's order);
//   k_gemv_e  : out_proj and the residual add;
// and per step k_embed_e (row gather or Q8 dequantisation, device argument check), the
// final norm, the head, and optionally the shared softmax.  exact_gemv_launch hands the same
// F32 projection to the RWKV-7 step of this tier (rwkv_a8.hip).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "mfma_common.h"
#include "model.h"
#include "portable_math.h"
#include "step.h"

#pragma clang fp contract(off)

namespace rdk {

namespace {

constexpr int kEBlock = 256;      // threads (outputs) per workgroup
constexpr int kNormMax = 1024;    // d_model limit of the loader

// A RowMat stores each row in 32-column blocks interleaved by column residue: column c of
// row r at r cols + 32 (c / 32) + 4 (c % 8) + (c % 32) / 8, so lane l of an output's eight
// lanes finds its four columns of a block (l, l + 8, l + 16, l + 24) in one 16-byte (F32) or
// 4-byte (Q8) run, and the eight lanes read the block's 32 columns contiguously.
__device__ __forceinline__ size_t rowmat_index(size_t row_off, int c) {
    return row_off + (size_t)(c & ~31) + (size_t)(4 * (c & 7) + ((c & 31) >> 3));
}

// ---------------------------------------------------------------- embedding

struct EmbedEArgs {
    RowMat emb;
    float* x;
    const uint32_t* tokens;
    const uint32_t* slots_in;
    uint32_t* slots;
    uint32_t n, cap;
    int check;
    uint32_t* err;
};

// x[b] = emb[token[b]]: the row as stored (F32) or q * scale of its group (MambaMatrix::
// row_into, model.rs:93-101; Q8wMatrix::dequant_row_into, gemv.rs:285-295).  Block b also
// checks its entry (check_entry).
__global__ __launch_bounds__(kEBlock) void k_embed_e(EmbedEArgs a) {
    const uint32_t b = blockIdx.x;
    const RowMat& e = a.emb;
    uint32_t tok = a.tokens[b];
    check_entry(a.slots_in, a.slots, a.n, b, tok < (uint32_t)e.rows, a.cap, a.check, a.err);
    if (tok >= (uint32_t)e.rows) tok = e.rows - 1;
    const int cols = e.cols;
    float* xo = a.x + (size_t)b * cols;
    const size_t row_off = (size_t)tok * cols;
    if (e.group == 0) {
        for (int c = threadIdx.x; c < cols; c += kEBlock) xo[c] = ((const float*)e.w)[rowmat_index(row_off, c)];
    } else {
        const float* sc = e.scales + (size_t)tok * (cols / e.group);
        for (int c = threadIdx.x; c < cols; c += kEBlock)
            xo[c] = (float)((const int8_t*)e.w)[rowmat_index(row_off, c)] * sc[c / e.group];
    }
}

// ---------------------------------------------------------------- norms

struct NormEArgs {
    const float* x;     // [n][d]
    const float* w;
    const float* bias;  // LayerNorm bias, or null for RMSNorm
    float* out;         // [n][d]
    int d;
};

// One stream per workgroup: the row through LDS, the sums by one thread in index order
// (the reference's sequential loops), the scale to every thread, then the element-wise
// output.  RMSNorm (tensor.rs:900-908): inv = 1 / sqrt(sum(x^2) / d + 1e-5),
// out = x * inv * w.  LayerNorm (tensor.rs:1390-1398, two passes): mean = sum(x) / d,
// var = sum((x - mean)^2) / d, out = (x - mean) * (1 / sqrt(var + 1e-5)) * w + b.
// The sequential sum of t[0 .. d) (d a multiple of 4) by one thread, in index order: the
// reads go ahead in float4s, only the adds form the chain.
__device__ __forceinline__ float seq_sum(const float* t, int d) {
    float s = 0.0f;
#pragma unroll 8
    for (int i = 0; i < d; i += 4) {
        const float4 v = *(const float4*)(t + i);
        s = s + v.x;
        s = s + v.y;
        s = s + v.z;
        s = s + v.w;
    }
    return s;
}

__global__ __launch_bounds__(kEBlock) void k_norm_e(NormEArgs a) {
    __shared__ __align__(16) float xs[kNormMax];
    __shared__ __align__(16) float tv[kNormMax];   // the terms of the sum in flight
    __shared__ float stat[2];
    const int d = a.d;
    const float* x = a.x + (size_t)blockIdx.x * d;
    for (int i = threadIdx.x; i < d; i += kEBlock) xs[i] = x[i];
    __syncthreads();
    if (a.bias == nullptr) {
        // each term x * x rounded on its own, as in ss += x * x
        for (int i = threadIdx.x; i < d; i += kEBlock) tv[i] = xs[i] * xs[i];
        __syncthreads();
        if (threadIdx.x == 0) {
            const float rms = sqrtf(seq_sum(tv, d) / (float)d + 1e-5f);
            stat[0] = 0.0f;
            stat[1] = 1.0f / rms;
        }
    } else {
        if (threadIdx.x == 0) stat[0] = seq_sum(xs, d) / (float)d;
        __syncthreads();
        const float mean = stat[0];
        for (int i = threadIdx.x; i < d; i += kEBlock) tv[i] = (xs[i] - mean) * (xs[i] - mean);
        __syncthreads();
        if (threadIdx.x == 0) stat[1] = 1.0f / sqrtf(seq_sum(tv, d) / (float)d + 1e-5f);
    }
    __syncthreads();
    float* o = a.out + (size_t)blockIdx.x * d;
    if (a.bias == nullptr) {
        const float inv = stat[1];
        for (int i = threadIdx.x; i < d; i += kEBlock) o[i] = xs[i] * inv * a.w[i];
    } else {
        const float mean = stat[0], inv = stat[1];
        for (int i = threadIdx.x; i < d; i += kEBlock) o[i] = (xs[i] - mean) * inv * a.w[i] + a.bias[i];
    }
}

// ---------------------------------------------------------------- projections

enum : int { kEpiPlain = EXACT_STORE, kEpiIn = 1, kEpiRes = EXACT_RESID, kEpiRelu2 = EXACT_RELU2 };

struct GemvEArgs {
    RowMat w;               // [rows][cols]
    const float* act;       // [n][cols] input rows
    uint32_t n;
    float* out;             // kEpiPlain, kEpiRelu2: out[b * ostride + r]; kEpiRes: the residual x [n][rows]
    uint32_t ostride;
    // kEpiIn: rows below di are the conv branch (conv1d + SiLU into u, the conv state
    // updated), the rest the gate branch (z).
    float* conv_st;         // this layer's conv state [slot][di][3]
    const float* conv_w;    // [di][4]
    const float* conv_b;
    const uint32_t* slots;
    uint32_t scap;
    float* u;
    float* z;
    int di;
    // Products 1 and 2 of a launch of three of one shape (grid z; product 0 is w, act,
    // out): rows w_more[z - 1], input rows act_more[z - 1], outputs from out + out_more[z - 1].
    RowMat w_more[2];
    const float* act_more[2];
    uint32_t out_more[2];
};

// acc + w * x in the contract's arithmetic.
template <bool FMA>
__device__ __forceinline__ float madd(float w, float x, float acc) {
    return FMA ? __builtin_fmaf(w, x, acc) : acc + w * x;
}

// Lane l's four weights of the 32-column block at column c0, as exact f32.
template <bool Q8>
__device__ __forceinline__ void load4(const RowMat& m, size_t row_off, int c0, int l, float (&w)[4]) {
    const size_t at = row_off + (size_t)c0 + 4 * l;
    if (Q8) {
        const uint32_t q = *(const uint32_t*)((const int8_t*)m.w + at);
#pragma unroll
        for (int j = 0; j < 4; j++) w[j] = (float)(int8_t)(q >> (8 * j));
    } else {
        const float4 v = *(const float4*)((const float*)m.w + at);
        w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
    }
}

// Eight lanes compute one output (row, S streams): lane l holds accumulator l of the
// reference's eight, the columns c = l (mod 8) of each column group in order from +0; the
// horizontal sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) is formed in lane 0 of the eight
// by three DPP adds (hsum8_lane0); Q8 rows then take sum = sum + dot * scale from +0.
// Workgroup (bx, by) holds rows [32 bx, 32 bx + 32) and streams [S by, S by + S), the streams' input rows
// staged in LDS.  Every operation in the contract's arithmetic (madd).  Column counts and
// groups are whole 32-column blocks (checked at load).
// NB > 0: the rows have exactly NB 32-column blocks, and each lane requests its whole
// slice of the row (NB 4-byte int8 or 16-byte F32 runs) before the first product: a
// matrix with few rows has few lanes, so each lane keeps many loads in flight.
template <bool Q8, bool FMA, int S, int EPI, int NB>
__global__ __launch_bounds__(kEBlock) void k_gemv_e(GemvEArgs a) {
    extern __shared__ __align__(16) float acts[];   // [S][cols], 32-column blocks interleaved like the rows
    const uint32_t z = blockIdx.z;
    const RowMat& m = z == 0 ? a.w : z == 1 ? a.w_more[0] : a.w_more[1];
    const float* const act = z == 0 ? a.act : z == 1 ? a.act_more[0] : a.act_more[1];
    float* const out = z == 0 ? a.out : a.out + (z == 1 ? a.out_more[0] : a.out_more[1]);
    const int cols = m.cols;
    const uint32_t b0 = blockIdx.y * S;
    for (int s = 0; s < S; s++) {
        const uint32_t b = min(b0 + (uint32_t)s, a.n - 1);
        const float* src = act + (size_t)b * cols;
        for (int c = threadIdx.x; c < cols; c += kEBlock) acts[rowmat_index((size_t)s * cols, c)] = src[c];
    }
    __syncthreads();
    const int l = (int)threadIdx.x % 8;
    const int r_raw = (int)blockIdx.x * (kEBlock / 8) + (int)threadIdx.x / 8;
    const bool live = r_raw < m.rows;
    const int r = live ? r_raw : m.rows - 1;   // every lane joins the horizontal sums
    const size_t row_off = (size_t)r * cols;
    const int group = Q8 ? m.group : cols;
    const int ng = cols / group;
    float res[S];
#pragma unroll
    for (int s = 0; s < S; s++) res[s] = 0.0f;
    // The eight lanes' horizontal sum of each stream's accumulator, then the group's fold
    // (both complete in lane 0 of the eight, the lane that stores).
    auto finish_group = [&](float (&acc)[S], int g) {
#pragma unroll
        for (int s = 0; s < S; s++) {
            const float v = hsum8_lane0(acc[s]);
            res[s] = Q8 ? madd<FMA>(v, m.scales[(size_t)r * ng + g], res[s]) : v;
            acc[s] = 0.0f;
        }
    };
    if constexpr (NB > 0) {
        typedef typename std::conditional<Q8, uint32_t, float4>::type Raw;
        Raw raw[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const size_t at = row_off + 32 * (size_t)i + 4 * l;
            if constexpr (Q8)
                raw[i] = *(const uint32_t*)((const int8_t*)m.w + at);
            else
                raw[i] = *(const float4*)((const float*)m.w + at);
        }
        const int bpg = group / 32;
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; s++) acc[s] = 0.0f;
        int g = 0;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            float w[4];
            if constexpr (Q8) {
#pragma unroll
                for (int j = 0; j < 4; j++) w[j] = (float)(int8_t)(raw[i] >> (8 * j));
            } else {
                w[0] = raw[i].x, w[1] = raw[i].y, w[2] = raw[i].z, w[3] = raw[i].w;
            }
#pragma unroll
            for (int s = 0; s < S; s++) {
                const float4 x = *(const float4*)(acts + (size_t)s * cols + 32 * i + 4 * l);
                acc[s] = madd<FMA>(w[0], x.x, acc[s]);
                acc[s] = madd<FMA>(w[1], x.y, acc[s]);
                acc[s] = madd<FMA>(w[2], x.z, acc[s]);
                acc[s] = madd<FMA>(w[3], x.w, acc[s]);
            }
            if ((i + 1) % bpg == 0) finish_group(acc, g++);
        }
    } else
    for (int g = 0; g < ng; g++) {
        const int c0 = g * group;
        float acc[S];
#pragma unroll
        for (int s = 0; s < S; s++) acc[s] = 0.0f;
#pragma unroll 4
        for (int c = c0; c < c0 + group; c += 32) {
            float w[4];
            load4<Q8>(m, row_off, c, l, w);
#pragma unroll
            for (int s = 0; s < S; s++) {
                const float4 x = *(const float4*)(acts + (size_t)s * cols + c + 4 * l);
                acc[s] = madd<FMA>(w[0], x.x, acc[s]);
                acc[s] = madd<FMA>(w[1], x.y, acc[s]);
                acc[s] = madd<FMA>(w[2], x.z, acc[s]);
                acc[s] = madd<FMA>(w[3], x.w, acc[s]);
            }
        }
        finish_group(acc, g);
    }
    if (!live || l != 0) return;
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint32_t b = b0 + (uint32_t)s;
        if (b >= a.n) break;
        const float y = res[s];
        if (EPI == kEpiPlain) {
            out[(size_t)b * a.ostride + r] = y;
        } else if (EPI == kEpiRes) {
            // x += W_out * gated (model.rs:714-719): the residual add after the projection
            float* xp = out + (size_t)b * a.ostride + r;
            *xp = *xp + y;
        } else if (EPI == kEpiRelu2) {
            // squared_relu_into (tensor.rs:1386-1388): max(y, 0)^2, a NaN to 0
            const float t = y > 0.0f ? y : 0.0f;
            out[(size_t)b * a.ostride + r] = t * t;
        } else if (r >= a.di) {
            a.z[(size_t)b * a.di + (r - a.di)] = y;
        } else {
            // conv_silu_block (model.rs:134-153) for channel r of stream b, then SiLU with the
            // lane sigmoid: d_inner comes in whole 64-channel blocks, so every channel is in
            // the 8-aligned body of its 256-channel block (tensor.rs:1197-1211).
            const uint32_t slot = clamp_slot(a.slots[b], a.scap);
            float* st = a.conv_st + ((size_t)slot * a.di + r) * 3;
            const float4 cw = *(const float4*)(a.conv_w + (size_t)r * 4);
            const float s0 = st[0], s1 = st[1], s2 = st[2];
            float val = 0.0f;
            val += s0 * cw.x;
            val += s1 * cw.y;
            val += s2 * cw.z;
            val += y * cw.w;
            val += a.conv_b[r];
            st[0] = s1;
            st[1] = s2;
            st[2] = y;
            a.u[(size_t)b * a.di + r] = val * lane_sigmoid_f(val);
        }
    }
}

template <int S, int EPI, int NB>
const void* gemv_e_fn(bool q8, bool fma) {
    if (q8) return fma ? (const void*)k_gemv_e<true, true, S, EPI, NB> : (const void*)k_gemv_e<true, false, S, EPI, NB>;
    return fma ? (const void*)k_gemv_e<false, true, S, EPI, NB> : (const void*)k_gemv_e<false, false, S, EPI, NB>;
}

// The row slice in flight whole for Mamba-130M's widths (768 and 1536 columns), the
// generic loop for the others and for F32 batches (a whole F32 slice of 1536 columns
// takes 200 registers: two waves per SIMD, slower from a few streams on).
template <int S, int EPI>
const void* gemv_e_nb(int cols, bool q8, bool fma) {
    if (!q8 && S > 1) return gemv_e_fn<S, EPI, 0>(q8, fma);
    if (cols == 768) return gemv_e_fn<S, EPI, 24>(q8, fma);
    if (cols == 1536) return gemv_e_fn<S, EPI, 48>(q8, fma);
    return gemv_e_fn<S, EPI, 0>(q8, fma);
}

template <int EPI>
const void* gemv_e_pick(uint32_t s, int cols, bool q8, bool fma) {
    if (s == 8) return gemv_e_nb<8, EPI>(cols, q8, fma);
    return s == 1 ? gemv_e_nb<1, EPI>(cols, q8, fma) : gemv_e_nb<4, EPI>(cols, q8, fma);
}

// Streams per workgroup: one for a single stream, four otherwise (their input rows in LDS:
// 4 x d_inner floats at most 32 KB; sixteen, reading each row once per 16 streams, leave
// too few workgroups: 32 streams 1.78 -> 2.38 ms per step; eight at 64 and 128 streams
// double the out_proj time).  The head, with 50K rows, takes eight from 16 streams on
// (its weights read half as often: Mamba-130M F32 at 128 streams 643 -> 422 us; sixteen
// 597 us).  A stream's arithmetic does not depend on it.
uint32_t exact_streams(uint32_t n) { return n == 1 ? 1u : 4u; }
constexpr uint32_t kHeadStreams = 8;

Launch gemv_e_launch(const void* (*pick)(uint32_t, int, bool, bool), bool fma, int cls, const RowMat& w,
                     const float* act, uint32_t n, GemvEArgs a, uint32_t s_wide = 0, uint32_t products = 1) {
    // s_wide streams per workgroup once the batch fills two such workgroups
    const uint32_t S = s_wide && n >= 2 * s_wide ? s_wide : exact_streams(n);
    const void* fn = pick(S, w.cols, w.group != 0, fma);
    a.w = w;
    a.act = act;
    a.n = n;
    const uint32_t lds = S * (uint32_t)w.cols * 4u;
    constexpr int rows_per_wg = kEBlock / 8;
    return Launch::make(fn, dim3((unsigned)((w.rows + rows_per_wg - 1) / rows_per_wg), (n + S - 1) / S, products),
                        dim3(kEBlock), lds, (uint32_t)cls, a);
}

}  // namespace

Launch exact_gemv_launch(const RowMat& w, const float* act, uint32_t n, float* out, uint32_t ostride, int epi,
                         uint32_t cls) {
    GemvEArgs a{};
    a.out = out;
    a.ostride = ostride;
    const void* (*pick)(uint32_t, int, bool, bool) = epi == EXACT_RESID   ? gemv_e_pick<kEpiRes>
                                                      : epi == EXACT_RELU2 ? gemv_e_pick<kEpiRelu2>
                                                                           : gemv_e_pick<kEpiPlain>;
    return gemv_e_launch(pick, false, (int)cls, w, act, n, a, cls == KC_HEAD ? kHeadStreams : 0);
}

Launch exact_gemv3_launch(const RowMat* const (&w)[3], const float* const (&act)[3], uint32_t n, float* out,
                          const uint32_t (&out_off)[3], uint32_t ostride, uint32_t cls) {
    GemvEArgs a{};
    a.out = out + out_off[0];
    a.ostride = ostride;
    for (int k = 0; k < 2; k++) {
        a.w_more[k] = *w[k + 1];
        a.act_more[k] = act[k + 1];
        a.out_more[k] = out_off[k + 1] - out_off[0];
    }
    return gemv_e_launch(gemv_e_pick<kEpiPlain>, false, (int)cls, *w[0], act[0], n, a, 0, 3);
}

void ExactStep::build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const {
    const Dims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d, di = (int)D.di;
    const bool fma = m.fma;
    out.clear();
    io_i = (int)out.size();
    EmbedEArgs ea{*m.emb, p.x, io.tokens, io.slots, p.slots, n, p.cap, io.check ? 1 : 0, io.err};
    out.push_back(Launch::make((const void*)k_embed_e, dim3(n), dim3(kEBlock), 0, KC_EMBED, ea));
    const size_t conv_layer = (size_t)p.scap * di * (D.dc - 1);
    const size_t ssm_layer = (size_t)p.scap * di * 16;
    const uint32_t xr_pad = (uint32_t)(m.layers[0].x_proj.rt * kRowTile);
    for (uint32_t li = 0; li < D.nl; li++) {
        const DLayer& L = m.layers[li];
        out.push_back(Launch::make((const void*)k_norm_e, dim3(n), dim3(kEBlock), 0, KC_NORM,
                                   NormEArgs{p.x, L.norm_w, L.norm_b, p.normed, d}));
        GemvEArgs gi{};
        gi.conv_st = p.conv + li * conv_layer;
        gi.conv_w = L.conv_w;
        gi.conv_b = L.conv_b;
        gi.slots = p.slots;
        gi.scap = p.scap;
        gi.u = p.u;
        gi.z = p.z;
        gi.di = di;
        out.push_back(gemv_e_launch(gemv_e_pick<kEpiIn>, fma, KC_MIX_IN, L.e_in, p.normed, n, gi));
        GemvEArgs gx{};
        gx.out = p.xpart;
        gx.ostride = xr_pad;
        out.push_back(gemv_e_launch(gemv_e_pick<kEpiPlain>, fma, KC_XPROJ, L.e_xp, p.u, n, gx));
        out.push_back(scan_exact_launch(L, D, p, n, fma, p.g32, p.ssm + li * ssm_layer));
        GemvEArgs go{};
        go.out = p.x;
        go.ostride = (uint32_t)d;
        out.push_back(gemv_e_launch(gemv_e_pick<kEpiRes>, fma, KC_MIX_OUT, L.e_out, p.g32, n, go));
    }
    out.push_back(Launch::make((const void*)k_norm_e, dim3(n), dim3(kEBlock), 0, KC_NORM,
                               NormEArgs{p.x, m.norm_f_w, m.norm_f_b, p.normed, d}));
    head_i = (int)out.size();
    GemvEArgs gh{};
    gh.out = io.out;
    gh.ostride = D.vocab;
    out.push_back(gemv_e_launch(gemv_e_pick<kEpiPlain>, fma, KC_HEAD, *m.head, p.normed, n, gh, kHeadStreams));
    sm_i = -1;
    if (io.probs) {
        sm_i = (int)out.size();
        out.push_back(softmax_launch(io.out, (int)D.vocab, n));
    }
}

}  // namespace rdk
