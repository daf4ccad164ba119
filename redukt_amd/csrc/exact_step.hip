// exact_step.hip — the Mamba step in the reference CPU path's own arithmetic: the
// reference-order tier.
//
// Weight profile bit 6 selects it with numeric contract 1 (the reference's "Plain" kernel
// family: every product and every sum rounded on its own), bit 7 with numeric contract 2
// (fma-v1, src/domain/gemv_fma.rs:1-26: every acc + w * x of a GEMV one fused
// multiply-add).  Every projection output (row r, stream b) is the reference GEMV of that
// row, f32_rows / q8w_rows (src/domain/gemv.rs:181-194, 459-502) or their contract-2
// twins (gemv_fma.rs:98-134): eight accumulators by column residue from +0 over the
// 8-aligned body in column order, the horizontal sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)),
// then the sequential tail; Q8 rows fold dot_g * scale_g over the column groups from +0.
// One thread computes one output, so nothing depends on the launch shape, the batch or the
// slot.  The norms are the reference's sequential sums (rms_norm_into, layer_norm_into:
// src/domain/tensor.rs:900-908, 1390-1398), the scan takes the portable exp, and the
// element-wise code (conv, SiLU, softplus, the d16 recurrence, the gate, softmax) is the
// other tiers', already the CPU path's bit for bit; so the logits are the CPU path's
// logits.  Per layer:
//   k_norm_e  : the layer's RMSNorm (LayerNorm with a bias) of the residual stream;
//   k_gemv_e  : in_proj, then conv1d + SiLU (conv_silu_block order) on the conv-branch rows;
//   k_gemv_e  : x_proj, each stream's complete outputs;
//   k_scan    : shared with the other tiers (dt_proj in the contract's order);
//   k_gemv_e  : out_proj and the residual add;
// and per step k_embed_e (row gather or Q8 dequantisation, device argument check), the
// final norm, the head, and optionally the shared softmax.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "mfma_common.h"
#include "model.h"
#include "portable_math.h"
#include "step.h"

#pragma clang fp contract(off)

namespace rdk {

namespace {

constexpr int kEBlock = 256;      // threads (outputs) per workgroup
constexpr int kNormMax = 1024;    // d_model limit of the loader

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
    if (e.group == 0) {
        const float* row = (const float*)e.w + (size_t)tok * cols;
        for (int c = threadIdx.x; c < cols; c += kEBlock) xo[c] = row[c];
    } else {
        const int8_t* row = (const int8_t*)e.w + (size_t)tok * cols;
        const float* sc = e.scales + (size_t)tok * (cols / e.group);
        for (int c = threadIdx.x; c < cols; c += kEBlock) xo[c] = (float)row[c] * sc[c / e.group];
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
__global__ __launch_bounds__(kEBlock) void k_norm_e(NormEArgs a) {
    __shared__ float xs[kNormMax];
    __shared__ float stat[2];
    const int d = a.d;
    const float* x = a.x + (size_t)blockIdx.x * d;
    for (int i = threadIdx.x; i < d; i += kEBlock) xs[i] = x[i];
    __syncthreads();
    if (threadIdx.x == 0) {
        if (a.bias == nullptr) {
            float ss = 0.0f;
            for (int i = 0; i < d; i++) ss += xs[i] * xs[i];
            const float rms = sqrtf(ss / (float)d + 1e-5f);
            stat[0] = 0.0f;
            stat[1] = 1.0f / rms;
        } else {
            float sum = 0.0f;
            for (int i = 0; i < d; i++) sum += xs[i];
            const float mean = sum / (float)d;
            float vs = 0.0f;
            for (int i = 0; i < d; i++) vs += (xs[i] - mean) * (xs[i] - mean);
            const float var = vs / (float)d;
            stat[0] = mean;
            stat[1] = 1.0f / sqrtf(var + 1e-5f);
        }
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

enum : int { kEpiPlain = 0, kEpiIn = 1, kEpiRes = 2 };

struct GemvEArgs {
    RowMat w;               // [rows][cols]
    const float* act;       // [n][cols] input rows
    uint32_t n;
    float* out;             // kEpiPlain: out[b * ostride + r]; kEpiRes: the residual x [n][rows]
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
};

// acc + w * x in the contract's arithmetic.
template <bool FMA>
__device__ __forceinline__ float madd(float w, float x, float acc) {
    return FMA ? __builtin_fmaf(w, x, acc) : acc + w * x;
}

// Eight weights of row `row` from column c (c a multiple of 8): F32 as stored, Q8 as the
// exact f32 of each int8.
template <bool Q8>
__device__ __forceinline__ void load8(const RowMat& m, size_t row_off, int c, float (&w)[8]) {
    if (Q8) {
        const uint2 q = *(const uint2*)((const int8_t*)m.w + row_off + c);
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = (float)(int8_t)((i < 4 ? q.x : q.y) >> (8 * (i % 4)));
    } else {
        const float4* p = (const float4*)((const float*)m.w + row_off + c);
        const float4 lo = p[0], hi = p[1];
        w[0] = lo.x, w[1] = lo.y, w[2] = lo.z, w[3] = lo.w;
        w[4] = hi.x, w[5] = hi.y, w[6] = hi.z, w[7] = hi.w;
    }
}

template <bool Q8>
__device__ __forceinline__ float load1(const RowMat& m, size_t row_off, int c) {
    return Q8 ? (float)((const int8_t*)m.w)[row_off + c] : ((const float*)m.w)[row_off + c];
}

// Thread t of workgroup (bx, by) computes row bx * kEBlock + t for streams [S by, S by + S);
// the streams' input rows are staged in LDS (every thread reads the same words).  Per
// (row, stream), over each column group in order (F32: the whole row, one group without a
// scale): eight accumulators over the group's 8-aligned body, the fixed horizontal sum,
// the sequential tail; Q8: sum = sum + dot * scale from +0.  Every operation in the
// contract's arithmetic (madd), every add and product of contract 1 rounded on its own.
template <bool Q8, bool FMA, int S, int EPI>
__global__ __launch_bounds__(kEBlock) void k_gemv_e(GemvEArgs a) {
    extern __shared__ float acts[];   // [S][cols]
    const RowMat& m = a.w;
    const int cols = m.cols;
    const uint32_t b0 = blockIdx.y * S;
    for (int s = 0; s < S; s++) {
        const uint32_t b = min(b0 + (uint32_t)s, a.n - 1);
        const float* src = a.act + (size_t)b * cols;
        for (int c = threadIdx.x; c < cols; c += kEBlock) acts[s * cols + c] = src[c];
    }
    __syncthreads();
    const int r = (int)blockIdx.x * kEBlock + (int)threadIdx.x;
    if (r >= m.rows) return;
    const size_t row_off = (size_t)r * cols;
    const int group = Q8 ? m.group : cols;
    const int ng = cols / group;
    const int body = group / 8 * 8;
    float res[S];
#pragma unroll
    for (int s = 0; s < S; s++) res[s] = 0.0f;
    for (int g = 0; g < ng; g++) {
        const int c0 = g * group;
        float acc[S][8];
#pragma unroll
        for (int s = 0; s < S; s++)
#pragma unroll
            for (int l = 0; l < 8; l++) acc[s][l] = 0.0f;
#pragma unroll 4
        for (int c = c0; c < c0 + body; c += 8) {
            float w[8];
            load8<Q8>(m, row_off, c, w);
#pragma unroll
            for (int s = 0; s < S; s++) {
                const float4 x0 = *(const float4*)(acts + s * cols + c);
                const float4 x1 = *(const float4*)(acts + s * cols + c + 4);
                acc[s][0] = madd<FMA>(w[0], x0.x, acc[s][0]);
                acc[s][1] = madd<FMA>(w[1], x0.y, acc[s][1]);
                acc[s][2] = madd<FMA>(w[2], x0.z, acc[s][2]);
                acc[s][3] = madd<FMA>(w[3], x0.w, acc[s][3]);
                acc[s][4] = madd<FMA>(w[4], x1.x, acc[s][4]);
                acc[s][5] = madd<FMA>(w[5], x1.y, acc[s][5]);
                acc[s][6] = madd<FMA>(w[6], x1.z, acc[s][6]);
                acc[s][7] = madd<FMA>(w[7], x1.w, acc[s][7]);
            }
        }
#pragma unroll
        for (int s = 0; s < S; s++) {
            float dot = ((acc[s][0] + acc[s][4]) + (acc[s][2] + acc[s][6])) +
                        ((acc[s][1] + acc[s][5]) + (acc[s][3] + acc[s][7]));
            for (int c = c0 + body; c < c0 + group; c++) dot = madd<FMA>(load1<Q8>(m, row_off, c), acts[s * cols + c], dot);
            if (Q8)
                res[s] = madd<FMA>(dot, m.scales[(size_t)r * ng + g], res[s]);
            else
                res[s] = dot;
        }
    }
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint32_t b = b0 + (uint32_t)s;
        if (b >= a.n) break;
        const float y = res[s];
        if (EPI == kEpiPlain) {
            a.out[(size_t)b * a.ostride + r] = y;
        } else if (EPI == kEpiRes) {
            // x += W_out * gated (model.rs:714-719): the residual add after the projection
            float* xp = a.out + (size_t)b * a.ostride + r;
            *xp = *xp + y;
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

template <int S, int EPI>
const void* gemv_e_fn(bool q8, bool fma) {
    if (q8) return fma ? (const void*)k_gemv_e<true, true, S, EPI> : (const void*)k_gemv_e<true, false, S, EPI>;
    return fma ? (const void*)k_gemv_e<false, true, S, EPI> : (const void*)k_gemv_e<false, false, S, EPI>;
}

template <int EPI>
const void* gemv_e_pick(uint32_t s, bool q8, bool fma) {
    return s == 1 ? gemv_e_fn<1, EPI>(q8, fma) : gemv_e_fn<4, EPI>(q8, fma);
}

// Streams per workgroup: one for a single stream, four otherwise (their input rows in LDS:
// 4 x d_inner floats at most 32 KB).  A stream's arithmetic does not depend on it.
uint32_t exact_streams(uint32_t n) { return n == 1 ? 1u : 4u; }

Launch gemv_e_launch(const void* fn, int cls, const RowMat& w, const float* act, uint32_t n, uint32_t S, GemvEArgs a) {
    a.w = w;
    a.act = act;
    a.n = n;
    const uint32_t lds = S * (uint32_t)w.cols * 4u;
    return Launch::make(fn, dim3((unsigned)((w.rows + kEBlock - 1) / kEBlock), (n + S - 1) / S), dim3(kEBlock), lds,
                        (uint32_t)cls, a);
}

}  // namespace

void ExactStep::build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const {
    const Dims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d, di = (int)D.di;
    const uint32_t S = exact_streams(n);
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
        out.push_back(gemv_e_launch(gemv_e_pick<kEpiIn>(S, L.e_in.group != 0, fma), KC_MIX_IN, L.e_in, p.normed, n, S, gi));
        GemvEArgs gx{};
        gx.out = p.xpart;
        gx.ostride = xr_pad;
        out.push_back(gemv_e_launch(gemv_e_pick<kEpiPlain>(S, L.e_xp.group != 0, fma), KC_XPROJ, L.e_xp, p.u, n, S, gx));
        out.push_back(scan_exact_launch(L, D, p, n, fma, p.g32, p.ssm + li * ssm_layer));
        GemvEArgs go{};
        go.out = p.x;
        go.ostride = (uint32_t)d;
        out.push_back(gemv_e_launch(gemv_e_pick<kEpiRes>(S, L.e_out.group != 0, fma), KC_MIX_OUT, L.e_out, p.g32, n, S, go));
    }
    out.push_back(Launch::make((const void*)k_norm_e, dim3(n), dim3(kEBlock), 0, KC_NORM,
                               NormEArgs{p.x, m.norm_f_w, m.norm_f_b, p.normed, d}));
    head_i = (int)out.size();
    GemvEArgs gh{};
    gh.out = io.out;
    gh.ostride = D.vocab;
    out.push_back(gemv_e_launch(gemv_e_pick<kEpiPlain>(S, m.head->group != 0, fma), KC_HEAD, *m.head, p.normed, n, S, gh));
    sm_i = -1;
    if (io.probs) {
        sm_i = (int)out.size();
        out.push_back(softmax_launch(io.out, (int)D.vocab, n));
    }
}

}  // namespace rdk
