// mamba_kernels.hip — gfx950 kernels of one Mamba-1 token step for N lockstep streams.
//
// Determinism and batch invariance: every output element is produced by exactly one
// lane with a fixed operation sequence — a fixed per-lane accumulation order and a
// fixed xor-butterfly tree across the 64 lanes of a wavefront, read from lane 0 — and
// that sequence depends only on the element's own row and stream, never on n, the
// stream's batch position or its slot.  No atomics take part in any arithmetic.
//
// The element-wise phases (conv + SiLU, dt_proj + softplus, selective scan, gate) are
// per-thread code in the reference's own operation order and math
// (src/infrastructure/mamba/model.rs:134-190, src/domain/tensor.rs:1197-1325), so they
// reproduce the CPU path's bits for identical inputs.  Contraction is off in this file:
// only the explicit __builtin_fmaf calls of the projections fuse.
#include <hip/hip_runtime.h>

#include "model.h"
#include "portable_math.h"

#pragma clang fp contract(off)

namespace rdk {

namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;

__device__ __forceinline__ float wave_sum(float v) {
    // Fixed xor butterfly; lane 0's result is the one consumers use.
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ uint32_t clamp_slot(uint32_t s, uint32_t cap) { return s < cap ? s : cap - 1; }

// ---------------------------------------------------------------- embedding

// x[b] = emb[token[b]] (Q8: q * scale of its group), model.rs:93-101 / gemv.rs:285-295.
// With `check`, block (0, b) also validates slot and token of stream b against the pool
// and the vocabulary and against the other streams' slots, and records failures.
__global__ __launch_bounds__(kBlock) void k_embed(float* __restrict__ x, DMat emb, const uint32_t* __restrict__ tokens,
                                                  const uint32_t* __restrict__ slots, uint32_t n, uint32_t cap,
                                                  int check, uint32_t* __restrict__ err) {
    const uint32_t b = blockIdx.y;
    const int d = emb.cols;
    uint32_t tok = tokens[b];
    if (check && blockIdx.x == 0) {
        const uint32_t s = slots[b];
        bool bad = tok >= (uint32_t)emb.rows || s >= cap;
        bool dup = false;
        for (uint32_t c = threadIdx.x; c < n; c += blockDim.x)
            if (c != b && slots[c] == s) dup = true;
        if (bad && threadIdx.x == 0) atomicOr(err, 1u);
        if (dup) atomicOr(err, 2u);
    }
    if (tok >= (uint32_t)emb.rows) tok = emb.rows - 1;
    const int k = blockIdx.x * kBlock + threadIdx.x;
    if (k >= d) return;
    const size_t tile = (size_t)(tok >> 2) * (d >> 2) + (k >> 2);
    const int off = (tok & 3) * 4 + (k & 3);
    float v;
    if (emb.group == 0) {
        v = ((const float*)emb.w)[tile * 16 + off];
    } else {
        const int8_t q = ((const int8_t*)emb.w)[tile * 16 + off];
        v = (float)q * emb.scales[(size_t)tok * (d / emb.group) + k / emb.group];
    }
    x[(size_t)b * d + k] = v;
}

// ---------------------------------------------------------------- norms

__device__ __forceinline__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kBlock / kWave; w++) t += sh[w];
    __syncthreads();
    return t;
}

// RMSNorm (tensor.rs:900-908) or LayerNorm (tensor.rs:1390-1398) of one stream per block.
__global__ __launch_bounds__(kBlock) void k_norm(float* __restrict__ out, const float* __restrict__ x,
                                                 const float* __restrict__ w, const float* __restrict__ bias, int d) {
    __shared__ float sh[kBlock / kWave];
    const size_t base = (size_t)blockIdx.x * d;
    if (bias == nullptr) {
        float ss = 0.0f;
        for (int k = threadIdx.x; k < d; k += kBlock) {
            const float v = x[base + k];
            ss += v * v;
        }
        ss = block_sum(ss, sh);
        const float inv = 1.0f / sqrtf(ss / (float)d + 1e-5f);
        for (int k = threadIdx.x; k < d; k += kBlock) out[base + k] = x[base + k] * inv * w[k];
    } else {
        float s = 0.0f;
        for (int k = threadIdx.x; k < d; k += kBlock) s += x[base + k];
        const float mean = block_sum(s, sh) / (float)d;
        float vs = 0.0f;
        for (int k = threadIdx.x; k < d; k += kBlock) {
            const float c = x[base + k] - mean;
            vs += c * c;
        }
        const float inv = 1.0f / sqrtf(block_sum(vs, sh) / (float)d + 1e-5f);
        for (int k = threadIdx.x; k < d; k += kBlock) out[base + k] = (x[base + k] - mean) * inv * w[k] + bias[k];
    }
}

// ---------------------------------------------------------------- projections

struct GemvArgs {
    DMat m;
    const float* x;  // stream b's input: x + b*ldx (16-byte aligned, ldx % 4 == 0)
    int ldx;
    float* y;        // stream b's output: y + b*ldy
    int ldy;
    uint32_t n;      // streams
    uint32_t sb;     // streams per blockIdx.y
    int accumulate;  // y += W x (residual) instead of y = W x
};

// y[b][r] = sum_k W[r][k] x[b][k] for a row quad per wavefront.  Lane l owns column
// quads l, l+64, ..., holds their weight tiles in registers for the whole block, and
// for each stream accumulates tile by tile with fused multiply-adds in column order;
// the 64 lane partials are then summed by the fixed butterfly.  Q8 weights are
// widened to f32 exactly; a per-row scale multiplies the row sum, group scales
// (64 columns) multiply each tile's partial before it joins the row sum.
template <int NQ, int MODE>  // MODE 0: F32, 1: Q8 per-row scale, 2: Q8 group scales
__global__ __launch_bounds__(kBlock) void k_gemv(GemvArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int rq = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    if (rq >= a.m.rq) return;
    const int kqn = a.m.cols >> 2;
    float wt[NQ][4][4];
    float gs[NQ][4];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int kq = lane + q * kWave;
        const size_t tile = (size_t)rq * kqn + kq;
        if (kq < kqn) {
            if (MODE == 0) {
                const float4* p = (const float4*)a.m.w + tile * 4;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 v = p[i];
                    wt[q][i][0] = v.x; wt[q][i][1] = v.y; wt[q][i][2] = v.z; wt[q][i][3] = v.w;
                }
            } else {
                const int4 v = ((const int4*)a.m.w)[tile];
                const int words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int c = 0; c < 4; c++) wt[q][i][c] = (float)(int8_t)(words[i] >> (8 * c));
            }
            if (MODE == 2) {
                const int gpr = a.m.cols / a.m.group;
                const int g = (kq * 4) / a.m.group;
#pragma unroll
                for (int i = 0; i < 4; i++) gs[q][i] = a.m.scales[(size_t)(rq * 4 + i) * gpr + g];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                gs[q][i] = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; c++) wt[q][i][c] = 0.0f;
            }
        }
    }
    float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (MODE == 1) {
#pragma unroll
        for (int i = 0; i < 4; i++) rs[i] = a.m.scales[rq * 4 + i];
    }
    const uint32_t b0 = blockIdx.y * a.sb;
    const uint32_t b1 = min(b0 + a.sb, a.n);
    for (uint32_t b = b0; b < b1; b++) {
        const float4* xb = (const float4*)(a.x + (size_t)b * a.ldx);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int kq = lane + q * kWave;
            if (kq < kqn) {
                const float4 xv = xb[kq];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (MODE == 2) {
                        float t = wt[q][i][0] * xv.x;
                        t = __builtin_fmaf(wt[q][i][1], xv.y, t);
                        t = __builtin_fmaf(wt[q][i][2], xv.z, t);
                        t = __builtin_fmaf(wt[q][i][3], xv.w, t);
                        acc[i] = __builtin_fmaf(t, gs[q][i], acc[i]);
                    } else {
                        acc[i] = __builtin_fmaf(wt[q][i][0], xv.x, acc[i]);
                        acc[i] = __builtin_fmaf(wt[q][i][1], xv.y, acc[i]);
                        acc[i] = __builtin_fmaf(wt[q][i][2], xv.z, acc[i]);
                        acc[i] = __builtin_fmaf(wt[q][i][3], xv.w, acc[i]);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = wave_sum(acc[i]);
        if (lane == 0) {
            float* yb = a.y + (size_t)b * a.ldy;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = rq * 4 + i;
                if (r < a.m.rows) {
                    const float v = MODE == 1 ? acc[i] * rs[i] : acc[i];
                    yb[r] = a.accumulate ? yb[r] + v : v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------- conv1d step

// conv_silu_block (model.rs:134-153): v = sum_k st[k] w[k] + x w[dc-1] + b, shift the
// state, then SiLU as silu_inplace applies it to 256-channel blocks (tensor.rs:1207-1211:
// lane sigmoid on each block's 8-aligned body, portable sigmoid on its tail).
__global__ __launch_bounds__(kBlock) void k_conv(float* __restrict__ conv_out, float* __restrict__ conv_st,
                                                 const float* __restrict__ xz, const float* __restrict__ cw,
                                                 const float* __restrict__ cb, const uint32_t* __restrict__ slots,
                                                 uint32_t cap, int di, int dc) {
    const int j = blockIdx.x * kBlock + threadIdx.x;
    const uint32_t b = blockIdx.y;
    if (j >= di) return;
    const uint32_t s = clamp_slot(slots[b], cap);
    float* st = conv_st + ((size_t)s * di + j) * (dc - 1);
    const float* w = cw + (size_t)j * dc;
    const float xv = xz[(size_t)b * 2 * di + j];
    float val = 0.0f;
    for (int k = 0; k < dc - 1; k++) val += st[k] * w[k];
    val += xv * w[dc - 1];
    val += cb[j];
    for (int k = 0; k + 2 < dc; k++) st[k] = st[k + 1];
    st[dc - 2] = xv;
    const int blk0 = j / 256 * 256;
    const int len = min(256, di - blk0);
    const bool body = (j - blk0) < len / 8 * 8;
    const float sg = body ? lane_sigmoid_f(val) : 1.0f / (1.0f + exp_f(-val));
    conv_out[(size_t)b * di + j] = val * sg;
}

// ---------------------------------------------------------------- dt + scan + gate

struct ScanArgs {
    float* gated;          // [n][di]
    float* ssm;            // layer base, [slot][di][16]
    const float* zp;       // [n][xr]: dt_raw | B | C
    const float* xz;       // [n][2di]: z at di..2di
    const float* conv_out; // [n][di]
    const float* dt_wt;    // F32 [dr][di] or null
    const int8_t* dt_qt;   // Q8 [dr][di] or null
    const float* dt_scales;
    int dt_group;
    const float* dt_b;
    const float* a_exp;    // [di][16]
    const float* d_vec;
    const uint32_t* slots;
    uint32_t cap;
    int di, dr;
};

// One column of the transposed dt_proj in dot_avx2_order (tensor.rs:1680-1693): eight
// lanes by column residue from +0, ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), sequential tail.
template <typename T>
__device__ __forceinline__ float dot_ref_col(const T* __restrict__ wt, int stride, const float* __restrict__ v, int n) {
    const int body = n / 8 * 8;
    float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = 0; c < body; c += 8)
#pragma unroll
        for (int i = 0; i < 8; i++) l[i] += (float)wt[(size_t)(c + i) * stride] * v[c + i];
    float s = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
    for (int c = body; c < n; c++) s += (float)wt[(size_t)c * stride] * v[c];
    return s;
}

// scan_block (model.rs:174-190) for one (stream, channel): dt_proj row, softplus(dt+b)
// (tensor.rs:859-861), the d16 recurrence with the dt-sparse skip and the hsum_ssm tree
// (tensor.rs:1283-1325), then y * (z * sigmoid(z)) (tensor.rs:1239-1243, 64-channel
// blocks).
__global__ __launch_bounds__(kBlock) void k_scan(ScanArgs a) {
    const int j = blockIdx.x * kBlock + threadIdx.x;
    const uint32_t b = blockIdx.y;
    if (j >= a.di) return;
    const int di = a.di, dr = a.dr;
    const int xr = dr + 32;
    const float* zp = a.zp + (size_t)b * xr;
    float dt;
    if (a.dt_wt) {
        dt = dot_ref_col(a.dt_wt + j, di, zp, dr);
    } else {
        const int gpr = dr / a.dt_group;
        dt = 0.0f;
        for (int g = 0; g < gpr; g++)
            dt += dot_ref_col(a.dt_qt + (size_t)g * a.dt_group * di + j, di, zp + g * a.dt_group, a.dt_group) *
                  a.dt_scales[(size_t)j * gpr + g];
    }
    dt = softplus_f(dt + a.dt_b[j]);
    const float x = a.conv_out[(size_t)b * di + j];
    const uint32_t s = clamp_slot(a.slots[b], a.cap);
    float4* stp = (float4*)(a.ssm + ((size_t)s * di + j) * 16);
    float st[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = stp[i];
        st[4 * i] = v.x; st[4 * i + 1] = v.y; st[4 * i + 2] = v.z; st[4 * i + 3] = v.w;
    }
    const float* B = zp + dr;
    const float* C = zp + dr + 16;
    if (!(fabsf(dt) < 1e-6f)) {
        const float dtx = dt * x;
        const float4* ap = (const float4*)(a.a_exp + (size_t)j * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 av = ap[i];
            const float aa[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int k = 4 * i + c;
                const float da = lane_exp_f(0.0f - dt * aa[c]);
                st[k] = da * st[k] + dtx * B[k];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) stp[i] = make_float4(st[4 * i], st[4 * i + 1], st[4 * i + 2], st[4 * i + 3]);
    }
    float l[8];
#pragma unroll
    for (int i = 0; i < 8; i++) l[i] = st[i] * C[i] + st[i + 8] * C[i + 8];
    const float y = ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7])) + a.d_vec[j] * x;
    const float z = a.xz[(size_t)b * 2 * di + di + j];
    const int blk0 = j / 64 * 64;
    const int len = min(64, di - blk0);
    const bool body = (j - blk0) < len / 8 * 8;
    const float sg = body ? lane_sigmoid_f(z) : 1.0f / (1.0f + exp_f(-z));
    a.gated[(size_t)b * di + j] = y * (z * sg);
}

// ---------------------------------------------------------------- softmax

// softmax_into (tensor.rs:1917-1933) per stream: max, exp(l - max) with the portable
// exp, sum (fixed block tree instead of the sequential loop), division by
// max(sum, FLT_EPSILON).  In place on `out`.
__global__ __launch_bounds__(1024) void k_softmax(float* __restrict__ out, int vocab) {
    __shared__ float sh[1024 / kWave];
    float* row = out + (size_t)blockIdx.x * vocab;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < vocab; i += 1024) mx = fmaxf(mx, row[i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    if (lane == 0) sh[wave] = mx;
    __syncthreads();
    mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 1024 / kWave; w++) mx = fmaxf(mx, sh[w]);
    __syncthreads();
    if (mx == -INFINITY) {
        const float u = 1.0f / (float)vocab;
        for (int i = threadIdx.x; i < vocab; i += 1024) row[i] = u;
        return;
    }
    float s = 0.0f;
    for (int i = threadIdx.x; i < vocab; i += 1024) {
        const float e = exp_f(row[i] - mx);
        row[i] = e;
        s += e;
    }
    s = wave_sum(s);
    if (lane == 0) sh[wave] = s;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < 1024 / kWave; w++) t += sh[w];
    const float denom = fmaxf(t, 1.1920929e-07f);
    for (int i = threadIdx.x; i < vocab; i += 1024) row[i] = row[i] / denom;
}

// ---------------------------------------------------------------- reset

__global__ __launch_bounds__(kBlock) void k_zero_slots(float* __restrict__ base, const uint32_t* __restrict__ slots,
                                                       uint32_t cap, size_t stride, size_t layer_stride, int nl) {
    const uint32_t s = slots[blockIdx.y];
    if (s >= cap) return;
    for (int l = 0; l < nl; l++) {
        float* p = base + (size_t)l * layer_stride + (size_t)s * stride;
        for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < stride; i += (size_t)gridDim.x * kBlock)
            p[i] = 0.0f;
    }
}

// ---------------------------------------------------------------- launchers

template <int MODE>
hipError_t launch_gemv_mode(const GemvArgs& a, hipStream_t st) {
    const int nq = (a.m.cols / 4 + kWave - 1) / kWave;
    dim3 grid((a.m.rq + 3) / 4, (a.n + a.sb - 1) / a.sb);
    switch (nq) {
#define CASE(Q) case Q: k_gemv<Q, MODE><<<grid, kBlock, 0, st>>>(a); break;
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
#undef CASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv(const DMat& m, const float* x, int ldx, float* y, int ldy, uint32_t n, uint32_t sb,
                       int accumulate, hipStream_t st) {
    GemvArgs a{m, x, ldx, y, ldy, n, sb, accumulate};
    if (m.group == 0) return launch_gemv_mode<0>(a, st);
    if (m.group == m.cols) return launch_gemv_mode<1>(a, st);
    return launch_gemv_mode<2>(a, st);
}

// Streams per blockIdx.y: skinny matrices spread streams over more workgroups,
// wide ones keep every weight tile in registers across more streams.
uint32_t streams_per_block(const DMat& m, uint32_t n) {
    const uint32_t blocks = (uint32_t)(m.rq + 3) / 4;
    uint32_t sb = blocks >= 128 ? 32 : 4;
    return sb < n ? sb : (n ? n : 1);
}

}  // namespace

#define RDK_TRY(expr)                     \
    do {                                  \
        hipError_t e_ = (expr);           \
        if (e_ != hipSuccess) return e_;  \
    } while (0)

// Brackets one launch with the probe's next event pair when its class is probed.
struct ProbeScope {
    Probe* p;
    bool on;
    hipStream_t st;
    ProbeScope(Probe* probe, uint32_t cls, hipStream_t s)
        : p(probe), on(probe && probe->cls == cls && probe->used + 2 <= probe->cap), st(s) {
        if (on) (void)hipEventRecord(p->ev[p->used], st);
    }
    ~ProbeScope() {
        if (on) {
            (void)hipEventRecord(p->ev[p->used + 1], st);
            p->used += 2;
        }
    }
};

hipError_t enqueue_step(const StepArgs& a, hipStream_t st) {
    const Dims& D = *a.dims;
    Pool& P = *a.pool;
    const uint32_t n = a.n;
    const int d = (int)D.d, di = (int)D.di, xr = (int)D.xr();
    {
        ProbeScope ps(a.probe, KC_EMBED, st);
        k_embed<<<dim3((d + kBlock - 1) / kBlock, n), kBlock, 0, st>>>(P.x, *a.emb, a.tokens, a.slots, n, P.cap,
                                                                       a.check ? 1 : 0, a.err);
    }
    RDK_TRY(hipGetLastError());
    const size_t conv_layer = (size_t)P.cap * di * (D.dc - 1);
    const size_t ssm_layer = (size_t)P.cap * di * 16;
    for (uint32_t li = 0; li < D.nl; li++) {
        const DLayer& L = a.layers[li];
        {
            ProbeScope ps(a.probe, KC_NORM, st);
            k_norm<<<n, kBlock, 0, st>>>(P.normed, P.x, L.norm_w, L.norm_b, d);
        }
        RDK_TRY(hipGetLastError());
        {
            ProbeScope ps(a.probe, KC_IN_PROJ, st);
            RDK_TRY(launch_gemv(L.in_proj, P.normed, d, P.xz, 2 * di, n, streams_per_block(L.in_proj, n), 0, st));
        }
        {
            ProbeScope ps(a.probe, KC_CONV, st);
            k_conv<<<dim3((di + kBlock - 1) / kBlock, n), kBlock, 0, st>>>(P.conv_out, P.conv + li * conv_layer,
                                                                           P.xz, L.conv_w, L.conv_b, a.slots, P.cap,
                                                                           di, (int)D.dc);
        }
        RDK_TRY(hipGetLastError());
        {
            ProbeScope ps(a.probe, KC_X_PROJ, st);
            RDK_TRY(launch_gemv(L.x_proj, P.conv_out, di, P.zp, xr, n, streams_per_block(L.x_proj, n), 0, st));
        }
        ScanArgs s{P.gated, P.ssm + li * ssm_layer, P.zp, P.xz, P.conv_out, L.dt_wt, L.dt_qt, L.dt_scales,
                   L.dt_group, L.dt_b, L.a_exp, L.d_vec, a.slots, P.cap, di, (int)D.dr};
        {
            ProbeScope ps(a.probe, KC_SCAN, st);
            k_scan<<<dim3((di + kBlock - 1) / kBlock, n), kBlock, 0, st>>>(s);
        }
        RDK_TRY(hipGetLastError());
        {
            ProbeScope ps(a.probe, KC_OUT_PROJ, st);
            RDK_TRY(launch_gemv(L.out_proj, P.gated, di, P.x, d, n, streams_per_block(L.out_proj, n), 1, st));
        }
    }
    {
        ProbeScope ps(a.probe, KC_NORM, st);
        k_norm<<<n, kBlock, 0, st>>>(P.normed, P.x, a.norm_f_w, a.norm_f_b, d);
    }
    RDK_TRY(hipGetLastError());
    {
        ProbeScope ps(a.probe, KC_HEAD, st);
        RDK_TRY(launch_gemv(*a.head, P.normed, d, a.out, (int)D.vocab, n, streams_per_block(*a.head, n), 0, st));
    }
    if (a.probs) {
        {
            ProbeScope ps(a.probe, KC_SOFTMAX, st);
            k_softmax<<<n, 1024, 0, st>>>(a.out, (int)D.vocab);
        }
        RDK_TRY(hipGetLastError());
    }
    return hipSuccess;
}

hipError_t enqueue_reset(const Dims& D, Pool& P, const uint32_t* d_slots, uint32_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t conv_stride = (size_t)D.di * (D.dc - 1), ssm_stride = (size_t)D.di * 16;
    const unsigned gx = (unsigned)((ssm_stride + kBlock - 1) / kBlock);
    k_zero_slots<<<dim3((unsigned)((conv_stride + kBlock - 1) / kBlock), n), kBlock, 0, st>>>(
        P.conv, d_slots, P.cap, conv_stride, (size_t)P.cap * conv_stride, (int)D.nl);
    RDK_TRY(hipGetLastError());
    k_zero_slots<<<dim3(gx, n), kBlock, 0, st>>>(P.ssm, d_slots, P.cap, ssm_stride, (size_t)P.cap * ssm_stride,
                                                 (int)D.nl);
    return hipGetLastError();
}

}  // namespace rdk
