// gemv_step.hip — the Mamba step on wavefront-GEMV kernels: the small-batch tier.
//
// Selected at init by weight profile bit 4, never by the batch size, so that a stream's
// logits do not depend on n (the reference's batch-invariance rule, PLUGIN-FFI-V2.md:97-101):
// one family serves every batch of a loaded model.  The projections run as f32 dot
// products on the vector ALUs instead of matrix cores: int8 (or f32) weights streamed from
// HBM in whole 1 KB runs per wave, each lane holding a fixed slice of K whose activations
// stay in registers for every row, and a fixed xor butterfly over the lanes that share a
// row.  Per layer:
//   k_mix_in_g : RMSNorm, in_proj rows (32 per workgroup), conv1d step + SiLU, x_proj
//                split-K partials over the workgroup's 32 channels (the MFMA family's
//                partial format, so the scan is shared);
//   k_scan     : shared with the MFMA family, writing the gated vector in f32;
//   k_mix_out_g: out_proj + residual.
// and per step k_embed_g (gather from the GEMV layout, device argument check), k_head_g
// (final RMSNorm + LM head) and optionally the shared softmax.
//
// Arithmetic of one output (row r, stream b): each lane sums its chunks' products in order
// (chunk j ascending, element ascending, one FMA each), the lanes of the row are added in
// a fixed xor butterfly, then Q8 rows are 0 + dot * scale (gemv.rs:490-502).  Nothing
// depends on n, the batch position, the slot or the streams per workgroup.  Contraction
// stays off for the element-wise code (conv, SiLU, norms); the dots use explicit FMAs.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "mfma_common.h"
#include "model.h"
#include "portable_math.h"
#include "step.h"

#pragma clang fp contract(off)

namespace rdk {

size_t GMat::bytes() const {
    if (!w) return 0;
    const size_t n = (size_t)blocks * rpi * cols;
    return q8 ? n + (size_t)blocks * rpi * 4 : n * 4;
}

bool gemv_shape(int cols, int& rpi, int& cpl) {
    if (cols <= 0 || cols % 16) return false;
    const int cr = cols / 16;
    for (int c : {1, 2, 3, 4, 6, 8}) {
        if ((64 * c) % cr) continue;
        const int r = 64 * c / cr;
        if (r < 1 || r > 32 || (r & (r - 1))) continue;
        rpi = r;
        cpl = c;
        return true;
    }
    return false;
}

namespace {

constexpr int kGBlock = 256;
constexpr int kGWaves = kGBlock / kWave;
constexpr int kInRows = 32;     // in_proj rows per workgroup: one 32-channel x_proj block
constexpr int kOutRows = 16;    // out_proj rows per workgroup
constexpr int kHeadRows = 64;   // head rows per workgroup

// One lane's weights of one chunk: Q8 16 int8, F32 16 floats.
template <bool Q8>
struct GChunk {
    int4 v[Q8 ? 1 : 4];
};

// F32 chunks are stored as four 1 KB runs per wave load: [block][j][quarter][lane][4 f32].
template <bool Q8>
__device__ __forceinline__ GChunk<Q8> gload(const GMat& g, int block, int j, int lane) {
    GChunk<Q8> c;
    const size_t idx = (size_t)block * g.cpl + j;
    if (Q8) {
        c.v[0] = ((const int4*)g.w)[idx * 64 + lane];
    } else {
#pragma unroll
        for (int q = 0; q < 4; q++) c.v[q] = ((const int4*)g.w)[(idx * 4 + q) * 64 + lane];
    }
    return c;
}

template <bool Q8>
__device__ __forceinline__ float gweight(const GChunk<Q8>& c, int e) {
    if (Q8) {
        const int w = e < 4 ? c.v[0].x : e < 8 ? c.v[0].y : e < 12 ? c.v[0].z : c.v[0].w;
        return (float)(int8_t)(w >> (8 * (e % 4)));
    }
    const int4 q = c.v[e / 4];
    const int w = e % 4 == 0 ? q.x : e % 4 == 1 ? q.y : e % 4 == 2 ? q.z : q.w;
    return bits_to_f((uint32_t)w);
}

// The K index of element e of the lane's chunk j.
__device__ __forceinline__ int gk(int lane, int rpi, int j, int e) { return 16 * (lane / rpi + (64 / rpi) * j) + e; }

// The dots of one iteration block (rpi rows) for S streams: act[s][j * 16 + e] is the lane's
// activation slice.  After the butterfly lane l < rpi holds row l of the block.
template <bool Q8, int CPL, int S>
__device__ __forceinline__ void gdot(const GChunk<Q8> (&w)[CPL], const float (&act)[S][CPL * 16], int rpi,
                                     float (&out)[S]) {
#pragma unroll
    for (int s = 0; s < S; s++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc = __builtin_fmaf(gweight<Q8>(w[j], e), act[s][j * 16 + e], acc);
        for (int o = rpi; o < kWave; o <<= 1) acc += __shfl_xor(acc, o, kWave);
        out[s] = acc;
    }
}

// The lane's slice of stream row x (zeros for a stream past n) and its RMSNorm scale
// 1 / sqrt(mean(x^2) + 1e-5) (tensor.rs:900-908): the slices of the 64 lanes cover x
// exactly rpi times, so the fixed xor butterfly of the lanes' slice sums of squares is
// rpi * sum(x^2), divided exactly by the power of two rpi.  Every lane gets the same bits.
template <int CPL>
__device__ __forceinline__ void load_slice(const float* __restrict__ x, int rpi, bool live, float (&a)[CPL * 16]) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const float4* q = (const float4*)(x + gk(lane, rpi, j, 0));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float4 v = live ? q[e] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            a[j * 16 + 4 * e] = v.x;
            a[j * 16 + 4 * e + 1] = v.y;
            a[j * 16 + 4 * e + 2] = v.z;
            a[j * 16 + 4 * e + 3] = v.w;
        }
    }
}

template <int CPL>
__device__ __forceinline__ float slice_rms_inv(const float (&a)[CPL * 16], int d, int rpi) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL * 16; i++) ss += a[i] * a[i];
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    ss = ss / (float)rpi;
    return 1.0f / sqrtf(ss / (float)d + 1e-5f);
}

// ---------------------------------------------------------------- embedding

struct EmbedGArgs {
    GMat emb;
    float* x;
    const uint32_t* tokens;
    const uint32_t* slots_in;
    uint32_t* slots;
    uint32_t n, cap;
    int check;
    uint32_t* err;
};

// x[b] = emb[token[b]] (Q8: q * scale), model.rs:93-101 / gemv.rs:285-295, gathered from
// the GEMV layout; block b also validates its entry as k_embed does (a bad entry, or a slot
// an earlier entry already names, is routed to the scratch slot `cap`).
__global__ __launch_bounds__(kGBlock) void k_embed_g(EmbedGArgs a) {
    const uint32_t b = blockIdx.x;
    const GMat& g = a.emb;
    uint32_t tok = a.tokens[b];
    check_entry(a.slots_in, a.slots, a.n, b, tok < (uint32_t)g.rows, a.cap, a.check, a.err);
    if (tok >= (uint32_t)g.rows) tok = g.rows - 1;
    const int blk = (int)tok / g.rpi, rr = (int)tok % g.rpi, per = 64 / g.rpi;
    const float sc = g.q8 ? g.scales[tok] : 1.0f;
    for (int k = threadIdx.x; k < g.cols; k += kGBlock) {
        const int c = k / 16, e = k % 16;
        const int j = c / per, lane = rr + g.rpi * (c % per);
        const size_t idx = (size_t)blk * g.cpl + j;
        float v;
        if (g.q8) {
            v = (float)((const int8_t*)g.w)[(idx * 64 + lane) * 16 + e] * sc;
        } else {
            v = ((const float*)g.w)[((idx * 4 + e / 4) * 64 + lane) * 4 + e % 4];
        }
        a.x[(size_t)b * g.cols + k] = v;
    }
}

// ---------------------------------------------------------------- in_proj + conv + x_proj

struct MixInGArgs {
    const float* x;          // [n][d]
    const float* norm_w;
    GMat w;                  // in_proj [2 di][d]
    const float* xp_w;       // x_proj [xr][di] f32, or
    const int8_t* xp_q;      // Q8 with one scale per row
    const float* xp_scales;
    float* conv_st;          // this layer's conv state [slot][di][3]
    const float* conv_w;     // [di][4]
    const float* conv_b;
    const uint32_t* slots;
    uint32_t xcap, n, scap;
    float* u;
    float* z;
    float* xpart;            // [di / 32][xcap][xr_pad]
    int di, d, xr, xr_pad;
};

// Workgroup (row block rb of 32 in_proj rows, streams [S by, S by + S)): rows below di are
// the conv branch (channel = row), the rest the gate branch.  Wave w takes the block's
// iteration blocks w, w + 4, ... (BPW of them at most).  Every load is issued before the
// first use: the slots, the activation slices and norm weights, the weights of all the
// wave's blocks, the conv operands of the lane's rows and the x_proj row of the thread.
// The conv branch runs conv1d + SiLU per (channel, stream) in conv_silu_block order
// (model.rs:134-153) and leaves one x_proj partial per output over its 32 channels
// (sequential over the channels, x row scale), the format the scan sums.
template <bool Q8, bool Q8XP, int CPL, int S, int BPW>
__global__ __launch_bounds__(kGBlock) void k_mix_in_g(MixInGArgs a) {
    __shared__ float ul[S][kInRows];
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const GMat& g = a.w;
    const int rpi = g.rpi;
    const int rb = blockIdx.x;
    const uint32_t b0 = blockIdx.y * S;
    const bool conv = rb * kInRows < a.di;
    const int nblk = kInRows / rpi;
    uint32_t slot[S];
#pragma unroll
    for (int s = 0; s < S; s++) slot[s] = clamp_slot(a.slots[min(b0 + s, a.n - 1)], a.scap);
    float act[S][CPL * 16];
#pragma unroll
    for (int s = 0; s < S; s++) load_slice<CPL>(a.x + (size_t)min(b0 + s, a.n - 1) * a.d, rpi, b0 + s < a.n, act[s]);
    float nw[CPL * 16];
    load_slice<CPL>(a.norm_w, rpi, true, nw);
    GChunk<Q8> wc[BPW][CPL];
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int ib = min(wave + kGWaves * i, nblk - 1);
#pragma unroll
        for (int j = 0; j < CPL; j++) wc[i][j] = gload<Q8>(g, rb * nblk + ib, j, lane);
    }
    // conv operands of the lane's rows (lane < rpi; others read row 0's and never use them)
    float4 cw[BPW];
    float cb[BPW], st[BPW][S][3], rsc[BPW];
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int ib = min(wave + kGWaves * i, nblk - 1);
        const int row = (rb * nblk + ib) * rpi + (lane < rpi ? lane : 0);
        rsc[i] = Q8 ? g.scales[row] : 1.0f;
        const int ch = conv ? row : 0;
        cw[i] = *(const float4*)(a.conv_w + (size_t)ch * 4);
        cb[i] = a.conv_b[ch];
#pragma unroll
        for (int s = 0; s < S; s++) {
            const float* sp = a.conv_st + ((size_t)slot[s] * a.di + ch) * 3;
#pragma unroll
            for (int k = 0; k < 3; k++) st[i][s][k] = __builtin_nontemporal_load(sp + k);
        }
    }
    // the x_proj row of thread t over the block's 32 channels
    const int t = threadIdx.x;
    const int tr = min(t, a.xr - 1);
    const int c0 = conv ? rb * kInRows : 0;
    float xw[kInRows];
    if (Q8XP) {
        const int4* q = (const int4*)(a.xp_q + (size_t)tr * a.di + c0);
        const int4 q0 = q[0], q1 = q[1];
        const int wv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int c = 0; c < kInRows; c++) xw[c] = (float)(int8_t)(wv[c / 4] >> (8 * (c % 4)));
    } else {
        const float4* q = (const float4*)(a.xp_w + (size_t)tr * a.di + c0);
#pragma unroll
        for (int c = 0; c < kInRows / 4; c++) {
            const float4 v = q[c];
            xw[4 * c] = v.x;
            xw[4 * c + 1] = v.y;
            xw[4 * c + 2] = v.z;
            xw[4 * c + 3] = v.w;
        }
    }
    const float xs = Q8XP ? a.xp_scales[tr] : 1.0f;
    // x * inv * w (RMSNorm) on the slices
#pragma unroll
    for (int s = 0; s < S; s++) {
        const float inv = slice_rms_inv<CPL>(act[s], a.d, rpi);
#pragma unroll
        for (int i = 0; i < CPL * 16; i++) act[s][i] = act[s][i] * inv * nw[i];
    }
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int ib = wave + kGWaves * i;
        if (ib >= nblk) break;
        float dot[S];
        gdot<Q8, CPL, S>(wc[i], act, rpi, dot);
        if (lane >= rpi) continue;
        const int row = (rb * nblk + ib) * rpi + lane;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint32_t b = b0 + s;
            if (b >= a.n) continue;
            const float y = Q8 ? 0.0f + dot[s] * rsc[i] : dot[s];
            if (!conv) {
                a.z[(size_t)b * a.di + (row - a.di)] = y;
                continue;
            }
            float val = 0.0f;
            val += st[i][s][0] * cw[i].x;
            val += st[i][s][1] * cw[i].y;
            val += st[i][s][2] * cw[i].z;
            val += y * cw[i].w;
            val += cb[i];
            float* sp = a.conv_st + ((size_t)slot[s] * a.di + row) * 3;
            __builtin_nontemporal_store(st[i][s][1], sp);
            __builtin_nontemporal_store(st[i][s][2], sp + 1);
            __builtin_nontemporal_store(y, sp + 2);
            const float uv = val * lane_sigmoid_f(val);
            a.u[(size_t)b * a.di + row] = uv;
            ul[s][row - rb * kInRows] = uv;
        }
    }
    if (!conv) return;
    __syncthreads();
    if (t >= a.xr) return;
    float acc[S];
#pragma unroll
    for (int s = 0; s < S; s++) acc[s] = 0.0f;
#pragma unroll
    for (int c = 0; c < kInRows; c++)
#pragma unroll
        for (int s = 0; s < S; s++) acc[s] = __builtin_fmaf(xw[c], ul[s][c], acc[s]);
#pragma unroll
    for (int s = 0; s < S; s++) {
        const uint32_t b = b0 + s;
        if (b >= a.n) continue;
        a.xpart[((size_t)rb * a.xcap + b) * a.xr_pad + t] = Q8XP ? acc[s] * xs : acc[s];
    }
}

// ---------------------------------------------------------------- out_proj + residual

struct MixOutGArgs {
    GMat w;                  // out_proj [d][di]
    const float* g32;        // [n][di] gated
    float* x;                // [n][d] residual, updated in place
    uint32_t n;
    int d, di;
};

// Workgroup (kOutRows rows, S streams); every load issued first (activation slices, the
// weights of the wave's blocks, the residual rows of the lane).
template <bool Q8, int CPL, int S, int BPW>
__global__ __launch_bounds__(kGBlock) void k_mix_out_g(MixOutGArgs a) {
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const GMat& g = a.w;
    const int rpi = g.rpi;
    const uint32_t b0 = blockIdx.y * S;
    const int nblk = max(kOutRows / rpi, 1);
    float act[S][CPL * 16];
#pragma unroll
    for (int s = 0; s < S; s++) load_slice<CPL>(a.g32 + (size_t)min(b0 + s, a.n - 1) * a.di, rpi, b0 + s < a.n, act[s]);
    GChunk<Q8> wc[BPW][CPL];
    float xr[BPW][S], rsc[BPW];
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int blk = min((int)blockIdx.x * nblk + min(wave + kGWaves * i, nblk - 1), g.blocks - 1);
#pragma unroll
        for (int j = 0; j < CPL; j++) wc[i][j] = gload<Q8>(g, blk, j, lane);
        const int row = min(blk * rpi + (lane < rpi ? lane : 0), a.d - 1);
        rsc[i] = Q8 ? g.scales[row] : 1.0f;
#pragma unroll
        for (int s = 0; s < S; s++) xr[i][s] = a.x[(size_t)min(b0 + s, a.n - 1) * a.d + row];
    }
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int ib = wave + kGWaves * i;
        const int blk = (int)blockIdx.x * nblk + ib;
        if (ib >= nblk || blk >= g.blocks) break;
        float dot[S];
        gdot<Q8, CPL, S>(wc[i], act, rpi, dot);
        if (lane >= rpi) continue;
        const int row = blk * rpi + lane;
        if (row >= a.d) continue;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint32_t b = b0 + s;
            if (b >= a.n) continue;
            const float y = Q8 ? 0.0f + dot[s] * rsc[i] : dot[s];
            a.x[(size_t)b * a.d + row] = xr[i][s] + y;
        }
    }
}

// ---------------------------------------------------------------- head

struct HeadGArgs {
    const float* x;
    const float* norm_w;
    GMat w;                  // [vocab][d]
    float* out;              // [n][vocab]
    uint32_t n;
    int d;
};

// Final RMSNorm (model.rs:745-752) and the LM head (model.rs:921-927); kHeadRows rows per
// workgroup, every load issued first.
template <bool Q8, int CPL, int S, int BPW>
__global__ __launch_bounds__(kGBlock) void k_head_g(HeadGArgs a) {
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const GMat& g = a.w;
    const int rpi = g.rpi;
    const uint32_t b0 = blockIdx.y * S;
    const int nblk = max(kHeadRows / rpi, 1);
    float act[S][CPL * 16];
#pragma unroll
    for (int s = 0; s < S; s++) load_slice<CPL>(a.x + (size_t)min(b0 + s, a.n - 1) * a.d, rpi, b0 + s < a.n, act[s]);
    float nw[CPL * 16];
    load_slice<CPL>(a.norm_w, rpi, true, nw);
    GChunk<Q8> wc[BPW][CPL];
    float rsc[BPW];
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int blk = min((int)blockIdx.x * nblk + min(wave + kGWaves * i, nblk - 1), g.blocks - 1);
#pragma unroll
        for (int j = 0; j < CPL; j++) wc[i][j] = gload<Q8>(g, blk, j, lane);
        rsc[i] = Q8 ? g.scales[min(blk * rpi + (lane < rpi ? lane : 0), g.rows - 1)] : 1.0f;
    }
#pragma unroll
    for (int s = 0; s < S; s++) {
        const float inv = slice_rms_inv<CPL>(act[s], a.d, rpi);
#pragma unroll
        for (int i = 0; i < CPL * 16; i++) act[s][i] = act[s][i] * inv * nw[i];
    }
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int ib = wave + kGWaves * i;
        const int blk = (int)blockIdx.x * nblk + ib;
        if (ib >= nblk || blk >= g.blocks) break;
        float dot[S];
        gdot<Q8, CPL, S>(wc[i], act, rpi, dot);
        if (lane >= rpi) continue;
        const int row = blk * rpi + lane;
        if (row >= g.rows) continue;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint32_t b = b0 + s;
            if (b >= a.n) continue;
            __builtin_nontemporal_store(Q8 ? 0.0f + dot[s] * rsc[i] : dot[s], a.out + (size_t)b * g.rows + row);
        }
    }
}

// ---------------------------------------------------------------- instances

// Streams per workgroup: 1 for a single stream, 2 otherwise (the activation slice of a
// stream is CPL * 16 registers; a stream's arithmetic does not depend on the choice).
uint32_t gemv_streams(uint32_t n) { return n == 1 ? 1 : 2; }

// Blocks per wave: a workgroup's rows over rpi-row blocks dealt to its four waves.
int gemv_bpw(int rows_per_wg, int rpi) {
    const int blocks = std::max(rows_per_wg / rpi, 1);
    return blocks <= kGWaves ? 1 : (blocks <= 2 * kGWaves ? 2 : 4);
}

template <int CPL, int S, int BPW>
const void* mix_in_g_fn(bool q8, bool q8xp) {
    if (q8)
        return q8xp ? (const void*)k_mix_in_g<true, true, CPL, S, BPW> : (const void*)k_mix_in_g<true, false, CPL, S, BPW>;
    return q8xp ? (const void*)k_mix_in_g<false, true, CPL, S, BPW> : (const void*)k_mix_in_g<false, false, CPL, S, BPW>;
}
template <int CPL, int S, int BPW>
const void* mix_out_g_fn(bool q8) {
    return q8 ? (const void*)k_mix_out_g<true, CPL, S, BPW> : (const void*)k_mix_out_g<false, CPL, S, BPW>;
}
template <int CPL, int S, int BPW>
const void* head_g_fn(bool q8) {
    return q8 ? (const void*)k_head_g<true, CPL, S, BPW> : (const void*)k_head_g<false, CPL, S, BPW>;
}

// Chunks per lane are compiled for 1 and 3 (the shapes of d_model and d_inner in
// {64, 128, 256, 1024} and {96, 192, 384, 768, 1536, 3072}); the loader refuses others.
#define RDK_GEMV_BPW(NAME, CPL_, S_, BPW_, ...)                                                     \
    (BPW_ == 1 ? NAME<CPL_, S_, 1>(__VA_ARGS__) : BPW_ == 2 ? NAME<CPL_, S_, 2>(__VA_ARGS__) \
                                                            : NAME<CPL_, S_, 4>(__VA_ARGS__))
#define RDK_GEMV_PICK(NAME, CPL_, S_, BPW_, ...)                                                      \
    (CPL_ == 1 ? (S_ == 1 ? RDK_GEMV_BPW(NAME, 1, 1, BPW_, __VA_ARGS__) : RDK_GEMV_BPW(NAME, 1, 2, BPW_, __VA_ARGS__)) \
               : (S_ == 1 ? RDK_GEMV_BPW(NAME, 3, 1, BPW_, __VA_ARGS__) : RDK_GEMV_BPW(NAME, 3, 2, BPW_, __VA_ARGS__)))

}  // namespace

bool gemv_cpl_supported(int cpl) { return cpl == 1 || cpl == 3; }

Launch embed_g_launch(const GMat& emb, Pool& p, const StepIO& io) {
    EmbedGArgs ea{emb, p.x, io.tokens, io.slots, p.slots, io.n, p.cap, io.check ? 1 : 0, io.err};
    return Launch::make((const void*)k_embed_g, dim3(io.n), dim3(kGBlock), 0, KC_EMBED, ea);
}

void GemvStep::build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const {
    const Dims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d, di = (int)D.di;
    const uint32_t S = gemv_streams(n);
    const uint32_t chunks = (n + S - 1) / S;
    const DLayer& L0 = m.layers[0];
    const bool q8 = L0.g_in.q8, q8xp = L0.xp_q != nullptr;
    const int xr_pad = L0.x_proj.rt * kRowTile;
    out.clear();
    io_i = (int)out.size();
    out.push_back(embed_g_launch(*m.emb, p, io));
    const size_t conv_layer = (size_t)p.scap * di * (D.dc - 1);
    const size_t ssm_layer = (size_t)p.scap * di * 16;
    const void* fin = RDK_GEMV_PICK(mix_in_g_fn, L0.g_in.cpl, S, gemv_bpw(kInRows, L0.g_in.rpi), q8, q8xp);
    const void* fout = RDK_GEMV_PICK(mix_out_g_fn, L0.g_out.cpl, S, gemv_bpw(kOutRows, L0.g_out.rpi), q8);
    const uint32_t out_blocks = (uint32_t)((L0.g_out.blocks + std::max(kOutRows / L0.g_out.rpi, 1) - 1) /
                                           std::max(kOutRows / L0.g_out.rpi, 1));
    for (uint32_t li = 0; li < D.nl; li++) {
        const DLayer& L = m.layers[li];
        MixInGArgs ma{p.x, L.norm_w, L.g_in, L.xp_w, L.xp_q, L.xp_scales, p.conv + li * conv_layer, L.conv_w, L.conv_b,
                      p.slots, p.xcap, n, p.scap, p.u, p.z, p.xpart, di, d, (int)D.xr(), xr_pad};
        out.push_back(Launch::make(fin, dim3(2 * di / kInRows, chunks), dim3(kGBlock), 0, KC_MIX_IN, ma));
        out.push_back(scan_launch(L, D, p, n, m.exact_scan, nullptr, p.g32, p.ssm + li * ssm_layer));
        MixOutGArgs oa{L.g_out, p.g32, p.x, n, d, di};
        out.push_back(Launch::make(fout, dim3(out_blocks, chunks), dim3(kGBlock), 0, KC_MIX_OUT, oa));
    }
    const GMat& H = *m.head;
    head_i = (int)out.size();
    HeadGArgs ha{p.x, m.norm_f_w, H, io.out, n, d};
    const int hrows = std::max(kHeadRows / H.rpi, 1);
    out.push_back(Launch::make(RDK_GEMV_PICK(head_g_fn, H.cpl, S, gemv_bpw(kHeadRows, H.rpi), H.q8),
                               dim3((uint32_t)((H.blocks + hrows - 1) / hrows), chunks), dim3(kGBlock), 0, KC_HEAD, ha));
    sm_i = -1;
    if (io.probs) {
        sm_i = (int)out.size();
        out.push_back(softmax_launch(io.out, (int)D.vocab, n));
    }
}

}  // namespace rdk
