// mamba_step.hip — gfx950 kernels of one Mamba-1 token step for N lockstep streams.
//
// Per layer three kernels (all replayed from one hipGraph per step shape):
//   k_mix_in : RMSNorm of the residual stream, in_proj on the matrix cores, then for the
//              conv branch the causal conv1d step + SiLU and the split-K partial sums of
//              x_proj over this workgroup's 64 channels; for the gate branch z.
//   k_scan   : x_proj partials reduced in a fixed order, dt_proj + softplus, the d16
//              selective scan with the D skip, the SiLU gate; writes the gated vector as
//              bf16 limbs already tiled for the next matrix-core product.
//   k_mix_out: out_proj on the matrix cores, four k-quarters summed in a fixed order,
//              plus the residual.
// and per step k_embed (+ device-side argument check), k_head (final norm + LM head) and
// optionally k_softmax.
//
// Projections.  v_mfma_f32_16x16x32_bf16 multiplies bf16 operands exactly into f32
// accumulators.  Every f32 activation is split into three bf16 limbs (hi + mid + lo
// reproduces it to ~2^-24 relative); int8 weights are exact in bf16, so a Q8 product
// takes three MFMAs per k-step; F32 weights are split the same way and take the six
// limb products that reach 2^-24.  Activations are the B operand (16 streams per MFMA
// column group), weights the A operand (16 rows per tile).
//
// Determinism and batch invariance: an output element's value depends only on its own
// row and stream — MFMA columns are independent, every accumulation runs over k-steps
// and limbs in a fixed order, cross-wave and split-K partials are summed in a fixed
// order — never on n, the batch position or the slot; so one kernel family serves every
// batch size.  No atomics take part in any arithmetic.
//
// The element-wise phases (conv + SiLU, dt_proj + softplus, scan, gate, softmax) are
// per-thread code in the reference's own operation order and math
// (src/infrastructure/mamba/model.rs:134-190, src/domain/tensor.rs:759-1325), so they
// reproduce the CPU path's bits for identical inputs.  Contraction is off in this file.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>

#include "mfma_common.h"
#include "model.h"
#include "portable_math.h"
#include "step.h"

#pragma clang fp contract(off)

namespace rdk {

// Channels per x_proj split-K block at most: the channels of one k_mix_in conv-branch
// workgroup of two row tiles, one k-step of x_proj (four row tiles make 64-channel blocks).
constexpr int kXpBlock = 32;

size_t xpart_floats(const Dims& d, uint32_t cap) {
    const size_t xr_pad = (d.xr() + kRowTile - 1) / kRowTile * kRowTile;
    return (size_t)(d.di / kXpBlock) * cap * xr_pad;
}

size_t glimb_elems(const Dims& d, uint32_t cap) {
    const size_t groups = (cap + 15) / 16;
    return groups * (d.di / kKStep) * 3 * 64 * 8;
}

size_t xw_elems(const Dims& d, uint32_t cap) {
    const size_t groups = (cap + 15) / 16;
    const size_t ks = (d.d + kKAlign - 1) / kKAlign * (kKAlign / kKStep);
    return groups * ks * 3 * 64 * 8;
}

size_t ssp_floats(const Dims& d, uint32_t cap) { return (size_t)cap * (d.d / kRowTile); }

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kChunk = 32;                 // streams per k_head workgroup
constexpr int kGroups = kChunk / kRowTile; // MFMA column groups per chunk
constexpr int kInGroups = 1;               // column groups per k_mix_in workgroup
// Row tiles per k_mix_in workgroup: 2 up to kInWideFrom streams, 4 from there for int8
// weights with per-row scales.  F32 and column-group weights keep 2 at every batch size:
// their four-tile kernels hold one wave per SIMD (measured on Mamba-130M: 2 tiles are 3-5 %
// faster per step at 64, 128 and 256 streams).
constexpr int kInWideFrom = 64;
constexpr int kInChunk = kInGroups * kRowTile;
// Column groups (16 streams each) per k_mix_out workgroup: F32 weights take 2 from
// kOutWideFrom streams (their limb split then serves two groups), quantized weights always
// take 1 (measured on Mamba-130M int8: one group is 1-7 % faster per step from 64 to
// 1024 streams).  A stream's arithmetic does not depend on the choice.
constexpr int kOutWideFrom = 80;
// Chunk-major k_mix_out and k_mix_in grids from these many streams per part.  Measured on
// Mamba-130M int8, µs per step with neither / k_mix_out / both chunk major: 256 streams
// 917 / 907 / 907, 512 streams 1472 / 1451 / 1449, 1024 streams 2776 / 2723 / 2681; 128
// streams (two parts of 64) unchanged.  k_mix_in chunk major from 128 streams per part
// loses at 256 (922 against 908).
constexpr int kOutGroupMajorFrom = 128;
constexpr int kInGroupMajorFrom = 512;
constexpr int kHeadWaves = 8;              // waves per k_head workgroup (two per SIMD on one staged chunk)
constexpr int kHeadTiles = 2;              // row tiles per wave in k_head
// Weight k-pairs each wave keeps in flight (the product loop is unrolled by it): k_mix_in
// holds its whole quarter of four Q8 row tiles of a d <= 1024 projection, k_head four
// tiles' next eight pairs.
constexpr int kInRingQ8 = 4, kInRingF32 = 1;
constexpr int kHeadRingQ8 = 8, kHeadRingF32 = 2;
constexpr int kTps = 8;                    // threads per stream while staging activations
constexpr int kQuadBatch = 4;              // column quads a staging thread loads per iteration
constexpr int kMaxDr = 64;                 // dt_rank limit (d_model <= 1024)
constexpr int kMaxXr = kMaxDr + 32;        // x_proj rows
constexpr int kMaxNxb = 64;                // x_proj split-K blocks, d_inner / 32 (d_inner <= 2048)
constexpr int kOutWaves = 8;               // waves of k_mix_out
constexpr int kOutPairs = 3;               // k-pairs per k_mix_out wave per pass
constexpr int kInFixedPairs = 3;           // k_mix_in's fixed shape: three k-pairs per wave (d = 768)
static_assert(kSlotWordAlign % kInChunk == 0, "k_mix_in reads its chunk's slot words whole");

// Raw buffer access: a descriptor with a uniform base and an exact byte size (gfx9 word 3:
// 32-bit data format, untyped), a per-lane 32-bit byte offset and a uniform byte offset.
// Offsets past the size read 0 and drop stores, so every descriptor covers its array.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr int kBufWord3 = 0x00020000;
__device__ __forceinline__ BufRsrc buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufWord3);
}
// Cache policy of a buffer access (gfx9 "aux" bits): kStream = nt, for data read or
// written once per step (the recurrent state), so it does not displace reused lines.
constexpr int kCached = 0, kStream = 2;
template <int POLICY = kCached>
__device__ __forceinline__ float buf_ld_f32(BufRsrc r, uint32_t voff, uint32_t soff) {
    return bits_to_f(__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, POLICY));
}
__device__ __forceinline__ int4 buf_ld_i4(BufRsrc r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    return make_int4((int)v[0], (int)v[1], (int)v[2], (int)v[3]);
}
template <int POLICY = kCached>
__device__ __forceinline__ void buf_st_f32(float v, BufRsrc r, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b32(f_to_bits(v), r, (int)voff, (int)soff, POLICY);
}

__device__ __forceinline__ BufRsrc buf_rsrc_any(const void* base) { return buf_rsrc(base, 0x7fffffffu); }
template <int POLICY = kCached>
__device__ __forceinline__ int4 buf_ld_i4p(BufRsrc r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, POLICY);
    return make_int4((int)v[0], (int)v[1], (int)v[2], (int)v[3]);
}
__device__ __forceinline__ bf16x8 as_frag(int4 v) { return __builtin_bit_cast(bf16x8, v); }

// A store of what one phase hands to the next (u, z, x_proj partials, gated tiles, the
// residual and its pre-staged activations).  kCached: a plain store (the per-layer
// kernels, whose consumers start after the kernel boundary).  kCoherent (sc1): written
// through to the device's coherence point, so that a task of the persistent step kernel
// on any XCD reads it once the producer's phase counter says it is complete.  base is
// uniform, byte_off < 2 GiB.
constexpr int kCoherent = 16;
template <int AUX, class T>
__device__ __forceinline__ void st_hand(void* base, size_t byte_off, const T& v) {
    if constexpr (AUX == kCached) {
        *(T*)((unsigned char*)base + byte_off) = v;
    } else {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const BufRsrc r = buf_rsrc_any(base);
        const int off = (int)byte_off;
        if constexpr (sizeof(T) == 16)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, AUX);
        else if constexpr (sizeof(T) == 8)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, AUX);
        else if constexpr (sizeof(T) == 4)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, AUX);
        else {
            static_assert(sizeof(T) == 2, "2, 4, 8 or 16 bytes");
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), r, off, 0, AUX);
        }
    }
}

// ---------------------------------------------------------------- task synchronization

// A layer kernel's body runs either as a kernel of its own (NoWait: its inputs were
// complete when it started) or as a task of the persistent step kernel (FlowWait).  There
// the previous phase's outputs are written during the same launch by workgroups on any
// XCD: the task first requests everything that does not depend on them (weights, scales,
// recurrent state), then waits for the phase counter and reads those outputs.  Every
// layer of a step hands over through buffers of its own (written once per step), the
// producers write through to the coherence point (kStAux = sc1), their stores are complete
// (s_waitcnt) before the counter is raised, and the counter is read with device-scope
// atomics.  The consumers read with device scope too (kAux = sc1): some lines have writers
// on several XCDs (a stream's RMS partials of all 48 out_proj tiles, the gated limbs of
// 8 streams written by 4 scan tasks), and the L2 of an XCD that wrote part of such a line
// may hold it with the other XCDs' bytes from before they were written (default loads
// read such stale bytes now and then: one stream's logits differed at 150 streams).
// A stand-alone kernel reads what the previous kernel wrote with device scope as well (the
// kernel boundary has made it coherent either way; measured on Mamba-130M int8, µs per step
// default / device scope: one stream 353.0 / 350.3, 32 streams 382.3 / 379.8, 64 and 128
// streams the same; bits unchanged).
struct NoWait {
    static constexpr bool kFlow = false;
    static constexpr int kAux = kCoherent;
    static constexpr int kStAux = kCached;
    __device__ __forceinline__ void wait() const {}
};

// Polls of a wait before it gives up (each about a microsecond: 0.1 s or more, far past
// any phase of a step of at most kFlowMaxStreams streams): the task then sets bit 2 of the
// error word and goes on, and every later wait of the launch that finds the bit set gives
// up within 1024 polls, so every wave exits soon after a first failure.
constexpr uint32_t kFlowSpinMax = 1u << 17;
constexpr uint32_t kFlowCounterStride = 32;   // words between counters (one 128-byte line each)
// A phase counter is kFlowSlices counters, one per XCD (XCD x adds to slice x % kFlowSlices):
// the tasks of a phase end within a microsecond or so of each other, and their device-scope
// adds to one address are performed one after the other; on eight addresses they overlap.
constexpr uint32_t kFlowSlices = 8;

struct FlowWait {
    static constexpr bool kFlow = true;
    static constexpr int kAux = kCoherent;
    static constexpr int kStAux = kCoherent;
    const uint32_t* counter;   // slice 0 of the phase counter; null: nothing to wait for
    uint32_t target;           // sum of the slices when the phase is complete
    uint32_t* err;
    __device__ __forceinline__ void wait() const {
        // Wave 0 polls: lane s < kFlowSlices reads slice s, the wave sums them.
        if (threadIdx.x < kWave && counter != nullptr) {
            const uint32_t lane = threadIdx.x;
            const uint32_t* slice = counter + min(lane, kFlowSlices - 1) * kFlowCounterStride;
            uint32_t spins = 0;
            for (;;) {
                uint32_t v = __hip_atomic_load(slice, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                uint32_t sum = 0;
#pragma unroll
                for (uint32_t j = 0; j < kFlowSlices; j++) sum += __builtin_amdgcn_readlane(v, j);
                if (sum >= target) break;
                __builtin_amdgcn_s_sleep(1);
                if ((++spins & 1023u) == 0) {
                    const uint32_t e = __builtin_amdgcn_readfirstlane(
                        __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                    if (spins > kFlowSpinMax || (e & 4u)) {
                        if (lane == 0) atomicOr(err, 4u);
                        break;
                    }
                }
            }
        }
        // No cache maintenance follows: the lines the task reads next belong to this
        // layer's own hand-over buffers, which no CU or XCD has read in this launch before
        // the counter was complete (the kernel boundary invalidated what earlier steps read).
        __syncthreads();
    }
};

// ---------------------------------------------------------------- activation staging

// Norm of the chunk's streams and their bf16 limbs into LDS in B-fragment order:
// lds[((g*ks + s)*3 + limb)*512 + lane*8 + j] = limb of normed(x[b0 + 16g + lane%16])
// [32s + 8(lane/16) + j].  Streams >= n and columns >= d are zero.  RMSNorm
// x*inv*w with inv = 1/sqrt(mean(x^2) + 1e-5) (tensor.rs:900-908) or LayerNorm
// (tensor.rs:1390-1398).  Eight threads share a stream; each walks its column quads in
// order (kQuadBatch loads in flight), then the eight partials meet in a fixed xor
// butterfly (commutative pairings: every lane ends with the same bits).  The loops stay
// rolled: these kernels run once per CU per step, so their code must stay small.
__device__ __forceinline__ float4 quad_or_zero(const float4* p, int q, bool ok) {
    return ok ? p[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

__device__ void stage_normed(__bf16* lds, const float* __restrict__ x, const float* __restrict__ nw,
                             const float* __restrict__ nb, int d, int ks, uint32_t b0, uint32_t n, int streams) {
    const int bb = threadIdx.x / kTps, sub = threadIdx.x % kTps;
    const uint32_t b = b0 + bb;
    const bool live = b < n && bb < streams;
    const int dq = d / 4;
    const int qpt = ks * kKStep / 4 / kTps;  // quads per thread over the padded columns
    const float4* xb = (const float4*)(x + (size_t)(live ? b : b0) * d);
    float mean = 0.0f;
    if (nb != nullptr) {
        float s1 = 0.0f;
#pragma unroll 1
        for (int i0 = 0; i0 < qpt; i0 += kQuadBatch) {
            float4 v[kQuadBatch];
#pragma unroll
            for (int u = 0; u < kQuadBatch; u++) {
                const int q = sub + kTps * (i0 + u);
                v[u] = quad_or_zero(xb, q, live && i0 + u < qpt && q < dq);
            }
#pragma unroll
            for (int u = 0; u < kQuadBatch; u++) {
                s1 += v[u].x;
                s1 += v[u].y;
                s1 += v[u].z;
                s1 += v[u].w;
            }
        }
#pragma unroll
        for (int o = 1; o < kTps; o <<= 1) s1 += __shfl_xor(s1, o, kWave);
        mean = s1 / (float)d;
    }
    float ss = 0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < qpt; i0 += kQuadBatch) {
        float4 v[kQuadBatch];
#pragma unroll
        for (int u = 0; u < kQuadBatch; u++) {
            const int q = sub + kTps * (i0 + u);
            v[u] = quad_or_zero(xb, q, live && i0 + u < qpt && q < dq);
        }
#pragma unroll
        for (int u = 0; u < kQuadBatch; u++) {
            const int q = sub + kTps * (i0 + u);
            if (nb == nullptr) {
                ss += v[u].x * v[u].x;
                ss += v[u].y * v[u].y;
                ss += v[u].z * v[u].z;
                ss += v[u].w * v[u].w;
            } else if (q < dq) {
                const float c[4] = {v[u].x - mean, v[u].y - mean, v[u].z - mean, v[u].w - mean};
#pragma unroll
                for (int e = 0; e < 4; e++) ss += c[e] * c[e];
            }
        }
    }
#pragma unroll
    for (int o = 1; o < kTps; o <<= 1) ss += __shfl_xor(ss, o, kWave);
    const float inv = 1.0f / sqrtf(ss / (float)d + 1e-5f);
    const int g = bb / kRowTile;
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll 1
    for (int i0 = 0; i0 < qpt; i0 += kQuadBatch) {
        float4 v[kQuadBatch], w4[kQuadBatch], c4[kQuadBatch];
#pragma unroll
        for (int u = 0; u < kQuadBatch; u++) {
            const int q = sub + kTps * (i0 + u);
            const bool ok = live && i0 + u < qpt && q < dq;
            v[u] = quad_or_zero(xb, q, ok);
            w4[u] = quad_or_zero((const float4*)nw, q, ok);
            c4[u] = quad_or_zero((const float4*)nb, q, ok && nb != nullptr);
        }
#pragma unroll
        for (int u = 0; u < kQuadBatch; u++) {
            const int q = sub + kTps * (i0 + u);
            if (i0 + u >= qpt || bb >= streams) continue;
            const float xs[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            const float ws[4] = {w4[u].x, w4[u].y, w4[u].z, w4[u].w};
            const float cs[4] = {c4[u].x, c4[u].y, c4[u].z, c4[u].w};
            bf16x4 h, m, l;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float val = 0.0f;
                if (live && q < dq) val = nb == nullptr ? xs[e] * inv * ws[e] : (xs[e] - mean) * inv * ws[e] + cs[e];
                const Limb3 t3 = split3(val);
                h[e] = t3.h;
                m[e] = t3.m;
                l[e] = t3.l;
            }
            const int k0 = 4 * q, st = k0 / kKStep, within = k0 % kKStep;
            const int ln = (bb % kRowTile) + kRowTile * (within / 8);
            __bf16* dst = lds + ((size_t)(g * ks + st) * 3) * 512 + ln * 8 + (within % 8);
            *(bf16x4*)dst = h;
            *(bf16x4*)(dst + 512) = m;
            *(bf16x4*)(dst + 1024) = l;
        }
    }
    __syncthreads();
}

// Pre-staged activations (RMSNorm models).  The producer of the residual stream x
// (k_embed, k_mix_out) also writes x * norm_w as bf16 limbs in B-fragment tiles (xw) and
// partial sums of x^2 over each 16-column tile (ssp); a consumer copies its column groups'
// tiles straight into LDS and applies the per-stream RMS scale
// inv = 1 / sqrt(mean(x^2) + 1e-5) (tensor.rs:900-908) after the product:
// sum_k W[r][k] * (x[k] * w[k]) * inv.
//
// Copy of groups [g0, g0 + ng): contiguous in xw and in LDS, 1 KB per wave instruction
// (global_load_lds of 16 bytes per lane: lane i lands at LDS base + 16 i).  The caller
// waits for vmcnt(0) and syncs before reading.

__device__ __forceinline__ void stage_copy(unsigned char* lds, const __bf16* __restrict__ xw, uint32_t g0, int ng,
                                           int ks, int waves = kWaves) {
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const int blocks = ng * ks * 3;
    const __bf16* src = xw + (size_t)g0 * ks * 3 * 512 + lane * 8;
    lds_u8* dst = (lds_u8*)lds;
#pragma unroll 4
    for (int q = wave; q < blocks; q += waves)
        __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)q * 512), (void __attribute__((address_space(3)))*)(dst + q * kLimbBytes),
                                         16, 0, 0);
}

// RMS scale of the chunk's streams: eight threads per stream each take every eighth
// 16-column partial (up to kSspPerThread of them, all requested at once), then a fixed
// xor butterfly.  Split in a load half and a reduce half so the loads fly with the rest.
constexpr int kSspPerThread = 8;  // d <= 1024: at most 64 tiles

struct SspLoad {
    float v[kSspPerThread];
};

// Streams [b0, b0 + streams) of the workgroup; threads past them load a valid row that
// is never used.  The loads are unconditional (clamped rows and tiles) so that they are
// issued in straight-line code with the caller's other loads; ssp_reduce masks them.
// AUX: the cache policy (L1-bypassing inside the persistent step kernel).
template <int AUX = kCached>
__device__ __forceinline__ SspLoad ssp_load(const float* __restrict__ ssp, int tiles, uint32_t b0, uint32_t n,
                                            int streams) {
    const int bb = threadIdx.x / kTps, sub = threadIdx.x % kTps;
    const uint32_t b = b0 + bb;
    const bool on = bb < streams && b < n;
    SspLoad r;
    if constexpr (AUX == kCached) {
        const float* p = ssp + (size_t)(on ? b : 0) * tiles;
#pragma unroll
        for (int i = 0; i < kSspPerThread; i++) r.v[i] = p[min(sub + kTps * i, tiles - 1)];
    } else {
        const BufRsrc rs = buf_rsrc_any(ssp);
        const uint32_t row = (on ? b : 0u) * (uint32_t)tiles;
#pragma unroll
        for (int i = 0; i < kSspPerThread; i++)
            r.v[i] = buf_ld_f32<AUX>(rs, (row + (uint32_t)min(sub + kTps * i, tiles - 1)) * 4u, 0);
    }
    return r;
}

__device__ __forceinline__ void ssp_reduce(const SspLoad& r, float* invs, int tiles, int d, int streams) {
    const int bb = threadIdx.x / kTps, sub = threadIdx.x % kTps;
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kSspPerThread; i++)
        if (sub + kTps * i < tiles) ss += r.v[i];
#pragma unroll
    for (int o = 1; o < kTps; o <<= 1) ss += __shfl_xor(ss, o, kWave);
    if (sub == 0 && bb < streams) invs[bb] = 1.0f / sqrtf(ss / (float)d + 1e-5f);
}

// Producer side for one 16-column tile: lane l of the wave holds x[b][r0 + i], i < 4,
// r0 = 16 t + 4 (l / 16), b = b0 + (l % 16) (the MFMA D layout).  Writes the three limbs of
// x * w into column group b / 16 of xw and the tile's sum of x^2 for stream b into ssp
// (sequential over the lane's four values, then xor 16, xor 32).  All lanes must call it;
// `ok` masks the stores.
template <int AUX = kCached>
__device__ __forceinline__ void produce_tile(__bf16* __restrict__ xw, float* __restrict__ ssp, int ks, int tiles,
                                             int t, uint32_t b, bool ok, const float (&xv)[4], const float4& w4) {
    const int lane = threadIdx.x % kWave;
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
    float v[4];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[i] = xv[i] * wv[i];
        ss += xv[i] * xv[i];
    }
    ss += __shfl_xor(ss, 16, kWave);
    ss += __shfl_xor(ss, 32, kWave);
    if (!ok) return;
    write_limbs4<AUX>(xw, ks, t, b, v);
    if (lane < 16) st_hand<AUX>(ssp, ((size_t)b * tiles + t) * 4, ss);
}

// Row tiles a wave multiplies together, with a ring of their next R weight k-pairs
// (requested ahead of the product, for instance while the activations stage).
template <bool Q8, int T, int R>
struct Tiles {
    int t[T];
    bool ok[T];
    RawPair ring[R][T];
};

template <bool Q8, int T, int R>
__device__ __forceinline__ void tiles_prefetch(const TMat& w, Tiles<Q8, T, R>& tl, int p_lo, int p_hi) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int q = 0; q < R; q++)
#pragma unroll
        for (int i = 0; i < T; i++)
            if (tl.ok[i] && p_lo + q < p_hi) tl.ring[q][i] = load_pair<Q8>(w, tl.t[i], p_lo + q, lane);
}

// T row tiles times the staged activations of `ng` column groups over k-pairs
// [p_lo, p_hi).  Accumulators are kept per limb order so consecutive MFMAs are
// independent: Q8 order o holds the products with activation limb o; F32 order 0 holds
// hi*hi, order 1 hi*mid and mid*hi, order 2 hi*lo, mid*mid and lo*hi.  The sum is
// (o0 + o1) + o2.  With Q8 group-64 scales each k-pair's partial (all limbs, fixed order)
// is scaled into order 0.  The weight ring is refilled R pairs ahead; the loop body
// covers one turn of the ring and stays rolled.  Per-row scales are left to the caller.
template <bool Q8, int T, int R>
__device__ __forceinline__ void tiles_gemm(const TMat& w, Tiles<Q8, T, R>& tl, const __bf16* lds, int ng, int p_lo,
                                           int p_hi, f32x4 (&out)[T][kGroups]) {
    const int lane = threadIdx.x % kWave;
    const bool grp = Q8 && w.group != w.cols;
    const int gpr = w.ks / 2;
    f32x4 acc[T][kGroups][3];
#pragma unroll
    for (int i = 0; i < T; i++)
#pragma unroll
        for (int g = 0; g < kGroups; g++)
#pragma unroll
            for (int o = 0; o < 3; o++) acc[i][g][o] = f32x4{0, 0, 0, 0};
#pragma unroll 1
    for (int p0 = p_lo; p0 < p_hi; p0 += R) {
#pragma unroll
        for (int q = 0; q < R; q++) {
            const int p = p0 + q;
            if (p >= p_hi) continue;
            bf16x8 bf[kGroups][2][3];
#pragma unroll
            for (int g = 0; g < kGroups; g++) {
                if (g >= ng) continue;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const __bf16* f = lds + ((size_t)(g * w.ks + 2 * p + h) * 3) * 512 + lane * 8;
#pragma unroll
                    for (int m = 0; m < 3; m++) bf[g][h][m] = lds_frag(f + m * 512);
                }
            }
#pragma unroll
            for (int i = 0; i < T; i++) {
                if (!tl.ok[i]) continue;
                const RawPair cur = tl.ring[q][i];
                if (p + R < p_hi) tl.ring[q][i] = load_pair<Q8>(w, tl.t[i], p + R, lane);
                AFrag a[2];
                decode_pair<Q8>(cur, a[0], a[1]);
                float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
                if (grp) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        sc[e] = w.scales[(size_t)(tl.t[i] * kRowTile + (lane / 16) * 4 + e) * gpr + p];
                }
#pragma unroll
                for (int g = 0; g < kGroups; g++) {
                    if (g >= ng) continue;
                    if (grp) {
                        f32x4 tmp{0, 0, 0, 0};
#pragma unroll
                        for (int h = 0; h < 2; h++) tmp = mma_step<Q8>(a[h], bf[g][h][0], bf[g][h][1], bf[g][h][2], tmp);
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[i][g][0][e] = __builtin_fmaf(tmp[e], sc[e], acc[i][g][0][e]);
                    } else {
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            if (Q8) {
                                acc[i][g][0] = mma(a[h].h, bf[g][h][0], acc[i][g][0]);
                                acc[i][g][1] = mma(a[h].h, bf[g][h][1], acc[i][g][1]);
                                acc[i][g][2] = mma(a[h].h, bf[g][h][2], acc[i][g][2]);
                            } else {
                                acc[i][g][0] = mma(a[h].h, bf[g][h][0], acc[i][g][0]);
                                acc[i][g][1] = mma(a[h].h, bf[g][h][1], acc[i][g][1]);
                                acc[i][g][1] = mma(a[h].m, bf[g][h][0], acc[i][g][1]);
                                acc[i][g][2] = mma(a[h].h, bf[g][h][2], acc[i][g][2]);
                                acc[i][g][2] = mma(a[h].m, bf[g][h][1], acc[i][g][2]);
                                acc[i][g][2] = mma(a[h].l, bf[g][h][0], acc[i][g][2]);
                            }
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < T; i++)
#pragma unroll
        for (int g = 0; g < kGroups; g++) out[i][g] = (acc[i][g][0] + acc[i][g][1]) + acc[i][g][2];
}

// k_mix_in's product: the block's T row tiles times its column groups over this
// wave's k-pairs [p_lo, p_lo + cnt), cnt <= kQuarterMax.  The weights of the quarter are
// requested up front into a ring of R pairs (Q8: the whole quarter; F32 refills R pairs
// ahead).  One accumulator per (tile, group): per k-step the limb products go in the
// order hi, mid, lo (F32: hi*hi, hi*mid, mid*hi, hi*lo, mid*mid, lo*hi), issued across
// the tiles so that no MFMA waits for its predecessor.  Tiles past the matrix are clamped to its
// last tile and column groups past n read whatever the LDS holds: both only feed output
// elements that are never stored (MFMA output columns depend only on their own B column).
constexpr int kQuarterMax = 4;  // k-pairs per wave: d <= 1024 is 16 pairs over 4 waves

// Slot q of a quarter of cnt pairs loads pair p_lo + quarter_slot(q, cnt): slots past the
// quarter repeat its last pair, and a wave with no pairs (fewer k-pairs than waves) loads
// pair p_lo, which is always a pair of the matrix (p_lo = floor(wave np / kWaves) < np).
// Such loads are never used.
__device__ __forceinline__ int quarter_slot(int q, int cnt) { return max(min(q, cnt - 1), 0); }

template <bool Q8, int R, int T>
struct Quarter {
    RawPair ring[R][T];
};

// The activation (B) fragments of a wave's quarter, [k-pair][group][k-step of the pair]
// [limb].  No other wave reads them, so with pre-staged activations they are loaded from
// the tiles in global memory straight into registers.  CNT > 0 is the quarter's exact
// k-pair count; otherwise every slot is loaded as quarter_slot says.
template <int G>
struct BQuarter {
    bf16x8 f[kQuarterMax][G][2][3];
};

template <int G, int CNT, int AUX = kCached>
__device__ __forceinline__ void bquarter_load(BQuarter<G>& bq, const __bf16* __restrict__ xw, uint32_t g0, int ng,
                                              int ks, int p_lo, int cnt) {
    const int lane = threadIdx.x % kWave;
    constexpr int Q = CNT > 0 ? CNT : kQuarterMax;
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int gg = G > 1 ? min(g, ng - 1) : g;
        const __bf16* base = xw + ((size_t)(g0 + gg) * ks + 2 * p_lo) * 3 * 512;
        const BufRsrc rb = buf_rsrc_any(base);
#pragma unroll
        for (int q = 0; q < Q; q++) {
            const int qq = CNT > 0 ? q : quarter_slot(q, cnt);
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int m = 0; m < 3; m++) {
                    const int off = ((2 * qq + h) * 3 + m) * 512 + lane * 8;
                    if constexpr (AUX == kCached)
                        bq.f[q][g][h][m] = lds_frag(base + off);
                    else
                        bq.f[q][g][h][m] = as_frag(buf_ld_i4p<AUX>(rb, (uint32_t)off * 2u, 0));
                }
        }
    }
}

// The same fragments from activations staged in LDS (the LayerNorm path, normed in place).
template <int G>
__device__ __forceinline__ void bquarter_lds(BQuarter<G>& bq, const __bf16* lds, int ks, int p_lo, int cnt) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int q = 0; q < kQuarterMax; q++) {
        const int qq = quarter_slot(q, cnt);
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const __bf16* f = lds + ((size_t)(g * ks + 2 * (p_lo + qq) + h) * 3) * 512 + lane * 8;
#pragma unroll
                for (int m = 0; m < 3; m++) bq.f[q][g][h][m] = lds_frag(f + m * 512);
            }
    }
}

// Every ring slot is filled (loads in straight-line code, so none of them waits for
// another; the extra copies are unused).
template <bool Q8, int R, int T>
__device__ __forceinline__ void quarter_prefetch(const TMat& w, Quarter<Q8, R, T>& qw, int tb, int p_lo, int cnt) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int q = 0; q < R; q++)
#pragma unroll
        for (int i = 0; i < T; i++)
            qw.ring[q][i] = load_pair<Q8>(w, min(tb + i, w.rt - 1), p_lo + quarter_slot(q, cnt), lane);
}

template <bool Q8, bool GRP, int R, int T, int G>
__device__ __forceinline__ void quarter_gemm(const TMat& w, Quarter<Q8, R, T>& qw, int tb, const BQuarter<G>& bq,
                                             int p_lo, int cnt, f32x4 (&out)[T][G]) {
    const int lane = threadIdx.x % kWave;
    const int gpr = w.ks / 2;
#pragma unroll
    for (int i = 0; i < T; i++)
#pragma unroll
        for (int g = 0; g < G; g++) out[i][g] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < kQuarterMax; q++) {
        if (q >= cnt) continue;
        const int p = p_lo + q;
        const bf16x8 (&bf)[G][2][3] = bq.f[q];
        AFrag a[T][2];
        float sc[T][4];
#pragma unroll
        for (int i = 0; i < T; i++) {
            const RawPair cur = qw.ring[q % R][i];
            if (R < kQuarterMax && q + R < cnt) qw.ring[q % R][i] = load_pair<Q8>(w, min(tb + i, w.rt - 1), p + R, lane);
            decode_pair<Q8>(cur, a[i][0], a[i][1]);
            if (GRP) {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    sc[i][e] = w.scales[(size_t)(min(tb + i, w.rt - 1) * kRowTile + (lane / 16) * 4 + e) * gpr + p];
            }
        }
        // Product by product across the tiles: consecutive MFMAs feed different
        // accumulators, and each accumulator still takes mma_step's order, k-step by k-step.
        f32x4 tmp[T][G];
#pragma unroll
        for (int i = 0; i < T; i++)
#pragma unroll
            for (int g = 0; g < G; g++) tmp[i][g] = GRP ? f32x4{0, 0, 0, 0} : out[i][g];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int j = 0; j < kProds<Q8>; j++)
#pragma unroll
                for (int g = 0; g < G; g++)
#pragma unroll
                    for (int i = 0; i < T; i++)
                        tmp[i][g] = mma_prod<Q8>(j, a[i][h], bf[g][h][0], bf[g][h][1], bf[g][h][2], tmp[i][g]);
#pragma unroll
        for (int i = 0; i < T; i++)
#pragma unroll
            for (int g = 0; g < G; g++) {
                if (GRP) {
#pragma unroll
                    for (int e = 0; e < 4; e++) out[i][g][e] = __builtin_fmaf(tmp[i][g][e], sc[i][e], out[i][g][e]);
                } else {
                    out[i][g] = tmp[i][g];
                }
            }
    }
}

__device__ __forceinline__ void apply_row_scales(const TMat& w, int t, f32x4 (&acc)[kGroups], int ng) {
    if (w.group == 0 || w.group != w.cols) return;
    const int lane = threadIdx.x % kWave;
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sc[i] = w.scales[t * kRowTile + (lane / 16) * 4 + i];
#pragma unroll
    for (int g = 0; g < kGroups; g++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[g][i] = acc[g][i] * sc[i];
}

// ---------------------------------------------------------------- embedding

struct EmbedArgs {
    TMat emb;
    float* x;                  // [n][d]
    const uint32_t* tokens;    // caller's device pointers, at this part's first row
    const uint32_t* slots_in;
    uint32_t* slots;           // validated copy used by the rest of the step
    uint32_t n, cap;
    int check;
    uint32_t* err;
    const uint32_t* slots_all; // the whole step's slots (the check covers every part)
    uint32_t n_all, b_off;     // streams of the whole step; this part's first row in it
    uint32_t* zero;            // counters of the persistent step kernel to clear (or null):
    uint32_t zero_n, zero_stride;  // zero[i * zero_stride] for i < zero_n
    const float* nw0;          // layer 0 norm weight; with xw != null the pre-staged
    __bf16* xw;                // activations of layer 0 are produced here
    float* ssp;
    int ks_x, tiles;
};

// x[b] = emb[token[b]] (Q8: q * scale), model.rs:93-101 / gemv.rs:285-295.  Block (0, b)
// copies slot b into the step's slot list; with `check` it also validates the slot and
// the token and looks for duplicate slots, recording failures in *err.  An entry with a
// bad slot or token, or whose slot an earlier entry of the batch already names, is
// routed to the pool's scratch slot (index cap), so it never touches a real slot's state
// and no two streams of the step share one; its token is clamped into the vocabulary.  Thread q of block (x, b) owns columns 4q' .. 4q'+3,
// q' = 256 x + q; with xw it also writes their x * w limbs and, four threads per
// 16-column tile, the tile's sum of x^2 (sequential over the four, then xor 1, xor 2).
__global__ __launch_bounds__(kBlock) void k_embed(EmbedArgs a) {
    const uint32_t b = blockIdx.y;
    const int d = a.emb.cols;
    uint32_t tok = a.tokens[b];
    if (blockIdx.x == 0) {
        const uint32_t s = a.slots_in[b];
        if (a.check) {
            __shared__ int earlier;
            if (threadIdx.x == 0) earlier = 0;
            __syncthreads();
            const uint32_t gb = a.b_off + b;   // this entry's row in the whole step
            bool dup = false, first_dup = false;
            for (uint32_t c = threadIdx.x; c < a.n_all; c += blockDim.x)
                if (c != gb && a.slots_all[c] == s) {
                    dup = true;
                    if (c < gb) first_dup = true;
                }
            if (first_dup) earlier = 1;   // benign same-value race on the flag
            const bool bad = tok >= (uint32_t)a.emb.rows || s >= a.cap;
            if (threadIdx.x == 0 && bad) atomicOr(a.err, 1u);
            if (dup) atomicOr(a.err, 2u);
            __syncthreads();
            if (threadIdx.x == 0) a.slots[b] = bad || earlier ? a.cap : s;
        } else if (threadIdx.x == 0) {
            a.slots[b] = clamp_slot(s, a.cap);
        }
    }
    if (a.zero != nullptr && blockIdx.x == 0)
        for (uint32_t i = b * kBlock + threadIdx.x; i < a.zero_n; i += a.n * kBlock) a.zero[(size_t)i * a.zero_stride] = 0u;
    if (tok >= (uint32_t)a.emb.rows) tok = a.emb.rows - 1;
    const int k = 4 * (blockIdx.x * kBlock + threadIdx.x);
    const bool live = k < d;
    const int s = k / kKStep, j = k % 8;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
        const int t = tok / kRowTile;
        const int ln = (tok % kRowTile) + kRowTile * ((k % kKStep) / 8);
        if (a.emb.group == 0) {
            const float4 f = *(const float4*)((const float*)a.emb.w + (((size_t)t * a.emb.ks + s) * 64 + ln) * 8 + j);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        } else {
            const int8_t* q8 = (const int8_t*)a.emb.w;
            const int packed = *(const int*)(q8 + ((((size_t)t * (a.emb.ks / 2) + s / 2) * 64 + ln) * 2 + s % 2) * 8 + j);
            const float sc = a.emb.group == a.emb.cols ? a.emb.scales[tok]
                                                       : a.emb.scales[(size_t)tok * (a.emb.ks / 2) + k / a.emb.group];
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = (float)(int8_t)(packed >> (8 * e)) * sc;
        }
        *(float4*)(a.x + (size_t)b * d + k) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (a.xw == nullptr) return;
    const float4 w4 = live ? *(const float4*)(a.nw0 + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 h, m, l;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const Limb3 t3 = split3(v[e] * wv[e]);
        h[e] = t3.h;
        m[e] = t3.m;
        l[e] = t3.l;
        ss += v[e] * v[e];
    }
    ss += __shfl_xor(ss, 1, kWave);
    ss += __shfl_xor(ss, 2, kWave);
    if (!live) return;
    const int ln = (int)(b % kRowTile) + kRowTile * ((k % kKStep) / 8);
    __bf16* dst = a.xw + ((((size_t)(b / kRowTile) * a.ks_x + s) * 3) * 64 + ln) * 8 + j;
    *(bf16x4*)dst = h;
    *(bf16x4*)(dst + 512) = m;
    *(bf16x4*)(dst + 1024) = l;
    if (threadIdx.x % 4 == 0) a.ssp[(size_t)b * a.tiles + k / kRowTile] = ss;
}

// ---------------------------------------------------------------- k_mix_in

struct MixInArgs {
    const float* x;            // [n][d] residual stream (LayerNorm path)
    const float* norm_w;
    const float* norm_b;
    TMat wx, wz, wxp;          // in_proj conv branch, gate branch; x_proj
    int nxb;                   // conv-branch workgroups (16 T channels each)
    float* conv_st;            // this layer's conv state, [slot][di][dc-1]
    const float* conv_w;
    const float* conv_b;
    const uint32_t* slots;
    uint32_t cap, n;           // batch rows of the x_proj partials (their row stride), streams
    uint32_t scap;             // state slots (conv state rows; the slot clamp bound)
    float* u;                  // [n][di]
    float* z;                  // [n][di]
    float* xpart;              // [di / 32][cap][xr_pad] (32-channel x_proj partials)
    int di, dc, d, xr_pad;
    const __bf16* xw;          // pre-staged activations (RMSNorm path)
    const float* ssp;
    int tiles;
    uint32_t gmajor = 0;       // grid (chunks, blocks) instead of (blocks, chunks)
};

// in_proj for T row tiles (T = 2 or 4) x kInChunk streams, 4 waves.  The product is split
// over k: wave w multiplies the block's T tiles over k-pairs [w np / 4, (w + 1) np / 4).
// The quarters meet in LDS and are added in wave order, q0 + q1 + q2 + q3; wave w then
// finishes 4 T rows: tile w T / 4, rows 4 T (w % (4 / T)) .. + 4 T, E = T consecutive rows
// (channels) per lane, lane l for stream l % 16.  Every vector load is issued up front,
// in the order of first use: the quarter's weights and activations (the pre-staged tiles,
// straight into registers), the RMS partials, row scales, conv weights, x_proj fragments
// and the conv state.  A conv-branch block owns 16 T channels, T / 2 k-steps of x_proj,
// and leaves k_scan one split-K partial per k-step (32 channels), whatever T is, so every
// batch size sums the same partials.  Two tiles give more, smaller workgroups (small
// batches); four read each stream's activations half as often.
template <bool Q8, bool Q8XP, bool PRE, bool GRP, int QP, int T, class SYNC>
__device__ __forceinline__ void mix_in_body(const MixInArgs& a, uint32_t bx, uint32_t by, const SYNC& sync) {
    static_assert(kInGroups == 1 && (T == 2 || T == 4) && kWaves == 4, "one stream group, 2 or 4 tiles");
    static_assert(!SYNC::kFlow || PRE, "persistent tasks take pre-staged activations");
    constexpr int E = T;                   // rows per lane in the finish
    constexpr int WT = kWaves / T;         // waves per tile in the finish
    constexpr int KS = T / 2;              // x_proj k-steps per block
    typedef float fE __attribute__((ext_vector_type(E)));
    typedef __bf16 bfE __attribute__((ext_vector_type(E)));
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float invs[kInChunk];
    __bf16* lds = (__bf16*)smem;
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const uint32_t b0 = by * kInChunk;
    const bool conv_branch = (int)bx < a.nxb;
    const TMat& w = conv_branch ? a.wx : a.wz;
    const int tb = (conv_branch ? (int)bx : (int)bx - a.nxb) * T;  // the block's first row tile
    // The rows this wave finishes and this lane's E rows and stream.
    const int tf = wave / WT;
    const int r0 = (wave % WT) * (kRowTile / WT) + (lane / 16) * E;  // row within the tile
    const int ch = (tb + tf) * kRowTile + r0;                        // channel of the first row
    const uint32_t b = b0 + lane % 16;
    const bool has_rows = tb + tf < w.rt;
    const int dc = a.dc;
    // QP > 0: every wave takes exactly QP k-pairs (w.ks = 2 kWaves QP, checked on the host).
    const int np = w.ks / 2;
    const int p_lo = QP > 0 ? wave * QP : wave * np / kWaves, p_hi = QP > 0 ? p_lo + QP : (wave + 1) * np / kWaves;
    // The stream's slot by scalar loads, first: they do not count on the vector memory
    // counter.  The slot list is allocated in whole kSlotWordAlign blocks; a word past n
    // feeds only a stream that is never stored (and is clamped like any other).
    uint32_t slot_raw;
    {
        // Constant address space: the list is read-only for this kernel, and uniform loads
        // from that space always go through the scalar unit.
        const __attribute__((address_space(4))) uint32_t* sp =
            (const __attribute__((address_space(4))) uint32_t*)(a.slots + b0);
        uint32_t sv[kRowTile];
#pragma unroll
        for (int q = 0; q < kRowTile; q += 4) {
            sv[q] = sp[q];
            sv[q + 1] = sp[q + 1];
            sv[q + 2] = sp[q + 2];
            sv[q + 3] = sp[q + 3];
            // Pinned to scalar registers: otherwise the per-lane select below is folded
            // back into a per-lane vector load of the selected word.
            asm volatile("" : "+s"(sv[q]), "+s"(sv[q + 1]), "+s"(sv[q + 2]), "+s"(sv[q + 3]));
        }
        slot_raw = sv[0];
#pragma unroll
        for (int i = 1; i < kRowTile; i++) slot_raw = lane % 16 == i ? sv[i] : slot_raw;
    }
    // The ring holds a Q8 quarter whole: exactly QP pairs when the shape is fixed.
    constexpr int R = Q8 ? (QP > 0 ? QP : kInRingQ8) : kInRingF32;
    Quarter<Q8, R, T> qw;
    quarter_prefetch<Q8, R, T>(w, qw, tb, p_lo, p_hi - p_lo);
    BQuarter<1> bq;
    SspLoad sl;
    if constexpr (PRE && !SYNC::kFlow) {
        bquarter_load<1, QP, SYNC::kAux>(bq, a.xw, b0 / kRowTile, 1, a.wx.ks, p_lo, p_hi - p_lo);
        sl = ssp_load<SYNC::kAux>(a.ssp, a.tiles, b0, a.n, kInChunk);
    }
    // Per-row scales of the lane's rows (Q8 without column groups); rows past the matrix
    // read its last ones and are never stored.
    const int chc = min(ch, w.rt * kRowTile - E);
    fE rsc;
#pragma unroll
    for (int e = 0; e < E; e++) rsc[e] = 1.0f;
    if (Q8 && !GRP) rsc = *(const fE*)(w.scales + chc);
    // Conv weights and bias of the lane's channels (used when dc = 4), loaded by every lane
    // from indices clamped into the arrays: no branch in the load prologue.
    f32x4 cwv[E];
    fE cbv;
    {
        const int jc = min(ch, a.di - E);
        const f32x4* cw4 = (const f32x4*)(a.conv_w + min(jc * 4, a.di * dc - 4 * E));
#pragma unroll
        for (int e = 0; e < E; e++) cwv[e] = cw4[e];
        cbv = *(const fE*)(a.conv_b + jc);
    }
    // x_proj fragments of this block's k-pair (T = 4) or k-step p (T = 2: half p % 2 of
    // pair p / 2): row tiles wave and wave + 4 (x_proj has at most kMaxXr / 16 = 6 row
    // tiles), with their scales; loaded by every block from clamped, in-bounds tiles (a
    // gate-branch block or a tile past x_proj's rows reads the last one and never uses it).
    // Column-group scales take the block's 64-column group, one scale per row r.
    const int p = min((int)bx, a.nxb - 1);
    const int xpair = p * KS / 2;
    RawPair xpw[2];
    float4 xps[2];
    {
        const bool grp = a.wxp.group != a.wxp.cols;
        const size_t gs = grp ? (size_t)(a.wxp.ks / 2) : 1, po = grp ? (size_t)xpair : 0;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int tp = min(wave + kWaves * k, a.wxp.rt - 1);
            xpw[k] = load_pair<Q8XP>(a.wxp, tp, xpair, lane);
            const size_t r = (size_t)tp * kRowTile + (lane / 16) * 4;
            xps[k] = Q8XP ? make_float4(a.wxp.scales[r * gs + po], a.wxp.scales[(r + 1) * gs + po],
                                        a.wxp.scales[(r + 2) * gs + po], a.wxp.scales[(r + 3) * gs + po])
                          : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
        }
    }
    // Conv state of the lane's channels (used when dc = 4 on the conv branch): three loads
    // of E floats from an offset clamped into the state buffer; streamed (non-temporal), as
    // the state is read and written once per step.
    const uint32_t slot = conv_branch ? clamp_slot(slot_raw, a.scap) : 0u;
    const size_t conv_floats = (size_t)a.scap * a.di * (dc - 1);
    fE stv[3];
    {
        const size_t off = min(((size_t)slot * a.di + min(ch, a.di - E)) * 3, conv_floats - 3 * E);
        const fE* sp = (const fE*)(a.conv_st + off);
#pragma unroll
        for (int k = 0; k < 3; k++) stv[k] = __builtin_nontemporal_load(sp + k);
    }
    // As a task: the previous phase's outputs (the activation tiles and RMS partials) once
    // its counter is complete, everything else already in flight.
    if constexpr (PRE && SYNC::kFlow) {
        sync.wait();
        bquarter_load<1, QP, SYNC::kAux>(bq, a.xw, b0 / kRowTile, 1, a.wx.ks, p_lo, p_hi - p_lo);
        sl = ssp_load<SYNC::kAux>(a.ssp, a.tiles, b0, a.n, kInChunk);
    }
    // Every load above is issued before anything that waits for one of them.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!PRE) {
        stage_normed(lds, a.x, a.norm_w, a.norm_b, a.d, a.wx.ks, b0, a.n, kInChunk);
        bquarter_lds<1>(bq, lds, a.wx.ks, p_lo, p_hi - p_lo);
    }

    f32x4 q4[T][1];
    quarter_gemm<Q8, GRP, R, T, 1>(w, qw, tb, bq, p_lo, p_hi - p_lo, q4);
    // The RMS scales are first needed after the barrier below.
    if constexpr (PRE) ssp_reduce(sl, invs, a.tiles, a.d, kInChunk);
    // Quarters through LDS: red[src wave][tile][lane] in the MFMA D layout (on the
    // LayerNorm path over the staged activations, once every wave has read them).
    if constexpr (!PRE) __syncthreads();
    f32x4* red = (f32x4*)smem;
#pragma unroll
    for (int i = 0; i < T; i++) red[(wave * T + i) * kWave + lane] = q4[i][0];
    __syncthreads();
    // Rows r0 .. r0 + E - 1 of stream lane % 16 sit in D-layout lane (lane % 16) + 16 (r0 / 4),
    // components r0 % 4 .. r0 % 4 + E - 1.
    float v[E];
    {
        const int src_lane = lane % 16 + 16 * (r0 / 4);
        const float* rf = (const float*)red;
        fE sum;
#pragma unroll
        for (int src = 0; src < kWaves; src++) {
            const fE x = *(const fE*)(rf + ((src * T + tf) * kWave + src_lane) * 4 + r0 % 4);
            sum = src == 0 ? x : sum + x;
        }
#pragma unroll
        for (int e = 0; e < E; e++) {
            float y = sum[e];
            if (Q8 && !GRP) y = y * rsc[e];
            if constexpr (PRE) y = y * invs[lane % 16];
            v[e] = y;
        }
    }
    if (!conv_branch) {
        if (has_rows && b < a.n) {
            fE zv;
#pragma unroll
            for (int e = 0; e < E; e++) zv[e] = v[e];
            st_hand<SYNC::kStAux>(a.z, ((size_t)b * a.di + ch) * 4, zv);
        }
        return;
    }
    // Conv branch: conv1d step + SiLU per (channel, stream), conv_silu_block order
    // (model.rs:134-153).  silu_inplace takes lane_sigmoid for the 8-aligned body of each
    // 256-channel block and the scalar sigmoid for the rest (tensor.rs:1207-1211); d_inner
    // comes in whole 64-channel blocks here, so every channel is in a body.
    float uv[E];
#pragma unroll
    for (int e = 0; e < E; e++) uv[e] = 0.0f;
    if (has_rows && b < a.n) {
        if (dc == 4) {
            float st[3 * E];
#pragma unroll
            for (int k = 0; k < 3; k++)
#pragma unroll
                for (int e = 0; e < E; e++) st[k * E + e] = stv[k][e];
#pragma unroll
            for (int e = 0; e < E; e++) {
                const float xv = v[e];
                float val = 0.0f;
                val += st[3 * e] * cwv[e][0];
                val += st[3 * e + 1] * cwv[e][1];
                val += st[3 * e + 2] * cwv[e][2];
                val += xv * cwv[e][3];
                val += cbv[e];
                st[3 * e] = st[3 * e + 1];
                st[3 * e + 1] = st[3 * e + 2];
                st[3 * e + 2] = xv;
                uv[e] = val;
            }
            fE* sp = (fE*)(a.conv_st + ((size_t)slot * a.di + ch) * 3);
#pragma unroll
            for (int k = 0; k < 3; k++) {
                fE o;
#pragma unroll
                for (int e = 0; e < E; e++) o[e] = st[k * E + e];
                __builtin_nontemporal_store(o, sp + k);
            }
        } else {
#pragma unroll
            for (int e = 0; e < E; e++) {
                const int j = ch + e;
                float* st = a.conv_st + ((size_t)slot * a.di + j) * (dc - 1);
                const float* cw = a.conv_w + (size_t)j * dc;
                const float xv = v[e];
                float val = 0.0f;
                for (int k = 0; k < dc - 1; k++) val += st[k] * cw[k];
                val += xv * cw[dc - 1];
                val += a.conv_b[j];
                for (int k = 0; k + 2 < dc; k++) st[k] = st[k + 1];
                st[dc - 2] = xv;
                uv[e] = val;
            }
        }
        fE uo;
#pragma unroll
        for (int e = 0; e < E; e++) {
            uv[e] = uv[e] * lane_sigmoid_f(uv[e]);
            uo[e] = uv[e];
        }
        st_hand<SYNC::kStAux>(a.u, ((size_t)b * a.di + ch) * 4, uo);
    }
    // u as the B operand of x_proj over this block's 16 T channels (KS k-steps), past the
    // quarters: local channel c = 16 tf + r0 (+ e) of stream lane % 16 goes to k-step c / 32,
    // B lane (lane % 16) + 16 ((c % 32) / 8), element c % 8; a lane's E channels share it.
    __bf16* xop = lds + T * kWaves * kWave * 8;   // past red (bf16 elements)
    {
        const int c = tf * kRowTile + r0;
        const int ln = lane % 16 + kRowTile * ((c % kKStep) / 8);
        bfE h, m, l;
#pragma unroll
        for (int e = 0; e < E; e++) {
            const Limb3 t3 = split3(uv[e]);
            h[e] = t3.h;
            m[e] = t3.m;
            l[e] = t3.l;
        }
        __bf16* dst = xop + (c / kKStep) * 3 * 512 + ln * 8 + c % 8;
        *(bfE*)dst = h;
        *(bfE*)(dst + 512) = m;
        *(bfE*)(dst + 1024) = l;
    }
    __syncthreads();
    // Split-K partials of x_proj, one per k-step (32 channels): its row tiles against
    // this block's channels; partial block p KS + s.
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int tp = wave + kWaves * k;
        if (tp >= a.wxp.rt) continue;
        AFrag a0, a1;
        decode_pair<Q8XP>(xpw[k], a0, a1);
        const float xs[4] = {xps[k].x, xps[k].y, xps[k].z, xps[k].w};
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const AFrag& af = KS == 2 ? (s ? a1 : a0) : (p % 2 ? a1 : a0);
            const __bf16* f = xop + s * 3 * 512 + lane * 8;
            f32x4 part{0, 0, 0, 0};
            part = mma_step<Q8XP>(af, lds_frag(f), lds_frag(f + 512), lds_frag(f + 1024), part);
            if (b < a.n) {
                const size_t dst = ((size_t)(p * KS + s) * a.cap + b) * a.xr_pad + tp * kRowTile + (lane / 16) * 4;
                st_hand<SYNC::kStAux>(a.xpart, dst * 4,
                                      make_float4(part[0] * xs[0], part[1] * xs[1], part[2] * xs[2], part[3] * xs[3]));
            }
        }
    }
}

template <bool Q8, bool Q8XP, bool PRE, bool GRP, int QP, int T>
__global__ __launch_bounds__(kBlock) void k_mix_in(MixInArgs a) {
    const uint32_t bx = a.gmajor ? blockIdx.y : blockIdx.x, by = a.gmajor ? blockIdx.x : blockIdx.y;
    mix_in_body<Q8, Q8XP, PRE, GRP, QP, T>(a, bx, by, NoWait{});
}

// ---------------------------------------------------------------- k_scan

struct ScanArgs {
    const float* xpart;    // [nxb][cap][xr_pad]
    int nxb, xr_pad, xr;
    const float* u;        // [n][di]
    const float* z;        // [n][di]
    float* ssm;            // this layer's state, [slot][16][di] (state-major)
    const float* dt_w;     // F32 [dt_pad/4][di][4] (16-byte chunks, chunk-major) or null
    const int8_t* dt_q;    // Q8 [dt_pad/16][di][16] or null
    const float* dt_scales;  // Q8: one per row
    int dt_pad;
    const float* dt_b;
    const float* a_exp;    // [16][di]
    const float* d_vec;
    const uint32_t* slots;
    uint32_t cap, n;       // batch rows of the partials, streams
    uint32_t scap;         // state slots (the slot clamp bound)
    __bf16* glimb;         // [groups][di/32][3][64][8], or
    float* g32;            // [n][di] f32 (the wavefront-GEMV tier)
    int di, dr;
};

// scan_block (model.rs:174-190) for one (stream, channel): x_proj row sums, dt_proj row in
// the reference order, softplus(dt + b) (tensor.rs:859-861), the d16 recurrence with the
// dt-sparse skip and the hsum_ssm tree (tensor.rs:1283-1325), y * (z * sigmoid(z))
// (tensor.rs:1239-1243 on 64-channel blocks); the gated value leaves as bf16 limbs.
// Every operand is requested before the first wait.
//
// FAST takes the 16 decay factors exp(-dt * A[n]) from the hardware exp2 (v_exp_f32, on
// x * log2 e; about 1e-7 relative) instead of the reference's portable exp, which is
// about 30 VALU operations each and most of this kernel's instruction stream.  Every
// other element-wise operation keeps the reference's arithmetic.  DR and NXB fix dt_rank
// and the number of 32-channel x_proj partials at compile time (0: taken from the
// arguments, bounded by kMaxDr / kMaxNxb), which removes the guards of the unrolled loops.
// A thread runs SPT streams of one channel.
__device__ __forceinline__ float hw_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

template <bool Q8DT, bool FAST, int DR, int NXB, int SPT, class SYNC, bool FMA = false>
__device__ __forceinline__ void scan_body(const ScanArgs& a, uint32_t sy, uint32_t cbx, const SYNC& sync) {
    static_assert(DR >= 0 && DR <= kMaxDr && NXB >= 0 && NXB <= kMaxNxb && SPT >= 1 && SPT <= 2, "scan shape");
    // SPT streams per thread (streams SPT y .. SPT y + SPT - 1 of channel j): the channel's
    // operands (exp(A_log), the dt_proj row, biases, D) are loaded and decoded once for all
    // of them.  Every stream's arithmetic is the same whatever SPT is.
    constexpr int kParts = (DR && NXB) ? 3 : 1;  // threads per x_proj output (fixed shape)
    constexpr int kDr = DR ? DR : kMaxDr;
    constexpr int kNxb = NXB ? NXB : kMaxNxb;
    const int di = a.di, dr = DR ? DR : a.dr, nxb = NXB ? NXB : a.nxb;
    const int j_raw = (int)cbx * kBlock + threadIdx.x;
    const bool live = j_raw < di;
    const int j = live ? j_raw : di - 1;
    // Buffer addressing: one descriptor per array (uniform base and exact byte size), the
    // lane's 32-bit channel offset and a uniform row offset, so no load or store needs
    // per-lane 64-bit address arithmetic.
    const uint32_t ju = (uint32_t)j, diu = (uint32_t)di;
    const uint32_t j4 = ju * 4u, j16 = ju * 16u;
    const uint32_t row4 = diu * 4u;  // bytes of one [di] row
    const uint32_t bs0 = sy * SPT;  // first stream; streams past n load stream n - 1
    uint32_t bs[SPT];
#pragma unroll
    for (int s = 0; s < SPT; s++) bs[s] = min(bs0 + s, a.n - 1);
    // Requested in this order, all before the first wait: the slots, the slot-independent
    // operands, the x_proj partials, then the state once the slots are known (vector loads
    // return in order, so waiting for the slots does not wait for the rest).  Loads past a
    // short row or partial list read its last element instead of branching; those values
    // are never used.
    uint32_t slot_raw[SPT];
#pragma unroll
    for (int s = 0; s < SPT; s++) slot_raw[s] = a.slots[bs[s]];
    // State-major operands ([16][di]): for each n the wave's 64 channels are one
    // contiguous 256-byte run, so every load and store below is fully coalesced.
    float av[16];
    {
        const BufRsrc ra = buf_rsrc(a.a_exp, 16u * row4);
#pragma unroll
        for (int n = 0; n < 16; n++) av[n] = buf_ld_f32(ra, j4, (uint32_t)n * row4);
    }
    // The previous phase's outputs (u, z, the x_proj partials): requested here by a kernel
    // of its own, after the wait by a task of the persistent step kernel.
    float x[SPT], zz[SPT];
    auto load_uz = [&]() {
        const BufRsrc ru = buf_rsrc(a.u, (uint32_t)a.n * row4), rz = buf_rsrc(a.z, (uint32_t)a.n * row4);
#pragma unroll
        for (int s = 0; s < SPT; s++) {
            x[s] = buf_ld_f32<SYNC::kAux>(ru, j4, bs[s] * row4);
            zz[s] = buf_ld_f32<SYNC::kAux>(rz, j4, bs[s] * row4);
        }
    };
    if constexpr (!SYNC::kFlow) load_uz();
    const float dv = buf_ld_f32(buf_rsrc(a.d_vec, row4), j4, 0);
    const float dtb = buf_ld_f32(buf_rsrc(a.dt_b, row4), j4, 0);
    const float dts = Q8DT ? buf_ld_f32(buf_rsrc(a.dt_scales, row4), j4, 0) : 1.0f;
    constexpr int kRowVecs = Q8DT ? (kDr + 15) / 16 : (kDr + 3) / 4;  // 16-byte vectors of a dt row
    const int row_vecs = DR ? kRowVecs : (Q8DT ? a.dt_pad / 16 : a.dt_pad / 4);
    int4 wraw[kRowVecs];
    {
        const void* rp = Q8DT ? (const void*)a.dt_q : (const void*)a.dt_w;
        const BufRsrc rd = buf_rsrc(rp, (uint32_t)row_vecs * 16u * diu);
#pragma unroll
        for (int q = 0; q < kRowVecs; q++) wraw[q] = buf_ld_i4(rd, j16, (uint32_t)(DR ? q : min(q, row_vecs - 1)) * 16u * diu);
    }
    // x_proj partials of the block's streams.  With a fixed shape, kParts threads share
    // each (stream, output), item (s, part, o) summing blocks [part kPer, (part + 1) kPer)
    // in block order; the parts are then added in part order.  Otherwise item (s, o) sums
    // all blocks in order.  Thread r takes items r, r + kBlock, ...; every thread loads
    // for all of its item slots (items past the last re-read row 0, block 0), only real
    // items store: the loads stay in straight-line code.  The partial array is < 4 GiB,
    // so offsets are 32-bit.
    constexpr int kXrT = DR ? DR + 32 : kMaxXr;              // outputs per stream (bound)
    constexpr int kPer = (kNxb + kParts - 1) / kParts;
    static_assert(!(DR && NXB) || kParts * kPer == NXB, "whole parts");
    constexpr int kItems = (SPT * kParts * kXrT + kBlock - 1) / kBlock;
    // Item sums land at their item index, every slot written (unused items too) so that no
    // branch separates the partial loads from their use; with one part the sums are zp.
    __shared__ float zq[kItems * kBlock];
    __shared__ float zp_parts[kParts > 1 ? SPT * kXrT : 1];
    float* const zp = kParts > 1 ? zp_parts : zq;  // [SPT][kXrT]
    const int xr = a.xr;
    const int r = threadIdx.x;
    float pv[kItems][kPer];
    auto load_parts = [&]() {
        const uint32_t pstride = (uint32_t)a.cap * (uint32_t)a.xr_pad * 4u;
        const BufRsrc rp = buf_rsrc(a.xpart, (uint32_t)nxb * pstride);
#pragma unroll
        for (int it = 0; it < kItems; it++) {
            const int item = r + kBlock * it;
            const int o = item % kXrT, part = (item / kXrT) % kParts, s = item / (kXrT * kParts);
            const bool real = s < SPT && o < xr;
            // The lane's first block goes into the per-lane offset; block i of the part is a
            // uniform offset on top (a buffer access's scalar offset must be wave-uniform).
            const uint32_t ps = min(bs0 + (uint32_t)s, a.n - 1);  // the item's stream
            const uint32_t o0 = real ? (ps * (uint32_t)a.xr_pad + (uint32_t)o) * 4u + (uint32_t)(part * kPer) * pstride : 0u;
#pragma unroll
            for (int i = 0; i < kPer; i++)
                pv[it][i] = buf_ld_f32<SYNC::kAux>(rp, o0, (uint32_t)(NXB ? i : min(i, nxb - 1)) * pstride);
        }
    };
    if constexpr (!SYNC::kFlow) load_parts();
    float st[SPT][16];
    BufRsrc rs[SPT];
#pragma unroll
    for (int s = 0; s < SPT; s++) {
        rs[s] = buf_rsrc(a.ssm + (size_t)clamp_slot(slot_raw[s], a.scap) * 16 * diu, 16u * row4);
#pragma unroll
        for (int n = 0; n < 16; n++) st[s][n] = buf_ld_f32<kStream>(rs[s], j4, (uint32_t)n * row4);
    }
    if constexpr (SYNC::kFlow) {
        sync.wait();
        load_uz();
        load_parts();
    }
#pragma unroll
    for (int it = 0; it < kItems; it++) {
        float acc = pv[it][0];
#pragma unroll
        for (int i = 1; i < kPer; i++)
            if (NXB || i < nxb) acc += pv[it][i];
        zq[r + kBlock * it] = acc;
    }
    __syncthreads();
    if constexpr (kParts > 1) {
#pragma unroll
        for (int it = 0; it < (SPT * kXrT + kBlock - 1) / kBlock; it++) {
            const int item = r + kBlock * it;
            const int o = item % kXrT, s = item / kXrT;
            if (s < SPT && o < xr) {
                const float* q0 = zq + (size_t)s * kParts * kXrT + o;
                float zsum = q0[0];
#pragma unroll
                for (int q = 1; q < kParts; q++) zsum = zsum + q0[q * kXrT];
                zp[s * kXrT + o] = zsum;
            }
        }
        __syncthreads();
    }
    if (!live) return;
    float wdt[kRowVecs * (Q8DT ? 16 : 4)];
#pragma unroll
    for (int q = 0; q < kRowVecs; q++) {
        const int wv[4] = {wraw[q].x, wraw[q].y, wraw[q].z, wraw[q].w};
        if (Q8DT) {
#pragma unroll
            for (int e = 0; e < 16; e++) wdt[16 * q + e] = (float)(int8_t)(wv[e / 4] >> (8 * (e % 4)));
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) wdt[4 * q + e] = bits_to_f((uint32_t)wv[e]);
        }
    }
    // Gate: the 8-aligned body of each 64-channel block takes the lane form
    // 1 / (1 + lane_exp(0 - z)), the tail 1 / (1 + exp(-z)); one exp_f serves both.
    const int blk0 = j / 64 * 64;
    const int len = min(64, di - blk0);
    const bool gate_body = (j - blk0) < len / 8 * 8;
#pragma unroll
    for (int s = 0; s < SPT; s++) {
        const uint32_t b = bs0 + s;
        if (b >= a.n) break;
        const float* zps = zp + s * kXrT;
        // dot_avx2_order (tensor.rs:1680-1693): eight lanes by column residue, fixed tree,
        // tail.  dt_rank <= 64 means a quantized dt_proj has one scale per row (a 64-column
        // group spans the whole row or the group rule falls back to per-row), so the Q8
        // row is 0 + dot * scale (gemv.rs:490-502).  FMA: numeric contract 2, the same
        // order with every acc + w * x and 0 + dot * scale one fused multiply-add
        // (gemv_fma.rs:98-134).
        float dt;
        {
            const int body = dr / 8 * 8;
            float l[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c + 8 <= kDr; c += 8) {
                if (DR || c < body) {
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        l[i] = FMA ? __builtin_fmaf(wdt[c + i], zps[c + i], l[i]) : l[i] + wdt[c + i] * zps[c + i];
                }
            }
            float sdot = ((l[0] + l[4]) + (l[2] + l[6])) + ((l[1] + l[5]) + (l[3] + l[7]));
#pragma unroll
            for (int c = DR / 8 * 8; c < kDr; c++)
                if (c >= body && c < dr) sdot = FMA ? __builtin_fmaf(wdt[c], zps[c], sdot) : sdot + wdt[c] * zps[c];
            dt = Q8DT ? (FMA ? __builtin_fmaf(sdot, dts, 0.0f) : 0.0f + sdot * dts) : sdot;
        }
        dt = softplus_f(dt + dtb);
        const float* B = zps + dr;
        const float* C = zps + dr + 16;
        if (!(fabsf(dt) < 1e-6f)) {
            const float dtx = dt * x[s];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float e = 0.0f - dt * av[k];
                const float da = FAST ? hw_exp(e) : lane_exp_f(e);
                st[s][k] = da * st[s][k] + dtx * B[k];
            }
#pragma unroll
            for (int n = 0; n < 16; n++) buf_st_f32<kStream>(st[s][n], rs[s], j4, (uint32_t)n * row4);
        }
        float l[8];
#pragma unroll
        for (int i = 0; i < 8; i++) l[i] = st[s][i] * C[i] + st[s][i + 8] * C[i + 8];
        const float y = ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7])) + dv * x[s];
        const float sg = 1.0f / (1.0f + exp_f(gate_body ? lane_exp_arg(0.0f - zz[s]) : -zz[s]));
        const float gv = y * (zz[s] * sg);
        if (a.g32 != nullptr) {
            a.g32[(size_t)b * di + j] = gv;
            continue;
        }
        const Limb3 t3 = split3(gv);
        const int g = b / kRowTile, sk = j / kKStep;
        const int ln = (b % kRowTile) + kRowTile * ((j % kKStep) / 8);
        const size_t dst = ((((size_t)g * (di / kKStep) + sk) * 3) * 64 + ln) * 8 + (j % 8);
        st_hand<SYNC::kStAux>(a.glimb, dst * 2, t3.h);
        st_hand<SYNC::kStAux>(a.glimb, (dst + 512) * 2, t3.m);
        st_hand<SYNC::kStAux>(a.glimb, (dst + 1024) * 2, t3.l);
    }
}

// The channel blocks of a stream group (SPT streams) run on one XCD, so the group's x_proj
// partials are fetched into one L2 and shared by its channel blocks.
template <bool Q8DT, bool FAST, int DR, int NXB, int SPT, bool FMA = false>
__global__ __launch_bounds__(kBlock) void k_scan(ScanArgs a) {
    const XcdTile xt = xcd_tile(blockIdx.x, ((uint32_t)a.di + kBlock - 1) / kBlock, (a.n + SPT - 1) / SPT);
    if (!xt.live) return;
    scan_body<Q8DT, FAST, DR, NXB, SPT, NoWait, FMA>(a, xt.unit, xt.part, NoWait{});
}

// Streams per scan thread by batch size: sharing a channel's operands pays once a launch
// has several times more workgroups than the chip holds at once (measured on Mamba-130M:
// 1-2 % from 256 streams, a loss below; four streams per thread lose everywhere, from the
// halved occupancy).
constexpr uint32_t kScanSpt2From = 256;

uint32_t scan_spt(uint32_t n) { return n >= kScanSpt2From ? 2 : 1; }

template <bool Q8DT, bool FAST, int DR, int NXB>
const void* scan_fn_spt(uint32_t spt) {
    if (spt == 2) return (const void*)k_scan<Q8DT, FAST, DR, NXB, 2>;
    return (const void*)k_scan<Q8DT, FAST, DR, NXB, 1>;
}

// The scan instance for a layer shape: Mamba-130M's (dt_rank 48, 48 x_proj blocks of 32
// channels) is specialised, every other shape takes the generic kernel.
const void* scan_fn(bool q8dt, bool fast, int dr, int nxb, uint32_t spt) {
    const bool m130 = dr == 48 && nxb == 48;
    if (q8dt) {
        if (m130) return fast ? scan_fn_spt<true, true, 48, 48>(spt) : scan_fn_spt<true, false, 48, 48>(spt);
        return fast ? scan_fn_spt<true, true, 0, 0>(spt) : scan_fn_spt<true, false, 0, 0>(spt);
    }
    if (m130) return fast ? scan_fn_spt<false, true, 48, 48>(spt) : scan_fn_spt<false, false, 48, 48>(spt);
    return fast ? scan_fn_spt<false, true, 0, 0>(spt) : scan_fn_spt<false, false, 0, 0>(spt);
}

// ---------------------------------------------------------------- k_mix_out

struct MixOutArgs {
    TMat w;                  // out_proj [d][di]
    const __bf16* glimb;     // gated limbs, B fragments
    float* x;                // [n][d] residual, updated in place (or written to x_out)
    uint32_t n;
    int d;
    const float* nw_next;    // next norm weight (next layer's, or the final norm's); with
    __bf16* xw;              // xw != null the next consumer's pre-staged activations are
    float* ssp;              // produced here
    int ks_x, tiles;
    uint32_t gmajor = 0;     // grid (chunks, row tiles) instead of (row tiles, chunks)
    float* x_out = nullptr;  // the updated residual's rows, when not x itself
};

// out_proj + residual.  Eight waves share one 16-row tile, each summing an eighth of the
// k-pairs (limb orders in separate accumulators, as in tiles_gemm) with kOutPairs pairs of
// weight and activation fragments requested at once; the eighths are added in wave order,
// then the per-row scale, then the residual: x += (((q0 + q1) + q2) + ... + q7).  The new
// residual rows then leave as the next projection's pre-staged activations.
// FIXED: every wave takes exactly kOutPairs k-pairs (w.ks = 2 kOutWaves kOutPairs, checked
// on the host), one pass whose loads are all issued unconditionally (clamped group and
// row indices), the epilogue operands after them, before the first wait.
// WAVES < kOutWaves (a task of the persistent step kernel, 4 waves): each wave runs the
// k-ranges of kOutWaves / WAVES of the kernel's waves (virtual waves w, w + WAVES, ...),
// each in accumulators of its own, and the cross-wave sum takes them in the kernel's
// order, so a task's arithmetic is the kernel's.  As a task the weights and scales are
// requested first, the gated tiles and the residual rows after the wait.
template <bool Q8, int G, bool FIXED, int WAVES, class SYNC>
__device__ __forceinline__ void mix_out_body(const MixOutArgs& a, uint32_t t_blk, uint32_t by, const SYNC& sync) {
    constexpr int VW = kOutWaves / WAVES;
    static_assert(VW * WAVES == kOutWaves && (VW == 1 || FIXED), "virtual waves need the fixed shape");
    static_assert(!SYNC::kFlow || FIXED, "persistent tasks take the fixed shape");
    __shared__ f32x4 part[kOutWaves - 1][G][kWave];
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const int t = (int)t_blk;
    const uint32_t b0 = by * G * kRowTile;
    const int ng = (int)min((uint32_t)G, (a.n - b0 + kRowTile - 1) / kRowTile);
    const TMat& w = a.w;
    const int np = w.ks / 2;
    const int p_lo = wave * np / kOutWaves, p_hi = (wave + 1) * np / kOutWaves;
    const bool grp = Q8 && w.group != w.cols;
    const int gpr = w.ks / 2;
    const uint32_t g0 = b0 / kRowTile;
    const int r0 = t * kRowTile + (lane / 16) * 4;
    float4 xv[G];
    float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    float4 w4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    f32x4 acc3v[VW][G][3];
#pragma unroll
    for (int v = 0; v < VW; v++)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int o = 0; o < 3; o++) acc3v[v][g][o] = f32x4{0, 0, 0, 0};
    if constexpr (FIXED) {
        RawPair raw[VW][kOutPairs];
        bf16x8 bfr[VW][kOutPairs][G][2][3];
        float sc[VW][kOutPairs][4];
        const BufRsrc rg = buf_rsrc_any(a.glimb);
        auto load_acts = [&](int v, int q) {
            const int p = (wave + WAVES * v) * kOutPairs + q;
#pragma unroll
            for (int g = 0; g < G; g++) {
                const uint32_t gg = g0 + (G > 1 ? (uint32_t)min(g, ng - 1) : 0u);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const size_t off = (((size_t)gg * w.ks + 2 * p + h) * 3) * 512 + lane * 8;
#pragma unroll
                    for (int m = 0; m < 3; m++) {
                        if constexpr (SYNC::kAux == kCached)
                            bfr[v][q][g][h][m] = lds_frag(a.glimb + off + m * 512);
                        else
                            bfr[v][q][g][h][m] = as_frag(buf_ld_i4p<SYNC::kAux>(rg, (uint32_t)(off + m * 512) * 2u, 0));
                    }
                }
            }
        };
        auto load_x = [&]() {
            const BufRsrc rx = buf_rsrc_any(a.x);
#pragma unroll
            for (int g = 0; g < G; g++) {
                const uint32_t b = min(b0 + g * kRowTile + lane % 16, a.n - 1);
                if constexpr (SYNC::kAux == kCached) {
                    xv[g] = *(const float4*)(a.x + (size_t)b * a.d + r0);
                } else {
                    const int4 v = buf_ld_i4p<SYNC::kAux>(rx, (b * (uint32_t)a.d + (uint32_t)r0) * 4u, 0);
                    xv[g] = make_float4(bits_to_f((uint32_t)v.x), bits_to_f((uint32_t)v.y), bits_to_f((uint32_t)v.z),
                                        bits_to_f((uint32_t)v.w));
                }
            }
        };
#pragma unroll
        for (int v = 0; v < VW; v++)
#pragma unroll
            for (int q = 0; q < kOutPairs; q++) {
                const int p = (wave + WAVES * v) * kOutPairs + q;
                raw[v][q] = load_pair<Q8>(w, t, p, lane);
                if constexpr (!SYNC::kFlow) load_acts(v, q);
                if (grp) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        sc[v][q][i] = w.scales[(size_t)(t * kRowTile + (lane / 16) * 4 + i) * gpr + p];
                }
            }
        // Epilogue operands (used by wave 0), loaded by every wave from clamped rows.
        if constexpr (!SYNC::kFlow) load_x();
        if (Q8 && !grp) {
            const float4 r4 = *(const float4*)(w.scales + t * kRowTile + (lane / 16) * 4);
            rs[0] = r4.x; rs[1] = r4.y; rs[2] = r4.z; rs[3] = r4.w;
        }
        if (a.xw != nullptr) w4 = *(const float4*)(a.nw_next + r0);
        if constexpr (SYNC::kFlow) {
            sync.wait();
#pragma unroll
            for (int v = 0; v < VW; v++)
#pragma unroll
                for (int q = 0; q < kOutPairs; q++) load_acts(v, q);
            load_x();
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int v = 0; v < VW; v++) {
            f32x4 (&acc3)[G][3] = acc3v[v];
#pragma unroll
            for (int q = 0; q < kOutPairs; q++) {
                AFrag a0, a1;
                decode_pair<Q8>(raw[v][q], a0, a1);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    if (g >= ng) continue;
                    if (grp) {
                        f32x4 pp{0, 0, 0, 0};
                        pp = mma_step<Q8>(a0, bfr[v][q][g][0][0], bfr[v][q][g][0][1], bfr[v][q][g][0][2], pp);
                        pp = mma_step<Q8>(a1, bfr[v][q][g][1][0], bfr[v][q][g][1][1], bfr[v][q][g][1][2], pp);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc3[g][0][i] = __builtin_fmaf(pp[i], sc[v][q][i], acc3[g][0][i]);
                    } else {
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const AFrag& af = h ? a1 : a0;
                            const bf16x8* bb = bfr[v][q][g][h];
                            if (Q8) {
                                acc3[g][0] = mma(af.h, bb[0], acc3[g][0]);
                                acc3[g][1] = mma(af.h, bb[1], acc3[g][1]);
                                acc3[g][2] = mma(af.h, bb[2], acc3[g][2]);
                            } else {
                                acc3[g][0] = mma(af.h, bb[0], acc3[g][0]);
                                acc3[g][1] = mma(af.h, bb[1], acc3[g][1]);
                                acc3[g][1] = mma(af.m, bb[0], acc3[g][1]);
                                acc3[g][2] = mma(af.h, bb[2], acc3[g][2]);
                                acc3[g][2] = mma(af.m, bb[1], acc3[g][2]);
                                acc3[g][2] = mma(af.l, bb[0], acc3[g][2]);
                            }
                        }
                    }
                }
            }
        }
    } else {
    f32x4 (&acc3)[G][3] = acc3v[0];
    // Epilogue operands of wave 0, requested with the rest.
    if (wave == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const uint32_t b = b0 + g * kRowTile + lane % 16;
            xv[g] = g < ng && b < a.n && r0 < a.d ? *(const float4*)(a.x + (size_t)b * a.d + r0)
                                                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        if (Q8 && !grp) {
#pragma unroll
            for (int i = 0; i < 4; i++) rs[i] = w.scales[t * kRowTile + (lane / 16) * 4 + i];
        }
        if (a.xw != nullptr && r0 < a.d) w4 = *(const float4*)(a.nw_next + r0);
    }
#pragma unroll 1
    for (int pb = p_lo; pb < p_hi; pb += kOutPairs) {
        RawPair raw[kOutPairs];
        bf16x8 bfr[kOutPairs][G][2][3];
        float sc[kOutPairs][4];
#pragma unroll
        for (int q = 0; q < kOutPairs; q++) {
            const int p = pb + q;
            if (p >= p_hi) break;
            raw[q] = load_pair<Q8>(w, t, p, lane);
#pragma unroll
            for (int g = 0; g < G; g++) {
                if (g >= ng) continue;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const __bf16* f = a.glimb + (((size_t)(g0 + g) * w.ks + 2 * p + h) * 3) * 512 + lane * 8;
                    bfr[q][g][h][0] = lds_frag(f);
                    bfr[q][g][h][1] = lds_frag(f + 512);
                    bfr[q][g][h][2] = lds_frag(f + 1024);
                }
            }
            if (grp) {
#pragma unroll
                for (int i = 0; i < 4; i++) sc[q][i] = w.scales[(size_t)(t * kRowTile + (lane / 16) * 4 + i) * gpr + p];
            }
        }
#pragma unroll
        for (int q = 0; q < kOutPairs; q++) {
            const int p = pb + q;
            if (p >= p_hi) break;
            AFrag a0, a1;
            decode_pair<Q8>(raw[q], a0, a1);
#pragma unroll
            for (int g = 0; g < G; g++) {
                if (g >= ng) continue;
                if (grp) {
                    f32x4 pp{0, 0, 0, 0};
                    pp = mma_step<Q8>(a0, bfr[q][g][0][0], bfr[q][g][0][1], bfr[q][g][0][2], pp);
                    pp = mma_step<Q8>(a1, bfr[q][g][1][0], bfr[q][g][1][1], bfr[q][g][1][2], pp);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc3[g][0][i] = __builtin_fmaf(pp[i], sc[q][i], acc3[g][0][i]);
                } else {
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const AFrag& af = h ? a1 : a0;
                        const bf16x8* bb = bfr[q][g][h];
                        if (Q8) {
                            acc3[g][0] = mma(af.h, bb[0], acc3[g][0]);
                            acc3[g][1] = mma(af.h, bb[1], acc3[g][1]);
                            acc3[g][2] = mma(af.h, bb[2], acc3[g][2]);
                        } else {
                            acc3[g][0] = mma(af.h, bb[0], acc3[g][0]);
                            acc3[g][1] = mma(af.h, bb[1], acc3[g][1]);
                            acc3[g][1] = mma(af.m, bb[0], acc3[g][1]);
                            acc3[g][2] = mma(af.h, bb[2], acc3[g][2]);
                            acc3[g][2] = mma(af.m, bb[1], acc3[g][2]);
                            acc3[g][2] = mma(af.l, bb[0], acc3[g][2]);
                        }
                    }
                }
            }
        }
    }
    }
    f32x4 acc[VW][G];
#pragma unroll
    for (int v = 0; v < VW; v++)
#pragma unroll
        for (int g = 0; g < G; g++) acc[v][g] = (acc3v[v][g][0] + acc3v[v][g][1]) + acc3v[v][g][2];
#pragma unroll
    for (int v = 0; v < VW; v++) {
        const int vw = wave + WAVES * v;
        if (vw > 0) {
#pragma unroll
            for (int g = 0; g < G; g++) part[vw - 1][g][lane] = acc[v][g];
        }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int g = 0; g < G; g++) {
        if (g >= ng) continue;
        f32x4 s = acc[0][g];
        for (int q = 0; q < kOutWaves - 1; q++) s = s + part[q][g][lane];
        const uint32_t b = b0 + g * kRowTile + lane % 16;
        const bool ok = b < a.n && r0 < a.d;
        const float nx[4] = {xv[g].x + s[0] * rs[0], xv[g].y + s[1] * rs[1], xv[g].z + s[2] * rs[2],
                             xv[g].w + s[3] * rs[3]};
        if (ok) st_hand<SYNC::kStAux>(a.x_out ? a.x_out : a.x, ((size_t)b * a.d + r0) * 4,
                                      make_float4(nx[0], nx[1], nx[2], nx[3]));
        if (a.xw != nullptr) produce_tile<SYNC::kStAux>(a.xw, a.ssp, a.ks_x, a.tiles, t, b, ok, nx, w4);
    }
}

template <bool Q8, int G, bool FIXED>
__global__ __launch_bounds__(kOutWaves * kWave) void k_mix_out(MixOutArgs a) {
    const uint32_t t_blk = a.gmajor ? blockIdx.y : blockIdx.x, by = a.gmajor ? blockIdx.x : blockIdx.y;
    mix_out_body<Q8, G, FIXED, kOutWaves>(a, t_blk, by, NoWait{});
}

// out_proj + residual for TT row tiles of one stream group (the fixed shape: kOutPairs
// k-pairs per wave).  Each wave multiplies all TT tiles over its k-pairs against the same
// gated fragments, so a workgroup reads its group's gated tiles once for TT tiles instead
// of once per tile.  Per tile the arithmetic is mix_out_body's: the same k-split over the
// eight waves, the same products into the same accumulators, the eighths added in wave
// order, then the row scale and the residual; so a stream's bits do not depend on TT.
// Wave i < TT finishes tile TT t_blk + i.
template <bool Q8, int TT>
__device__ __forceinline__ void mix_out_tiles(const MixOutArgs& a, uint32_t t_blk, uint32_t by) {
    __shared__ f32x4 part[kOutWaves][TT][kWave];
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const TMat& w = a.w;
    const int t0 = (int)t_blk * TT;
    const uint32_t b0 = by * kRowTile;
    const bool grp = Q8 && w.group != w.cols;
    const int gpr = w.ks / 2;
    RawPair raw[kOutPairs][TT];
    bf16x8 bfr[kOutPairs][2][3];
    float sc[kOutPairs][TT][4];
#pragma unroll
    for (int q = 0; q < kOutPairs; q++) {
        const int p = wave * kOutPairs + q;
#pragma unroll
        for (int i = 0; i < TT; i++) raw[q][i] = load_pair<Q8>(w, min(t0 + i, w.rt - 1), p, lane);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const __bf16* f = a.glimb + (((size_t)by * w.ks + 2 * p + h) * 3) * 512 + lane * 8;
#pragma unroll
            for (int m = 0; m < 3; m++) bfr[q][h][m] = lds_frag(f + m * 512);
        }
        if (grp) {
#pragma unroll
            for (int i = 0; i < TT; i++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    sc[q][i][e] = w.scales[(size_t)(min(t0 + i, w.rt - 1) * kRowTile + (lane / 16) * 4 + e) * gpr + p];
        }
    }
    // Epilogue operands of the tile this wave finishes (waves past TT load tile TT - 1's).
    const int tf = min(t0 + min(wave, TT - 1), w.rt - 1);
    const int r0 = tf * kRowTile + (lane / 16) * 4;
    const uint32_t b = b0 + lane % 16;
    const float4 xv = *(const float4*)(a.x + (size_t)min(b, a.n - 1) * a.d + r0);
    float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    if (Q8 && !grp) {
        const float4 r4 = *(const float4*)(w.scales + r0);
        rs[0] = r4.x; rs[1] = r4.y; rs[2] = r4.z; rs[3] = r4.w;
    }
    const float4 w4 = a.xw != nullptr ? *(const float4*)(a.nw_next + r0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc3[TT][3];
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
        for (int o = 0; o < 3; o++) acc3[i][o] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < kOutPairs; q++) {
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
#pragma unroll
    for (int i = 0; i < TT; i++) part[wave][i][lane] = (acc3[i][0] + acc3[i][1]) + acc3[i][2];
    __syncthreads();
    if (wave >= TT || t0 + wave >= w.rt) return;
    f32x4 s = part[0][wave][lane];
#pragma unroll
    for (int q = 1; q < kOutWaves; q++) s = s + part[q][wave][lane];
    const bool ok = b < a.n && r0 < a.d;
    const float nx[4] = {xv.x + s[0] * rs[0], xv.y + s[1] * rs[1], xv.z + s[2] * rs[2], xv.w + s[3] * rs[3]};
    if (ok) *(float4*)((a.x_out ? a.x_out : a.x) + (size_t)b * a.d + r0) = make_float4(nx[0], nx[1], nx[2], nx[3]);
    if (a.xw != nullptr) produce_tile(a.xw, a.ssp, a.ks_x, a.tiles, tf, b, ok, nx, w4);
}

template <bool Q8, int TT>
__global__ __launch_bounds__(kOutWaves * kWave) void k_mix_out_t(MixOutArgs a) {
    const uint32_t t_blk = a.gmajor ? blockIdx.y : blockIdx.x, by = a.gmajor ? blockIdx.x : blockIdx.y;
    mix_out_tiles<Q8, TT>(a, t_blk, by);
}

// ---------------------------------------------------------------- persistent step kernel

// All layers of a step in one cooperative launch (int8 per-row weights, the Mamba-130M
// shape).  Every phase of every stream group is spread over all XCDs: task t of a
// (layer, phase, group) runs on XCD t % nx (the XCD a workgroup runs on is read from the
// hardware), so tile t of in_proj or out_proj reads its weights into one XCD's L2 for
// all groups, and the groups' phases overlap on every XCD (one group's scan runs while
// the next group's in_proj still does).  XCD x's list holds its tasks ordered by layer,
// then phase (in_proj, scan, out_proj), then group, then tile; its workgroups take them
// in list order from a ticket counter.  Every task depends only on tasks earlier in that
// global order (the previous phase of its group), and every workgroup is resident
// (cooperative launch), so the globally earliest unfinished task always has its inputs
// and its ticket's holder reaches it: the step advances.  A task's body requests its
// weights, scales and recurrent state, waits until the counter of the phase it reads
// reaches that phase's task count, then reads those outputs (each layer hands over
// through buffers of its own, written through to the coherence point); after its stores
// are complete it adds one to its own phase's counter.  The bodies are the stand-alone
// kernels' (same tiles, k-splits and orders), so a stream's bits do not depend on which
// path ran it.
constexpr uint32_t kFlowMaxStreams = 1024;    // largest step the kernel serves (bounds every wait and its buffers)
constexpr uint32_t kFlowScanSpt = 2;          // streams per scan task thread

struct FlowLayer {
    MixInArgs mi;
    ScanArgs sc;
    MixOutArgs mo;
};

struct FlowArgs {
    const FlowLayer* layers;  // [nl], device memory, read through the scalar unit
    uint32_t nl, groups;
    uint32_t* cnt;            // [nl][3][groups][kFlowSlices] phase counters, then [nx] task tickets, kFlowCounterStride words apart
    uint32_t* err;
    uint32_t mi_tasks, cb, mo_tasks;  // in_proj row blocks, scan channel blocks, out_proj row tiles (per group)
    uint32_t nx;              // XCDs of the device (divides each phase's tasks per group)
    uint32_t fixed;           // 1: static assignment (every phase has the same tasks per group and XCD)
    uint8_t xmap[16];         // XCC_ID -> XCD index 0 .. nx - 1 (0xff: not seen when the grid was planned)
};

// The XCD this wave runs on (hardware register XCC_ID, bits 3:0).
__device__ __forceinline__ uint32_t xcc_id() { return __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 0xfu; }

// Workgroup w writes its XCC_ID to map[w]: the host learns the device's XCDs from one
// launch of the persistent kernel's grid.
__global__ __launch_bounds__(kBlock) void k_xcc_map(uint32_t* map) {
    if (threadIdx.x == 0) map[blockIdx.x] = xcc_id();
}

// Phase ph of layer l for group g: kFlowSlices counters, one per XCD.
__device__ __forceinline__ uint32_t* flow_counter(const FlowArgs& f, uint32_t l, uint32_t ph, uint32_t g) {
    return f.cnt + ((size_t)(l * 3 + ph) * f.groups + g) * kFlowSlices * kFlowCounterStride;
}

// Task `task` of phase `phase` of layer l for stream group g: its wait and its body.
template <bool Q8S, bool FAST>
__device__ __forceinline__ void flow_task(const FlowArgs& f, const FlowLayer& L, uint32_t l, uint32_t phase, uint32_t g,
                                          uint32_t task) {
    constexpr uint32_t kSpt = kFlowScanSpt;
    if (phase == 0) {
        const FlowWait w{l > 0 ? flow_counter(f, l - 1, 2, g) : nullptr, f.mo_tasks, f.err};
        mix_in_body<true, Q8S, true, false, kInFixedPairs, 4>(L.mi, task, g, w);
    } else if (phase == 1) {
        // kSpt streams per task: the tasks of streams past n (a last, partial group) only count
        const uint32_t sy = g * (kRowTile / kSpt) + task / f.cb;
        const FlowWait w{flow_counter(f, l, 0, g), f.mi_tasks, f.err};
        if (sy * kSpt < L.sc.n) scan_body<Q8S, FAST, 48, 48, kSpt>(L.sc, sy, task % f.cb, w);
    } else {
        const FlowWait w{flow_counter(f, l, 1, g), kRowTile / kSpt * f.cb, f.err};
        mix_out_body<true, 1, true, kWaves>(L.mo, task, g, w);
    }
}

// Which workgroup runs a task is decided at run time: the workgroups of XCD x take the
// tasks of x's list in order from x's ticket counter (one device-scope atomic per task,
// requested when the previous task's body is done), or, with f.fixed, one ticket each that
// names a group and a task index for the whole step.  The hardware deals workgroups to
// XCDs round-robin from where the previous dispatch stopped, so the block index does not
// name the XCD; the ticket order keeps every dependency on an earlier ticket, taken by a
// resident workgroup.
template <bool Q8S, bool FAST>
__global__ __launch_bounds__(kBlock, 2) void k_flow(FlowArgs f) {
    __shared__ uint32_t s_next;
    const uint32_t x = f.xmap[xcc_id()];
    if (x >= f.nx) {
        if (threadIdx.x == 0) atomicOr(f.err, 8u);
        return;
    }
    constexpr uint32_t kSpt = kFlowScanSpt;
    const uint32_t G = f.groups, nx = f.nx;
    // Tasks of one (layer, phase, group) on this XCD: tiles x, x + nx, ...
    const uint32_t mi = f.mi_tasks / nx, sc = kRowTile / kSpt * f.cb / nx, mo = f.mo_tasks / nx;
    const uint32_t per_layer = G * (mi + sc + mo);
    const uint32_t total = per_layer * f.nl;
    uint32_t* const ticket = f.cnt + ((size_t)f.nl * 3 * G * kFlowSlices + x) * kFlowCounterStride;
    typedef const __attribute__((address_space(4))) FlowLayer* FlowLayerK;
    const FlowLayerK layers = (FlowLayerK)f.layers;
    if (threadIdx.x == 0) s_next = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (f.fixed) {
        // Static assignment (mi == sc == mo): the workgroup's ticket s names its group,
        // s / mi, and its task, x + nx (s % mi), in every phase of every layer; it runs them
        // layer by layer, waiting only for its own group's counters, so each phase of a group
        // runs all its tasks at once.  Tickets past the groups' tasks exit.  Every group's
        // tasks are held by resident workgroups (the grid is the device's full occupancy and
        // the host planned G mi <= grid / nx).
        const uint32_t slot = __builtin_amdgcn_readfirstlane(s_next);
        if (slot >= G * mi) return;
        const uint32_t g = slot / mi, task = x + nx * (slot % mi);
        for (uint32_t l = 0; l < f.nl; l++)
            for (uint32_t phase = 0; phase < 3; phase++) {
                flow_task<Q8S, FAST>(f, *(const FlowLayer*)(layers + l), l, phase, g, task);
                // every store of the task is complete at the coherence point before the counter says so
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                if (threadIdx.x == 0)
                    __hip_atomic_fetch_add(flow_counter(f, l, phase, g) + (x % kFlowSlices) * kFlowCounterStride, 1u,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        return;
    }
    for (uint32_t i = s_next; i < total;) {
        const uint32_t l = i / per_layer;
        uint32_t r = i % per_layer;
        uint32_t phase, g, k;
        if (r < G * mi) {
            phase = 0, g = r / mi, k = r % mi;
        } else if ((r -= G * mi) < G * sc) {
            phase = 1, g = r / sc, k = r % sc;
        } else {
            r -= G * sc;
            phase = 2, g = r / mo, k = r % mo;
        }
        const uint32_t task = x + nx * k;
        flow_task<Q8S, FAST>(f, *(const FlowLayer*)(layers + l), l, phase, g, task);
        // The next ticket is taken only once this task's body is done, so a workgroup never
        // holds two tasks at once (two of one phase would run one after the other); its
        // round trip overlaps the drain of the task's stores.
        uint32_t ahead = 0;
        if (threadIdx.x == 0) ahead = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // every store of the task is complete at the coherence point before the counter says so
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            __hip_atomic_fetch_add(flow_counter(f, l, phase, g) + (x % kFlowSlices) * kFlowCounterStride, 1u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_next = ahead;
        }
        __syncthreads();
        i = s_next;
    }
}

// ---------------------------------------------------------------- k_head

struct HeadArgs {
    const float* x;
    const float* norm_w;
    const float* norm_b;
    TMat w;                  // head [vocab][d]
    float* out;              // [n][vocab]
    uint32_t n;
    int d;
    const __bf16* xw;        // pre-staged activations (RMSNorm path)
    const float* ssp;
    int tiles;
};

// Final norm (model.rs:745-752) and the LM head (model.rs:921-927, tied to the
// embedding unless the file carries lm_head).  Each wave multiplies kHeadTiles row tiles
// together, so every activation fragment read from LDS serves all of them; kHeadWaves
// waves share one staged chunk, two per SIMD (the chunk's LDS allows one workgroup per
// CU).  The stream chunks of a row block run on one XCD (xcd_tile), which fetches the
// block's weights into its L2 once for all of them.
template <bool Q8, bool PRE>
__global__ __launch_bounds__(kHeadWaves * kWave) void k_head(HeadArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float invs[kChunk];
    __bf16* lds = (__bf16*)smem;
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const XcdTile xt = xcd_tile(blockIdx.x, (a.n + kChunk - 1) / kChunk,
                                ((uint32_t)a.w.rt + kHeadWaves * kHeadTiles - 1) / (kHeadWaves * kHeadTiles));
    if (!xt.live) return;
    const uint32_t b0 = xt.part * kChunk;
    const int ng = (int)min((uint32_t)kGroups, (a.n - b0 + kRowTile - 1) / kRowTile);
    const int V = a.w.rows;
    const int t_first = ((int)xt.unit * kHeadWaves + wave) * kHeadTiles;
    SspLoad sl;
    if constexpr (PRE) sl = ssp_load(a.ssp, a.tiles, b0, a.n, kChunk);
    constexpr int R = Q8 ? kHeadRingQ8 : kHeadRingF32;
    Tiles<Q8, kHeadTiles, R> tl;
#pragma unroll
    for (int i = 0; i < kHeadTiles; i++) {
        tl.t[i] = t_first + i;
        tl.ok[i] = t_first + i < a.w.rt;
    }
    const int np = a.w.ks / 2;
    tiles_prefetch<Q8, kHeadTiles, R>(a.w, tl, 0, np);
    if constexpr (PRE) {
        stage_copy(smem, a.xw, b0 / kRowTile, ng, a.w.ks, kHeadWaves);
        ssp_reduce(sl, invs, a.tiles, a.d, kChunk);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    } else {
        stage_normed(lds, a.x, a.norm_w, a.norm_b, a.d, a.w.ks, b0, a.n, kChunk);
    }
    f32x4 res[kHeadTiles][kGroups];
    tiles_gemm<Q8, kHeadTiles, R>(a.w, tl, lds, ng, 0, np, res);
#pragma unroll
    for (int tt = 0; tt < kHeadTiles; tt++) {
        const int t = t_first + tt;
        if (t >= a.w.rt) continue;
        f32x4 acc[kGroups];
#pragma unroll
        for (int g = 0; g < kGroups; g++) acc[g] = res[tt][g];
        apply_row_scales(a.w, t, acc, ng);
        if constexpr (PRE) {
#pragma unroll
            for (int g = 0; g < kGroups; g++) acc[g] = acc[g] * invs[g * kRowTile + lane % 16];
        }
        const int r0 = t * kRowTile + (lane / 16) * 4;
#pragma unroll
        for (int g = 0; g < kGroups; g++) {
            const uint32_t b = b0 + g * kRowTile + lane % 16;
            if (g >= ng || b >= a.n) continue;
            float* o = a.out + (size_t)b * V + r0;
            // Logits are written once and read later (host copy, softmax): streamed.
            if (r0 + 3 < V && (V & 3) == 0) {
                __builtin_nontemporal_store(f32x4{acc[g][0], acc[g][1], acc[g][2], acc[g][3]}, (f32x4*)o);
            } else {
                for (int i = 0; i < 4; i++)
                    if (r0 + i < V) __builtin_nontemporal_store(acc[g][i], o + i);
            }
        }
    }
}

// Weights-stationary LM head for Q8 per-row weights and pre-staged activations.  Each of
// the kHwWaves waves decodes its kHwTiles row tiles (all NP k-pairs) into bf16 registers
// once and keeps them for the whole kernel, walking the workgroup's column groups: group
// g's activation tiles are copied into one LDS buffer while group g - 1 is multiplied
// from the other.  Per tile and group: one accumulator over k-steps in order, limbs hi,
// mid, lo per k-step; then the row scale and the stream's RMS scale.  Above 128 streams
// the chunks of a row block run on one XCD (xcd_tile) and share its L2.
constexpr int kHwWaves = 8;    // waves per workgroup
constexpr int kHwTiles = 2;    // row tiles per wave
constexpr int kHwGroups = 8;   // column groups (16 streams) per workgroup

__device__ __forceinline__ void copy_group(unsigned char* buf, const __bf16* __restrict__ xw, uint32_t g, int ks) {
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const int blocks = ks * 3;
    const __bf16* src = xw + (size_t)g * blocks * 512 + lane * 8;
    lds_u8* dst = (lds_u8*)buf;
#pragma unroll 2
    for (int q = wave; q < blocks; q += kHwWaves)
        __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)q * 512),
                                         (void __attribute__((address_space(3)))*)(dst + q * kLimbBytes), 16, 0, 0);
}

template <int NP>
__global__ __launch_bounds__(kHwWaves * kWave) void k_head_ws(HeadArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float invs[kHwGroups * kRowTile];
    const int lane = threadIdx.x % kWave, wave = wave_index();
    const TMat& w = a.w;
    const int np = w.ks / 2, ks = w.ks;
    const int V = w.rows;
    const uint32_t n_groups = (a.n + kRowTile - 1) / kRowTile;
    const XcdTile xt = xcd_tile(blockIdx.x, (n_groups + kHwGroups - 1) / kHwGroups,
                                ((uint32_t)w.rt + kHwWaves * kHwTiles - 1) / (kHwWaves * kHwTiles));
    if (!xt.live) return;
    const uint32_t gb = xt.part * kHwGroups;
    const int ngr = (int)min((uint32_t)kHwGroups, n_groups - gb);
    const int t0 = ((int)xt.unit * kHwWaves + wave) * kHwTiles;
    const size_t buf_bytes = (size_t)ks * 3 * kLimbBytes;
    // Requested first: the RMS partials of every stream of the workgroup, the weights and
    // row scales, the first group's activations.
    float ssv[kSspPerThread];
    const int sb = threadIdx.x / kTps, ssub = threadIdx.x % kTps;  // 64 streams per pass, two passes
    float ssv2[kSspPerThread];
    const bool rms = a.ssp != nullptr;  // else the activations arrive normed (scale 1)
    {
        const uint32_t b1 = gb * kRowTile + sb, b2 = b1 + 64;
#pragma unroll
        for (int i = 0; i < kSspPerThread; i++) {
            const int t = ssub + kTps * i;
            ssv[i] = rms && b1 < a.n && t < a.tiles ? a.ssp[(size_t)b1 * a.tiles + t] : 0.0f;
            ssv2[i] = rms && b2 < a.n && t < a.tiles ? a.ssp[(size_t)b2 * a.tiles + t] : 0.0f;
        }
    }
    int4 wq[NP][kHwTiles];
    float4 rsc[kHwTiles];
#pragma unroll
    for (int i = 0; i < kHwTiles; i++) {
        const int t = min(t0 + i, w.rt - 1);
#pragma unroll
        for (int p = 0; p < NP; p++)
            if (p < np) wq[p][i] = ((const int4*)w.w)[((size_t)t * np + p) * 64 + lane];
        rsc[i] = *(const float4*)(w.scales + t * kRowTile + (lane / 16) * 4);
    }
    copy_group(smem, a.xw, gb, ks);
    {
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int i = 0; i < kSspPerThread; i++)
            if (ssub + kTps * i < a.tiles) {
                s1 += ssv[i];
                s2 += ssv2[i];
            }
#pragma unroll
        for (int o = 1; o < kTps; o <<= 1) {
            s1 += __shfl_xor(s1, o, kWave);
            s2 += __shfl_xor(s2, o, kWave);
        }
        if (ssub == 0) {
            invs[sb] = rms ? 1.0f / sqrtf(s1 / (float)a.d + 1e-5f) : 1.0f;
            invs[sb + 64] = rms ? 1.0f / sqrtf(s2 / (float)a.d + 1e-5f) : 1.0f;
        }
    }
    AFrag wd[NP][kHwTiles][2];
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int i = 0; i < kHwTiles; i++) {
            RawPair raw;
            raw.v[0] = p < np ? wq[p][i] : make_int4(0, 0, 0, 0);
            decode_pair<true>(raw, wd[p][i][0], wd[p][i][1]);
        }
    // Group gi's logits leave one iteration later, right after group gi + 2's copy is
    // requested: the wait at the top of an iteration (vector loads and stores share one
    // counter) then finds them issued a whole product earlier instead of just before.
    f32x4 held[kHwTiles];
    auto store_group = [&](int g) {
        const uint32_t b = (gb + g) * kRowTile + lane % 16;
        const float inv = invs[g * kRowTile + lane % 16];
#pragma unroll
        for (int i = 0; i < kHwTiles; i++) {
            const int t = t0 + i;
            const int r0 = t * kRowTile + (lane / 16) * 4;
            if (t >= w.rt || b >= a.n) continue;
            const float v[4] = {held[i][0] * rsc[i].x * inv, held[i][1] * rsc[i].y * inv, held[i][2] * rsc[i].z * inv,
                                held[i][3] * rsc[i].w * inv};
            float* o = a.out + (size_t)b * V + r0;
            // Logits are written once and read later (host copy, softmax): streamed.
            if (r0 + 3 < V && (V & 3) == 0) {
                __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, (f32x4*)o);
            } else {
                for (int e = 0; e < 4; e++)
                    if (r0 + e < V) __builtin_nontemporal_store(v[e], o + e);
            }
        }
    };
#pragma unroll 1
    for (int gi = 0; gi < ngr; gi++) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's copies and its stores of two groups back
        __syncthreads();                // every wave's copies of group gi, and reads of gi - 1
        if (gi + 1 < ngr) copy_group(smem + ((gi + 1) & 1) * buf_bytes, a.xw, gb + gi + 1, ks);
        if (gi > 0) store_group(gi - 1);
        const __bf16* lds = (const __bf16*)(smem + (gi & 1) * buf_bytes);
        f32x4 acc[kHwTiles];
#pragma unroll
        for (int i = 0; i < kHwTiles; i++) acc[i] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < NP; p++) {
            if (p >= np) continue;
            bf16x8 bf[2][3];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const __bf16* f = lds + ((size_t)(2 * p + h) * 3) * 512 + lane * 8;
#pragma unroll
                for (int m = 0; m < 3; m++) bf[h][m] = lds_frag(f + m * 512);
            }
            // mma_step's order per tile, the tiles' products interleaved.
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int j = 0; j < kProds<true>; j++)
#pragma unroll
                    for (int i = 0; i < kHwTiles; i++)
                        acc[i] = mma_prod<true>(j, wd[p][i][h], bf[h][0], bf[h][1], bf[h][2], acc[i]);
        }
#pragma unroll
        for (int i = 0; i < kHwTiles; i++) held[i] = acc[i];
    }
    if (ngr > 0) store_group(ngr - 1);
}

// ---------------------------------------------------------------- softmax

struct SoftmaxArgs {
    float* out;
    int vocab;
};

// softmax_into (tensor.rs:1917-1933) per stream, in place: max, exp(l - max) with the
// portable exp, the sum (fixed block tree instead of the sequential loop), division
// by max(sum, FLT_EPSILON).  Thread t owns elements t, t + 1024, ... and sums them in
// that order; the wave sums then meet in wave order.  PER > 0 (vocab <= 1024 PER) holds
// the thread's elements in registers, so the row is read once and written once; PER = 0
// walks the row in memory for each phase.  Both give the same bits.
constexpr int kSoftmaxPer = 50;  // vocab <= 51200 in registers (Mamba-130M: 50280)
template <int PER>
__global__ __launch_bounds__(1024) void k_softmax(SoftmaxArgs a) {
    __shared__ float sh[1024 / kWave];
    float* row = a.out + (size_t)blockIdx.x * a.vocab;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    float mx = -INFINITY;
    if constexpr (PER > 0) {
        float v[PER];
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = threadIdx.x + 1024 * k;
            v[k] = i < a.vocab ? row[i] : -INFINITY;
        }
#pragma unroll
        for (int k = 0; k < PER; k++) mx = fmaxf(mx, v[k]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
        if (lane == 0) sh[wave] = mx;
        __syncthreads();
        mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < 1024 / kWave; w++) mx = fmaxf(mx, sh[w]);
        __syncthreads();
        if (mx == -INFINITY) {
            const float u = 1.0f / (float)a.vocab;
#pragma unroll
            for (int k = 0; k < PER; k++)
                if (threadIdx.x + 1024 * k < a.vocab) row[threadIdx.x + 1024 * k] = u;
            return;
        }
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; k++) {
            if (threadIdx.x + 1024 * k < a.vocab) {
                v[k] = exp_f(v[k] - mx);
                s += v[k];
            }
        }
        s = wave_sum(s);
        if (lane == 0) sh[wave] = s;
        __syncthreads();
        float tsum = 0.0f;
#pragma unroll
        for (int w = 0; w < 1024 / kWave; w++) tsum += sh[w];
        const float denom = fmaxf(tsum, 1.1920929e-07f);
#pragma unroll
        for (int k = 0; k < PER; k++)
            if (threadIdx.x + 1024 * k < a.vocab) __builtin_nontemporal_store(v[k] / denom, row + threadIdx.x + 1024 * k);
        return;
    }
    for (int i = threadIdx.x; i < a.vocab; i += 1024) mx = fmaxf(mx, row[i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    if (lane == 0) sh[wave] = mx;
    __syncthreads();
    mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 1024 / kWave; w++) mx = fmaxf(mx, sh[w]);
    __syncthreads();
    if (mx == -INFINITY) {
        const float u = 1.0f / (float)a.vocab;
        for (int i = threadIdx.x; i < a.vocab; i += 1024) row[i] = u;
        return;
    }
    float s = 0.0f;
    for (int i = threadIdx.x; i < a.vocab; i += 1024) {
        const float e = exp_f(row[i] - mx);
        row[i] = e;
        s += e;
    }
    s = wave_sum(s);
    if (lane == 0) sh[wave] = s;
    __syncthreads();
    float tsum = 0.0f;
#pragma unroll
    for (int w = 0; w < 1024 / kWave; w++) tsum += sh[w];
    const float denom = fmaxf(tsum, 1.1920929e-07f);
    for (int i = threadIdx.x; i < a.vocab; i += 1024) row[i] = row[i] / denom;
}

// ---------------------------------------------------------------- reset

struct ZeroArgs {
    float* base;
    const uint32_t* slots;
    uint32_t cap;
    size_t stride, layer_stride;
    int nl;
};

__global__ __launch_bounds__(kBlock) void k_zero_slots(ZeroArgs a) {
    const uint32_t s = a.slots[blockIdx.y];
    if (s >= a.cap) return;
    for (int l = 0; l < a.nl; l++) {
        float* p = a.base + (size_t)l * a.layer_stride + (size_t)s * a.stride;
        for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < a.stride; i += (size_t)gridDim.x * kBlock)
            p[i] = 0.0f;
    }
}

// ---------------------------------------------------------------- step assembly

}  // namespace


namespace {

uint32_t stage_lds_bytes(int ks) { return (uint32_t)(kGroups * ks * 3 * kLimbBytes); }

// k_mix_in: the k-quarter partials, then the x_proj operand, and on the LayerNorm path the
// staged activations of kInGroups column groups (the same area, reused).
uint32_t mix_in_lds_bytes(int ks, bool pre, int tiles) {
    const uint32_t acts = pre ? 0u : kInGroups * ks * 3 * kLimbBytes;
    const uint32_t quarters = kWaves * tiles * kWave * sizeof(f32x4);
    const uint32_t xp_operand = (tiles / 2) * 3 * kLimbBytes;
    return std::max(acts, quarters + xp_operand);
}

template <bool Q8, bool Q8XP, bool PRE, bool GRP, int QP, int T>
const void* mix_in_fn6(uint32_t lds) {
    allow_lds(k_mix_in<Q8, Q8XP, PRE, GRP, QP, T>, lds);
    return (const void*)k_mix_in<Q8, Q8XP, PRE, GRP, QP, T>;
}

// The fixed shape and four-tile blocks are compiled for the pre-staged (RMSNorm) path,
// where the activations go straight to registers; the LayerNorm path keeps the general
// two-tile kernel.
template <bool Q8, bool Q8XP, bool PRE, bool GRP>
const void* mix_in_fn4(uint32_t lds, bool fixed, int tiles) {
    if constexpr (PRE) {
        if (tiles == 4)
            return fixed ? mix_in_fn6<Q8, Q8XP, PRE, GRP, kInFixedPairs, 4>(lds) : mix_in_fn6<Q8, Q8XP, PRE, GRP, 0, 4>(lds);
        return fixed ? mix_in_fn6<Q8, Q8XP, PRE, GRP, kInFixedPairs, 2>(lds) : mix_in_fn6<Q8, Q8XP, PRE, GRP, 0, 2>(lds);
    } else {
        return mix_in_fn6<Q8, Q8XP, PRE, GRP, 0, 2>(lds);
    }
}

template <bool Q8, bool Q8XP>
const void* mix_in_fn2(bool pre, bool grp, bool fixed, int tiles, uint32_t lds) {
    if (pre)
        return grp ? mix_in_fn4<Q8, Q8XP, true, Q8>(lds, fixed, tiles) : mix_in_fn4<Q8, Q8XP, true, false>(lds, fixed, tiles);
    return grp ? mix_in_fn4<Q8, Q8XP, false, Q8>(lds, false, 2) : mix_in_fn4<Q8, Q8XP, false, false>(lds, false, 2);
}

// k_mix_out: the fixed shape (kOutPairs k-pairs per wave) where out_proj's k-steps fit it.
const void* mix_out_fn(bool q8, int groups, bool fixed) {
    if (q8) {
        if (groups == 2) return fixed ? (const void*)k_mix_out<true, 2, true> : (const void*)k_mix_out<true, 2, false>;
        return fixed ? (const void*)k_mix_out<true, 1, true> : (const void*)k_mix_out<true, 1, false>;
    }
    if (groups == 2) return fixed ? (const void*)k_mix_out<false, 2, true> : (const void*)k_mix_out<false, 2, false>;
    return fixed ? (const void*)k_mix_out<false, 1, true> : (const void*)k_mix_out<false, 1, false>;
}

const void* mix_out_t_fn(int tt) {
    return tt == 4 ? (const void*)k_mix_out_t<true, 4> : tt == 3 ? (const void*)k_mix_out_t<true, 3>
                                                               : (const void*)k_mix_out_t<true, 2>;
}

// Row tiles per out_proj workgroup (quantized weights).  A step split into parts runs two
// parts' kernels at once, and their reads of the gated tiles (a group's tiles are read once
// per workgroup) compete for the caches' bandwidth: there two tiles per workgroup read them
// half as often (Mamba-130M int8 at 128 streams, two parts of 64: 624.8 -> 613.5 µs per
// step; 1024 streams unchanged).  One part alone loses by the halved number of workgroups
// (64 streams 470.8 -> 480.2 µs), so it keeps one tile; so do F32 weights, whose tiles
// outweigh the gated ones (128 streams 918 -> 962 µs with two).  REDUKT_GPU_OUT_TILES=1..4
// overrides the choice for quantized weights.
int out_tiles(bool q8, uint32_t n, uint32_t n_all) {
    const char* e = getenv("REDUKT_GPU_OUT_TILES");
    const int v = e && *e ? atoi(e) : 0;
    const int forced = v >= 1 && v <= 4 ? v : 0;
    if (!q8) return 1;
    return forced ? forced : (n_all > n ? 2 : 1);
}

const void* mix_in_fn(bool q8, bool q8xp, bool pre, bool grp, bool fixed, int tiles, uint32_t lds) {
    if (q8 && q8xp) return mix_in_fn2<true, true>(pre, grp, fixed, tiles, lds);
    if (q8) return mix_in_fn2<true, false>(pre, grp, fixed, tiles, lds);
    if (q8xp) return mix_in_fn2<false, true>(pre, false, fixed, tiles, lds);
    return mix_in_fn2<false, false>(pre, false, fixed, tiles, lds);
}

template <bool Q8>
const void* head_fn2(bool pre, uint32_t lds) {
    if (pre) {
        allow_lds(k_head<Q8, true>, lds);
        return (const void*)k_head<Q8, true>;
    }
    allow_lds(k_head<Q8, false>, lds);
    return (const void*)k_head<Q8, false>;
}

const void* head_fn(bool q8, bool pre, uint32_t lds) { return q8 ? head_fn2<true>(pre, lds) : head_fn2<false>(pre, lds); }

// Weights-stationary head for Q8 per-row weights with pre-staged activations and
// d <= 768 (12 k-pairs held per tile); null where it does not apply.
const void* head_ws_fn(int np, uint32_t lds) {
    if (np <= 2) { allow_lds(k_head_ws<2>, lds); return (const void*)k_head_ws<2>; }
    if (np <= 4) { allow_lds(k_head_ws<4>, lds); return (const void*)k_head_ws<4>; }
    if (np <= 8) { allow_lds(k_head_ws<8>, lds); return (const void*)k_head_ws<8>; }
    if (np <= 12) { allow_lds(k_head_ws<12>, lds); return (const void*)k_head_ws<12>; }
    return nullptr;
}

}  // namespace

Launch embed_launch(const TMat& emb, Pool& p, const StepIO& io, const float* nw0, __bf16* xw, float* ssp, int ks_x,
                    int tiles) {
    const int d = emb.cols;
    const uint32_t n_all = io.n_all ? io.n_all : io.n;
    EmbedArgs ea{emb, p.x, io.tokens + io.b0, io.slots + io.b0, p.slots, io.n, p.cap, io.check ? 1 : 0, io.err,
                 io.slots, n_all, io.b0, nullptr, 0, 0, nw0, xw, ssp, ks_x, tiles};
    return Launch::make((const void*)k_embed, dim3((d + 4 * kBlock - 1) / (4 * kBlock), io.n), dim3(kBlock), 0, KC_EMBED,
                        ea);
}

Launch head_launch(const TMat& H, Pool& p, const StepIO& io, const float* x, const float* nw, const float* nb,
                   const __bf16* xw, const float* ssp, int d, int tiles, bool ws) {
    const uint32_t n = io.n;
    HeadArgs ha{x, nw, nb, H, io.out + (size_t)io.b0 * H.rows, n, d, xw, ssp, tiles};
    if (ws) {
        const uint32_t lds_h = 2 * (uint32_t)H.ks * 3 * kLimbBytes;
        const int tiles_per_block = kHwWaves * kHwTiles;
        const uint32_t groups = (n + kRowTile - 1) / kRowTile;
        return Launch::make(head_ws_fn(H.ks / 2, lds_h),
                            dim3(xcd_grid((groups + kHwGroups - 1) / kHwGroups,
                                          (H.rt + tiles_per_block - 1) / tiles_per_block)),
                            dim3(kHwWaves * kWave), lds_h, KC_HEAD, ha);
    }
    const uint32_t lds_h = stage_lds_bytes(H.ks);
    const int tiles_per_block = kHeadWaves * kHeadTiles;
    return Launch::make(head_fn(H.group != 0, xw != nullptr, lds_h),
                        dim3(xcd_grid((n + kChunk - 1) / kChunk, (H.rt + tiles_per_block - 1) / tiles_per_block)),
                        dim3(kHeadWaves * kWave), lds_h, KC_HEAD, ha);
}

namespace {

ScanArgs scan_args(const DLayer& L, const Dims& D, const Pool& p, uint32_t n, __bf16* glimb, float* g32,
                   float* ssm_layer) {
    const int di = (int)D.di, nxp = di / kXpBlock;
    const int xr_pad = L.x_proj.rt * kRowTile;
    return ScanArgs{p.xpart, nxp, xr_pad, (int)D.xr(), p.u, p.z, ssm_layer, L.dt_w, L.dt_q, L.dt_scales, L.dt_pad,
                    L.dt_b, L.a_exp, L.d_vec, p.slots, p.xcap, n, p.scap, glimb, g32, di, (int)D.dr};
}

}  // namespace

Launch scan_launch(const DLayer& L, const Dims& D, Pool& p, uint32_t n, bool exact, __bf16* glimb, float* g32,
                   float* ssm_layer) {
    const int di = (int)D.di, nxp = di / kXpBlock;
    const uint32_t spt = scan_spt(n);
    const ScanArgs sa = scan_args(L, D, p, n, glimb, g32, ssm_layer);
    const void* fs = scan_fn(L.dt_q != nullptr, !exact, (int)D.dr, nxp, spt);
    return Launch::make(fs, dim3(xcd_grid((di + kBlock - 1) / kBlock, (n + spt - 1) / spt)), dim3(kBlock), 0, KC_SCAN,
                        sa);
}

Launch scan_exact_launch(const DLayer& L, const Dims& D, Pool& p, uint32_t n, bool fma, float* g32, float* ssm_layer) {
    const int di = (int)D.di;
    ScanArgs sa = scan_args(L, D, p, n, nullptr, g32, ssm_layer);
    sa.nxb = 1;   // one block: each stream's complete x_proj outputs
    const bool q8 = L.dt_q != nullptr;
    const void* fs = q8 ? (fma ? (const void*)k_scan<true, false, 0, 1, 1, true> : (const void*)k_scan<true, false, 0, 1, 1, false>)
                        : (fma ? (const void*)k_scan<false, false, 0, 1, 1, true> : (const void*)k_scan<false, false, 0, 1, 1, false>);
    return Launch::make(fs, dim3(xcd_grid((di + kBlock - 1) / kBlock, n)), dim3(kBlock), 0, KC_SCAN, sa);
}

Launch softmax_launch(float* out, int vocab, uint32_t n) {
    const void* f = vocab <= 1024 * kSoftmaxPer ? (const void*)k_softmax<kSoftmaxPer> : (const void*)k_softmax<0>;
    return Launch::make(f, dim3(n), dim3(1024), 0, KC_SOFTMAX, SoftmaxArgs{out, vocab});
}

namespace {

// The launches of one step, in stream order; io_index / head_index / softmax_index name
// the launches whose arguments carry caller pointers.
// The scratch arrays of one part of a step (rows from b0, a multiple of 16): every
// per-row array offset by b0 rows, every per-group array by b0 / 16 groups; the state,
// the partials' row stride (cap) and everything else unchanged.
Pool part_view(const Pool& p, const Dims& D, int ks_x, int xr_pad, uint32_t b0) {
    Pool q = p;
    if (b0 == 0) return q;
    const size_t g0 = b0 / kRowTile;
    q.x = p.x + (size_t)b0 * D.d;
    q.xw = p.xw + g0 * ks_x * 3 * 512;
    q.ssp = p.ssp + (size_t)b0 * (D.d / kRowTile);
    q.u = p.u + (size_t)b0 * D.di;
    q.z = p.z + (size_t)b0 * D.di;
    q.xpart = p.xpart + (size_t)b0 * xr_pad;
    q.glimb = p.glimb + g0 * (D.di / kKStep) * 3 * 512;
    q.slots = p.slots + b0;
    return q;
}

// The arguments of layer li's three kernels for a step of n streams on the scratch of p
// (the per-layer kernels and the persistent kernel's tasks take the same ones).
FlowLayer layer_args(const ModelView& m, const Pool& p, uint32_t n, uint32_t li, int nxb) {
    const Dims& D = *m.dims;
    const DLayer& L = m.layers[li];
    const int d = (int)D.d, di = (int)D.di;
    const bool pre = m.layers[0].norm_b == nullptr && m.norm_f_b == nullptr;
    const int xr_pad = m.layers[0].x_proj.rt * kRowTile;
    const int ks_x = m.layers[0].in_x.ks, tiles = d / kRowTile;
    const size_t conv_layer = (size_t)p.scap * di * (D.dc - 1);
    const size_t ssm_layer = (size_t)p.scap * di * 16;
    const float* nw_next = li + 1 < D.nl ? m.layers[li + 1].norm_w : m.norm_f_w;
    return FlowLayer{
        MixInArgs{p.x, L.norm_w, L.norm_b, L.in_x, L.in_z, L.x_proj, nxb, p.conv + li * conv_layer, L.conv_w, L.conv_b,
                  p.slots, p.xcap, n, p.scap, p.u, p.z, p.xpart, di, (int)D.dc, d, xr_pad, p.xw, p.ssp, tiles},
        scan_args(L, D, p, n, p.glimb, nullptr, p.ssm + li * ssm_layer),
        MixOutArgs{L.out_proj, p.glimb, p.x, n, d, nw_next, pre ? p.xw : nullptr, p.ssp, ks_x, tiles}};
}

void build_step(const ModelView& m, Pool& pool, const StepIO& io, std::vector<Launch>& out, int& io_index,
                int& head_index, int& softmax_index) {
    const Dims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d, di = (int)D.di;
    Pool p = part_view(pool, D, m.layers[0].in_x.ks, m.layers[0].x_proj.rt * kRowTile, io.b0);
    const uint32_t in_chunks = (n + kInChunk - 1) / kInChunk;
    const int out_g = m.layers[0].out_proj.group == 0 && n >= (uint32_t)kOutWideFrom ? 2 : 1;
    const uint32_t out_chunks = (n + out_g * kRowTile - 1) / (out_g * kRowTile);
    // k_mix_out's XCD layout: workgroups L and L + 8 share an XCD (and its L2).  Row-tile
    // major (the default) gives each XCD an eighth of the out_proj weights and every stream
    // group's gated tiles; chunk major (from kOutGroupMajorFrom streams, when the chunks come
    // in multiples of 8) gives each XCD an eighth of the stream groups and all the weights.
    // The first repeats the gated tiles (N x 9 KB), the second the weights (1.2 MB at
    // Mamba-130M int8), so the second reads less once N x 9 KB passes them.
    const bool gmajor = n >= (uint32_t)kOutGroupMajorFrom && out_chunks % kXcds == 0;
    // k_mix_in the same way: block major repeats each stream group's staged activations
    // (74 KB) on every XCD, chunk major repeats the in_proj and x_proj weights (2.5 MB).
    const bool in_gmajor = n >= (uint32_t)kInGroupMajorFrom && in_chunks % kXcds == 0;
    out.clear();
    // RMSNorm models take the pre-staged activation path; LayerNorm models norm in the
    // consumer.
    const bool pre = m.layers[0].norm_b == nullptr && m.norm_f_b == nullptr;
    // k_mix_in row tiles per workgroup and its conv-branch blocks; x_proj's split-K
    // partials stay 32-channel blocks (nxp) either way, so a stream's arithmetic does not
    // depend on the choice.
    const bool q8_row = m.layers[0].in_x.group != 0 && m.layers[0].in_x.group == m.layers[0].in_x.cols;
    const int in_tiles = pre && q8_row && n >= (uint32_t)kInWideFrom ? 4 : 2;
    const int nxb = di / (kRowTile * in_tiles);
    const int ks_x = m.layers[0].in_x.ks, tiles = d / kRowTile;
    io_index = (int)out.size();
    out.push_back(embed_launch(*m.emb, p, io, m.layers[0].norm_w, pre ? p.xw : nullptr, p.ssp, ks_x, tiles));
    const bool q8 = m.layers[0].in_x.group != 0;
    const bool q8xp = m.layers[0].x_proj.group != 0;
    const uint32_t lds_in = mix_in_lds_bytes(ks_x, pre, in_tiles);
    const bool grp = q8 && m.layers[0].in_x.group != m.layers[0].in_x.cols;
    const bool fixed = ks_x == 2 * kWaves * kInFixedPairs && m.layers[0].in_z.ks == ks_x;
    const void* fin = mix_in_fn(q8, q8xp, pre, grp, fixed, in_tiles, lds_in);
    const int tt = out_tiles(q8, n, io.n_all ? io.n_all : n);
    const size_t ssm_layer = (size_t)p.scap * di * 16;
    for (uint32_t li = 0; li < D.nl; li++) {
        const DLayer& L = m.layers[li];
        const FlowLayer la = layer_args(m, p, n, li, nxb);
        const int zb = L.in_z.rt / in_tiles;
        MixInArgs mi = la.mi;
        mi.gmajor = in_gmajor ? 1u : 0u;
        out.push_back(Launch::make(fin, in_gmajor ? dim3(in_chunks, nxb + zb) : dim3(nxb + zb, in_chunks), dim3(kBlock),
                                   lds_in, KC_MIX_IN, mi));
        out.push_back(scan_launch(L, D, p, n, m.exact_scan, p.glimb, nullptr, p.ssm + li * ssm_layer));
        const bool ofixed = m.layers[0].out_proj.ks == 2 * kOutWaves * kOutPairs;
        MixOutArgs mo = la.mo;
        mo.gmajor = gmajor ? 1u : 0u;
        if (ofixed && out_g == 1 && tt > 1 && L.out_proj.rt % tt == 0) {
            const uint32_t blocks = (uint32_t)(L.out_proj.rt / tt);
            out.push_back(Launch::make(mix_out_t_fn(tt), gmajor ? dim3(out_chunks, blocks) : dim3(blocks, out_chunks),
                                       dim3(kOutWaves * kWave), 0, KC_MIX_OUT, mo));
            continue;
        }
        const void* fo = mix_out_fn(q8, out_g, ofixed);
        out.push_back(Launch::make(fo, gmajor ? dim3(out_chunks, L.out_proj.rt) : dim3(L.out_proj.rt, out_chunks),
                                   dim3(kOutWaves * kWave), 0, KC_MIX_OUT, mo));
    }
    const TMat& H = *m.head;
    head_index = (int)out.size();
    const bool ws = pre && H.group != 0 && H.group == H.cols && H.ks / 2 <= 12;
    out.push_back(head_launch(H, p, io, p.x, m.norm_f_w, m.norm_f_b, pre ? p.xw : nullptr, p.ssp, d, tiles, ws));
    softmax_index = -1;
    if (io.probs) {
        softmax_index = (int)out.size();
        out.push_back(softmax_launch(io.out + (size_t)io.b0 * D.vocab, (int)D.vocab, n));
    }
}

hipError_t launch_direct(const Launch& l, hipStream_t st) {
    void* params[] = {l.argp};
    if (l.coop) return hipLaunchCooperativeKernel(l.fn, l.grid, l.block, params, l.lds, st);
    return hipLaunchKernel(l.fn, l.grid, l.block, params, l.lds, st);
}

hipKernelNodeParams node_params(const Launch& l, void** params) {
    hipKernelNodeParams kp{};
    kp.func = (void*)l.fn;
    kp.gridDim = l.grid;
    kp.blockDim = l.block;
    kp.sharedMemBytes = l.lds;
    kp.kernelParams = params;
    kp.extra = nullptr;
    return kp;
}

}  // namespace

#define RDK_TRY(expr)                    \
    do {                                 \
        hipError_t e_ = (expr);          \
        if (e_ != hipSuccess) return e_; \
    } while (0)

// REDUKT_GPU_GRAPH=0 issues every step as direct launches instead of a replayed hipGraph
// (for tools that do not follow graph launches).
static bool use_graphs() {
    static const bool on = [] {
        const char* e = getenv("REDUKT_GPU_GRAPH");
        return !(e && e[0] == '0');
    }();
    return on;
}

StepRunner::~StepRunner() { release(); }

void StepRunner::release() {
    clear();
    for (uint32_t k = 0; k < kMaxParts; k++) {
        if (aux_[k]) (void)hipStreamDestroy(aux_[k]);
        if (join_[k]) (void)hipEventDestroy(join_[k]);
        if (fork_[k]) (void)hipEventDestroy(fork_[k]);
        aux_[k] = nullptr;
        join_[k] = nullptr;
        fork_[k] = nullptr;
    }
    direct_.clear();
}

StepRunner& StepRunner::operator=(StepRunner&& o) noexcept {
    if (this == &o) return *this;
    release();
    graphs_ = std::move(o.graphs_);
    o.graphs_.clear();
    plans_ = std::move(o.plans_);
    o.plans_.clear();
    flow_from_ = o.flow_from_;
    direct_ = std::move(o.direct_);
    o.direct_.clear();
    clock_ = o.clock_;
    split_ = o.split_;
    skew_ = o.skew_;
    min_part_ = o.min_part_;
    for (uint32_t k = 0; k < kMaxParts; k++) {
        aux_[k] = o.aux_[k];
        join_[k] = o.join_[k];
        fork_[k] = o.fork_[k];
        o.aux_[k] = nullptr;
        o.join_[k] = nullptr;
        o.fork_[k] = nullptr;
    }
    return *this;
}

bool StepRunner::Graph::updatable() const {
    for (uint32_t k = 0; k < nparts; k++)
        if (!parts[k].updatable) return false;
    return true;
}

void StepRunner::destroy(Graph& g) {
    for (uint32_t k = 0; k < g.nparts; k++) {
        Part& pt = g.parts[k];
        if (pt.exec) (void)hipGraphExecDestroy(pt.exec);
        if (pt.g) (void)hipGraphDestroy(pt.g);
        delete pt.launches;
    }
    g = Graph{};
}

void StepRunner::clear() {
    for (Graph& g : graphs_) destroy(g);
    graphs_.clear();
    for (FlowPlan& f : plans_)
        if (f.dev) (void)hipFree(f.dev);
    plans_.clear();
}

// The persistent kernel's arguments for (p, n), made on first use (at most 8 kept, the
// least recently used evicted once the stream has finished with it).  out->shape.grid == 0
// when the kernel cannot run on this device.
hipError_t StepRunner::flow_plan(const StepSource& src, Pool& p, uint32_t n, size_t bytes, hipStream_t st,
                                 FlowPlan*& out) {
    out = nullptr;
    for (FlowPlan& f : plans_)
        if (f.pool == &p && f.n == n) out = &f;
    if (!out) {
        if (plans_.size() >= 8) {
            auto old = std::min_element(plans_.begin(), plans_.end(),
                                        [](const FlowPlan& a, const FlowPlan& b) { return a.last_use < b.last_use; });
            RDK_TRY(hipStreamSynchronize(st));
            if (old->dev) RDK_TRY(hipFree(old->dev));
            plans_.erase(old);
        }
        FlowPlan f;
        f.pool = &p;
        f.n = n;
        RDK_TRY(hipMalloc(&f.dev, bytes));
        const hipError_t e = src.flow_init(p, n, f.dev, &f.shape, st);
        if (e != hipSuccess) {
            (void)hipFree(f.dev);
            return e;
        }
        plans_.push_back(f);
        out = &plans_.back();
    }
    out->last_use = ++clock_;
    return hipSuccess;
}

uint32_t StepRunner::parts_of(uint32_t n, uint32_t k, uint32_t* b0, uint32_t* cnt) {
    // Whole 16-stream groups dealt as evenly as they go, the larger shares first; only the
    // last part may end in a partial group.
    const uint32_t groups = (n + kRowTile - 1) / kRowTile;
    const uint32_t parts = std::max(1u, std::min(k, groups));
    uint32_t g = 0;
    for (uint32_t i = 0; i < parts; i++) {
        const uint32_t take = groups / parts + (i < groups % parts ? 1 : 0);
        b0[i] = g * kRowTile;
        cnt[i] = std::min(n, (g + take) * kRowTile) - b0[i];
        g += take;
    }
    return parts;
}

// Streams for parts 1.. and the fork / join events, created once, at the default priority
// like the library's own stream.
hipError_t StepRunner::streams_ready(hipStream_t st, uint32_t parts) {
    (void)st;
    if (parts <= 1) return hipSuccess;
    for (uint32_t k = 0; k < parts; k++) {
        if (k > 0 && !aux_[k]) RDK_TRY(hipStreamCreateWithFlags(&aux_[k], hipStreamNonBlocking));
        if (k > 0 && !join_[k]) RDK_TRY(hipEventCreateWithFlags(&join_[k], hipEventDisableTiming));
        if (k + 1 < parts && !fork_[k]) RDK_TRY(hipEventCreateWithFlags(&fork_[k], hipEventDisableTiming));
    }
    return hipSuccess;
}

// Record launches [first, end) of one part as a graph by stream capture; the nodes whose
// arguments carry caller pointers are looked up in capture order and checked against their
// kernels (a launch before `first` is issued directly at every step).
hipError_t StepRunner::capture(const std::vector<Launch>& seq, uint32_t first, hipStream_t st, Part& pt) {
    RDK_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    hipError_t err = hipSuccess;
    for (size_t i = first; i < seq.size(); i++) {
        err = launch_direct(seq[i], st);
        if (err != hipSuccess) break;
    }
    hipGraph_t graph = nullptr;
    const hipError_t end = hipStreamEndCapture(st, &graph);
    if (err == hipSuccess) err = end;
    if (err != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return err;
    }
    pt.g = graph;
    size_t count = 0;
    RDK_TRY(hipGraphGetNodes(graph, nullptr, &count));
    std::vector<hipGraphNode_t> nodes(count);
    RDK_TRY(hipGraphGetNodes(graph, nodes.data(), &count));
    pt.updatable = count == seq.size() - first;
    auto pick = [&](int i, hipGraphNode_t& out) {
        out = nullptr;
        if (i < (int)first || !pt.updatable) return;
        hipKernelNodeParams kp{};
        if (hipGraphKernelNodeGetParams(nodes[i - first], &kp) == hipSuccess && kp.func == seq[i].fn) {
            out = nodes[i - first];
        } else {
            pt.updatable = false;
        }
    };
    pick(pt.io_i, pt.io_node);
    pick(pt.head_i, pt.head_node);
    pick(pt.sm_i, pt.softmax_node);
    return hipGraphInstantiate(&pt.exec, graph, nullptr, nullptr, 0);
}

void MambaStep::build(Pool& p, const StepIO& io, std::vector<Launch>& out, int& io_i, int& head_i, int& sm_i) const {
    build_step(m, p, io, out, io_i, head_i, sm_i);
}

// ---------------------------------------------------------------- persistent step kernel (host)

namespace {

// The shapes k_flow is compiled for: RMSNorm, int8 per-row in_proj and out_proj, x_proj
// and dt_proj both int8 per-row or both F32, d = 768 (k_mix_in's fixed shape),
// d_inner = 1536 (k_mix_out's fixed shape), dt_rank 48 and 48 x_proj blocks (the scan's).
bool flow_fits(const ModelView& m) {
    const Dims& D = *m.dims;
    const DLayer& L = m.layers[0];
    const bool pre = L.norm_b == nullptr && m.norm_f_b == nullptr;
    const bool row = [](const TMat& w) { return w.group != 0 && w.group == w.cols; }(L.in_x);
    const bool q8s = L.x_proj.group != 0;
    return pre && row && L.in_z.group == L.in_z.cols && L.out_proj.group == L.out_proj.cols &&
           (!q8s || L.x_proj.group == L.x_proj.cols) && q8s == (L.dt_q != nullptr) &&
           L.in_x.ks == 2 * kWaves * kInFixedPairs && L.in_z.ks == L.in_x.ks &&
           L.out_proj.ks == 2 * kOutWaves * kOutPairs && D.dr == 48 && D.di / kXpBlock == 48 &&
           D.di % kBlock == 0 && L.in_x.rt % 4 == 0 && L.in_z.rt % 4 == 0;
}

const void* flow_fn(const ModelView& m) {
    const bool q8s = m.layers[0].x_proj.group != 0, fast = !m.exact_scan;
    if (q8s) return fast ? (const void*)k_flow<true, true> : (const void*)k_flow<true, false>;
    return fast ? (const void*)k_flow<false, true> : (const void*)k_flow<false, false>;
}

size_t flow_table_bytes(uint32_t nl) { return ((size_t)nl * sizeof(FlowLayer) + 255) & ~(size_t)255; }
// Phase counters (kFlowSlices each), then one task ticket per XCC_ID value.
uint32_t flow_counters(uint32_t nl, uint32_t n) { return nl * 3u * ((n + kRowTile - 1) / kRowTile) * kFlowSlices + 16u; }
size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// The hand-over buffers of one layer of the persistent step kernel, rows rounded up to
// whole 16-stream groups, every array 256-byte aligned (so no cache line holds two
// groups' or two arrays' data): region l holds layer l's input (the residual x and its
// pre-staged activations xw / ssp) and what its phases pass on (u, z, the x_proj
// partials, the gated tiles); layer l's out_proj writes region l + 1's x / xw / ssp and
// region nl holds the head's input.
struct FlowRegion {
    float* x;
    __bf16* xw;
    float* ssp;
    float* u;
    float* z;
    float* xpart;
    __bf16* glimb;
};

size_t flow_region(const ModelView& m, uint32_t n, unsigned char* base, FlowRegion* r) {
    const Dims& D = *m.dims;
    const size_t groups = (n + kRowTile - 1) / kRowTile, rows = groups * kRowTile;
    const size_t ks_x = (size_t)m.layers[0].in_x.ks, xr_pad = (size_t)m.layers[0].x_proj.rt * kRowTile;
    const size_t sizes[7] = {rows * D.d * 4, groups * ks_x * 3 * 512 * 2, rows * (D.d / kRowTile) * 4,
                             rows * D.di * 4, rows * D.di * 4, (D.di / kXpBlock) * rows * xr_pad * 4,
                             groups * (D.di / kKStep) * 3 * 512 * 2};
    size_t off = 0;
    void* at[7];
    for (int i = 0; i < 7; i++) {
        at[i] = base ? base + off : nullptr;
        off += align256(sizes[i]);
    }
    if (r) *r = FlowRegion{(float*)at[0], (__bf16*)at[1], (float*)at[2], (float*)at[3], (float*)at[4],
                           (float*)at[5], (__bf16*)at[6]};
    return off;
}

size_t flow_regions_at(uint32_t nl, uint32_t n) {
    return align256(flow_table_bytes(nl) + (size_t)flow_counters(nl, n) * kFlowCounterStride * 4);
}

FlowRegion flow_region_of(const ModelView& m, uint32_t n, void* dev, uint32_t l) {
    FlowRegion r;
    const size_t one = flow_region(m, n, nullptr, nullptr);
    flow_region(m, n, (unsigned char*)dev + flow_regions_at(m.dims->nl, n) + l * one, &r);
    return r;
}

// Workgroups per CU of the persistent kernel: REDUKT_GPU_FLOW_WGS, else one below 512
// streams (a second workgroup on a CU slows both: 0.87 vs 1.10 ms per step at 128
// streams) and two from there (3.2 vs 5.0 ms at 1024), at most as many as fit.
// REDUKT_GPU_FLOW_STATIC=0: the persistent kernel keeps the ticket order even where the
// static assignment applies.
bool flow_static_wanted() {
    const char* e = getenv("REDUKT_GPU_FLOW_STATIC");
    return !(e && *e && !strcmp(e, "0"));
}

// Workgroups per CU of the persistent kernel: REDUKT_GPU_FLOW_WGS, else 2 (when 2 fit) for
// a static assignment of slots_per_xcd > 0, else 1 below 512 streams and 2 from there.
uint32_t flow_wgs_per_cu(uint32_t fit, uint32_t n, uint32_t slots_per_xcd) {
    const char* e = getenv("REDUKT_GPU_FLOW_WGS");
    if (e && *e) return std::max(1u, std::min((uint32_t)strtoul(e, nullptr, 10), fit));
    return std::max(1u, std::min(slots_per_xcd || n >= 512 ? 2u : 1u, fit));
}

// The static assignment's task slots per XCD (0: it does not apply): every phase has the
// same number of tasks per group, a multiple of the XCD count.
uint32_t flow_static_slots(const ModelView& m, uint32_t n, uint32_t nx) {
    const Dims& D = *m.dims;
    const DLayer& L0 = m.layers[0];
    const uint32_t mi = (uint32_t)((int)D.di / (kRowTile * 4) + L0.in_z.rt / 4);
    const uint32_t sc = kRowTile / kFlowScanSpt * (D.di / kBlock), mo = (uint32_t)L0.out_proj.rt;
    if (!flow_static_wanted() || nx == 0 || mi != sc || sc != mo || mi % nx) return 0;
    return (n + kRowTile - 1) / kRowTile * (mi / nx);
}

}  // namespace

size_t MambaStep::flow_bytes(const Pool& p, uint32_t n) const {
    (void)p;
    if (n == 0 || n > kFlowMaxStreams || !flow_fits(m)) return 0;
    return flow_regions_at(m.dims->nl, n) + (size_t)(m.dims->nl + 1) * flow_region(m, n, nullptr, nullptr);
}

hipError_t MambaStep::flow_init(Pool& p, uint32_t n, void* dev, FlowShape* shape, hipStream_t st) const {
    *shape = FlowShape{};
    const Dims& D = *m.dims;
    const void* fn = flow_fn(m);
    const uint32_t lds = mix_in_lds_bytes(m.layers[0].in_x.ks, true, 4);
    RDK_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    int fit = 0, cus = 0, dev_id = 0;
    RDK_TRY(hipGetDevice(&dev_id));
    RDK_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev_id));
    RDK_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&fit, fn, kBlock, lds));
    if (fit < 1 || cus < (int)kXcds || cus % kXcds != 0) {
        fprintf(stderr, "[redukt-gpu-hip] persistent step kernel off: %d workgroups per CU fit, %d CUs\n", fit, cus);
        return hipSuccess;
    }
    // The static assignment where one workgroup per CU cannot hold its slots (there the ticket
    // order would run each phase in several rounds) and two can: measured on Mamba-130M int8,
    // µs per step static / ticket order: 128 streams 715 / 757; one stream 431 / 407, 16
    // streams 488 / 477, 64 streams 520 / 507 (where one per CU holds them).
    const uint32_t slots = flow_static_slots(m, n, kXcds);
    const bool fixed = slots > (uint32_t)cus / kXcds && fit >= 2 && slots <= 2u * (uint32_t)cus / kXcds;
    const uint32_t g = flow_wgs_per_cu((uint32_t)fit, n, fixed ? slots : 0u) * (uint32_t)cus;
    // The device's XCDs, from one launch of the grid: the map goes to the counter area
    // (at least nl * 3 * 32 >= g words; the step's embedding clears it before every use).
    uint32_t* map = (uint32_t*)((unsigned char*)dev + flow_table_bytes(D.nl));
    if ((size_t)flow_counters(D.nl, n) * kFlowCounterStride < g) return hipSuccess;
    void* params[] = {&map};
    RDK_TRY(hipLaunchCooperativeKernel((const void*)k_xcc_map, dim3(g), dim3(kBlock), params, 0, st));
    RDK_TRY(hipStreamSynchronize(st));
    std::vector<uint32_t> seen(g);
    RDK_TRY(hipMemcpy(seen.data(), map, g * sizeof(uint32_t), hipMemcpyDeviceToHost));
    FlowShape sh;
    memset(sh.xmap, 0xff, sizeof(sh.xmap));
    for (uint32_t w = 0; w < g; w++)
        if (seen[w] < 16 && sh.xmap[seen[w]] == 0xff) sh.xmap[seen[w]] = (uint8_t)sh.nx++;
    // Each XCD takes the same number of tasks of every (layer, phase, group).
    const DLayer& L0 = m.layers[0];
    const int nxb = (int)D.di / (kRowTile * 4);
    const uint32_t tasks[3] = {(uint32_t)(nxb + L0.in_z.rt / 4), kRowTile / kFlowScanSpt * (D.di / kBlock),
                               (uint32_t)L0.out_proj.rt};
    if (sh.nx == 0 || tasks[0] % sh.nx || tasks[1] % sh.nx || tasks[2] % sh.nx) {
        fprintf(stderr, "[redukt-gpu-hip] persistent step kernel off: %u XCDs do not divide the phases' tasks\n",
                sh.nx);
        return hipSuccess;
    }
    // The per-layer argument table, for the whole step (one part): layer li reads and
    // writes its own hand-over region and leaves the next layer's input in region li + 1.
    std::vector<FlowLayer> table;
    table.reserve(D.nl);
    const uint32_t rows = (n + kRowTile - 1) / kRowTile * kRowTile;
    for (uint32_t li = 0; li < D.nl; li++) {
        const FlowRegion r = flow_region_of(m, n, dev, li), next = flow_region_of(m, n, dev, li + 1);
        Pool q = p;
        q.x = r.x;
        q.xw = r.xw;
        q.ssp = r.ssp;
        q.u = r.u;
        q.z = r.z;
        q.xpart = r.xpart;
        q.glimb = r.glimb;
        q.xcap = rows;
        FlowLayer fl = layer_args(m, q, n, li, nxb);
        fl.mo.x_out = next.x;
        fl.mo.xw = next.xw;
        fl.mo.ssp = next.ssp;
        table.push_back(fl);
    }
    RDK_TRY(hipMemcpy(dev, table.data(), table.size() * sizeof(FlowLayer), hipMemcpyHostToDevice));
    sh.grid = g;
    *shape = sh;
    sh.fixed = fixed && flow_static_slots(m, n, sh.nx) == slots && slots <= g / sh.nx ? 1u : 0u;
    fprintf(stderr, "[redukt-gpu-hip] persistent step kernel: %u streams, %u workgroups on %u XCDs, %s\n", n, g, sh.nx,
            sh.fixed ? "static tasks" : "ticket order");
    return hipSuccess;
}

void MambaStep::build_flow(Pool& p, const StepIO& io, void* dev, const FlowShape& shape, std::vector<Launch>& out) const {
    const Dims& D = *m.dims;
    const uint32_t n = io.n;
    const int d = (int)D.d, tiles = d / kRowTile, ks_x = m.layers[0].in_x.ks;
    const uint32_t groups = (n + kRowTile - 1) / kRowTile;
    uint32_t* cnt = (uint32_t*)((unsigned char*)dev + flow_table_bytes(D.nl));
    const FlowRegion first = flow_region_of(m, n, dev, 0), last = flow_region_of(m, n, dev, D.nl);
    out.clear();
    Pool q = p;
    q.x = first.x;   // the embedding writes layer 0's input region
    Launch e = embed_launch(*m.emb, q, io, m.layers[0].norm_w, first.xw, first.ssp, ks_x, tiles);
    EmbedArgs* ea = (EmbedArgs*)e.argp;
    ea->zero = cnt;
    ea->zero_n = flow_counters(D.nl, n);
    ea->zero_stride = kFlowCounterStride;
    out.push_back(std::move(e));
    const DLayer& L0 = m.layers[0];
    FlowArgs fa{(const FlowLayer*)dev, D.nl, groups, cnt, io.err,
                (uint32_t)((int)D.di / (kRowTile * 4) + L0.in_z.rt / 4), D.di / kBlock, (uint32_t)L0.out_proj.rt,
                shape.nx, shape.fixed, {}};
    memcpy(fa.xmap, shape.xmap, sizeof(fa.xmap));
    Launch f = Launch::make(flow_fn(m), dim3(shape.grid), dim3(kBlock), mix_in_lds_bytes(ks_x, true, 4), KC_FLOW, fa);
    f.coop = true;
    out.push_back(std::move(f));
    const TMat& H = *m.head;
    const bool ws = H.group != 0 && H.group == H.cols && H.ks / 2 <= 12;
    out.push_back(head_launch(H, p, io, last.x, m.norm_f_w, m.norm_f_b, last.xw, last.ssp, d, tiles, ws));
    if (io.probs) out.push_back(softmax_launch(io.out, (int)D.vocab, n));
}

hipError_t StepRunner::run_direct(const StepSource& src, Pool& p, const StepIO& io, hipStream_t st) {
    int io_i = -1, head_i = -1, sm_i = -1;
    src.build(p, io, direct_, io_i, head_i, sm_i);
    for (const Launch& l : direct_) RDK_TRY(launch_direct(l, st));
    return hipSuccess;
}

hipError_t StepRunner::run(const StepSource& src, Pool& p, const StepIO& io, hipStream_t st, Probe* probe) {
    const bool probing = probe && probe->cls != KC_NONE;
    if (flow_from_ && io.n >= flow_from_ && (!probing || probe->cls == KC_FLOW)) {
        const size_t fb = src.flow_bytes(p, io.n);
        FlowPlan* pl = nullptr;
        if (fb) RDK_TRY(flow_plan(src, p, io.n, fb, st, pl));
        if (pl && pl->shape.grid) {
            src.build_flow(p, io, pl->dev, pl->shape, direct_);
            for (const Launch& l : direct_) {
                // A probe of the persistent kernel brackets its launch with events on st.
                const bool on = probing && l.cls == KC_FLOW && probe->used + 2 <= probe->cap;
                if (on) RDK_TRY(hipEventRecord(probe->ev[probe->used], st));
                RDK_TRY(launch_direct(l, st));
                if (on) {
                    RDK_TRY(hipEventRecord(probe->ev[probe->used + 1], st));
                    probe->used += 2;
                }
            }
            return hipSuccess;
        }
    }
    if (probing) {
        std::vector<Launch> seq;
        int io_i = -1, head_i = -1, sm_i = -1;
        src.build(p, io, seq, io_i, head_i, sm_i);
        if (probe->only) {
            const bool rec = probe->used + 2 <= probe->cap;
            if (rec) RDK_TRY(hipEventRecord(probe->ev[probe->used], st));
            for (const Launch& l : seq)
                if (l.cls == probe->cls) RDK_TRY(launch_direct(l, st));
            if (rec) {
                RDK_TRY(hipEventRecord(probe->ev[probe->used + 1], st));
                probe->used += 2;
            }
            return hipSuccess;
        }
        // Probed launches carry their own dispatch start/stop timestamps.
        for (const Launch& l : seq) {
            const bool on = l.cls == probe->cls && probe->used + 2 <= probe->cap;
            if (on) {
                void* params[] = {l.argp};
                RDK_TRY(hipExtLaunchKernel(l.fn, l.grid, l.block, params, l.lds, st, probe->ev[probe->used],
                                           probe->ev[probe->used + 1], 0));
                probe->used += 2;
            } else {
                RDK_TRY(launch_direct(l, st));
            }
        }
        return hipSuccess;
    }
    uint32_t b0[kMaxParts], cnt[kMaxParts];
    const uint32_t want = std::min(split_, std::max(1u, io.n / min_part_));
    const uint32_t nparts = parts_of(io.n, src.splittable() ? want : 1, b0, cnt);
    RDK_TRY(streams_ready(st, nparts));
    auto part_io = [&](uint32_t k) {
        StepIO q = io;
        q.b0 = b0[k];
        q.n = cnt[k];
        q.n_all = io.n;
        return q;
    };
    auto stream_of = [&](uint32_t k) { return k == 0 ? st : aux_[k]; };
    // Part k > 0 starts once part k - 1 has issued its lead (so after everything queued on
    // st so far), and st waits for every part.
    auto start_part = [&](uint32_t k) -> hipError_t {
        if (k > 0) RDK_TRY(hipStreamWaitEvent(aux_[k], fork_[k - 1], 0));
        return hipSuccess;
    };
    auto after_lead = [&](uint32_t k) -> hipError_t {
        if (k + 1 < nparts) RDK_TRY(hipEventRecord(fork_[k], stream_of(k)));
        return hipSuccess;
    };
    auto join = [&]() -> hipError_t {
        for (uint32_t k = 1; k < nparts; k++) {
            RDK_TRY(hipEventRecord(join_[k], aux_[k]));
            RDK_TRY(hipStreamWaitEvent(st, join_[k], 0));
        }
        return hipSuccess;
    };
    if (!use_graphs()) {
        static const uint32_t skew = [] {
            const char* e = getenv("REDUKT_GPU_SKEW");
            return e && *e ? (uint32_t)strtoul(e, nullptr, 10) : 0u;
        }();
        std::vector<Launch> seqs[kMaxParts];
        for (uint32_t k = 0; k < nparts; k++) {
            int io_i = -1, head_i = -1, sm_i = -1;
            src.build(p, part_io(k), seqs[k], io_i, head_i, sm_i);
        }
        // Each part but the last issues its first `skew` kernels before the next part
        // starts, so consecutive parts run that many kernels apart.
        for (uint32_t k = 0; k < nparts; k++) {
            RDK_TRY(start_part(k));
            const size_t ahead = k + 1 < nparts ? std::min<size_t>(skew, seqs[k].size()) : 0;
            for (size_t i = 0; i < ahead; i++) RDK_TRY(launch_direct(seqs[k][i], stream_of(k)));
            RDK_TRY(after_lead(k));
            for (size_t i = ahead; i < seqs[k].size(); i++) RDK_TRY(launch_direct(seqs[k][i], stream_of(k)));
        }
        return join();
    }
    auto same_io = [&](const Graph& g) {
        return g.tokens == io.tokens && g.slots == io.slots && g.out == io.out && g.err == io.err;
    };
    Graph* hit = nullptr;
    for (Graph& g : graphs_)
        if (g.n == io.n && g.split == split_ && g.probs == io.probs && g.check == io.check && g.pool == &p &&
            (g.updatable() || same_io(g)))
            hit = &g;
    if (!hit) {
        if (graphs_.size() >= 8) {
            auto old = std::min_element(graphs_.begin(), graphs_.end(),
                                        [](const Graph& a, const Graph& b) { return a.last_use < b.last_use; });
            // The stream-ordered entry point returns without waiting: the evicted graphs
            // may still be queued or running (st waits for every part).
            RDK_TRY(hipStreamSynchronize(st));
            destroy(*old);
            graphs_.erase(old);
        }
        Graph g;
        g.n = io.n;
        g.split = split_;
        g.probs = io.probs;
        g.check = io.check;
        g.pool = &p;
        g.nparts = nparts;
        for (uint32_t k = 0; k < nparts; k++) {
            Part& pt = g.parts[k];
            pt.b0 = b0[k];
            pt.n = cnt[k];
            std::unique_ptr<std::vector<Launch>> seq(new std::vector<Launch>());
            src.build(p, part_io(k), *seq, pt.io_i, pt.head_i, pt.sm_i);
            pt.lead = k + 1 < nparts ? std::min<uint32_t>(skew_, (uint32_t)seq->size()) : 0u;
            const hipError_t e = capture(*seq, pt.lead, st, pt);
            if (e != hipSuccess) {
                destroy(g);
                return e;
            }
            pt.launches = seq.release();
        }
        graphs_.push_back(g);
        hit = &graphs_.back();
    } else if (!same_io(*hit)) {
        // Same shape, other caller pointers: each part's new arguments replace the stored
        // ones, so the graph's parameter storage stays alive with it.
        for (uint32_t k = 0; k < hit->nparts; k++) {
            Part& pt = hit->parts[k];
            std::vector<Launch> seq;
            int io_i = -1, head_i = -1, sm_i = -1;
            src.build(p, part_io(k), seq, io_i, head_i, sm_i);
            std::vector<Launch>& keep = *pt.launches;
            const int idx[3] = {pt.io_i, pt.head_i, pt.sm_i};
            const hipGraphNode_t nodes[3] = {pt.io_node, pt.head_node, pt.softmax_node};
            for (int j = 0; j < 3; j++) {
                if (idx[j] < 0) continue;
                keep[idx[j]] = std::move(seq[idx[j]]);
                if (idx[j] < (int)pt.lead) continue;   // issued directly from keep at every step
                void* prm[] = {keep[idx[j]].argp};
                hipKernelNodeParams kp = node_params(keep[idx[j]], prm);
                RDK_TRY(hipGraphExecKernelNodeSetParams(pt.exec, nodes[j], &kp));
            }
        }
    }
    hit->tokens = io.tokens;
    hit->slots = io.slots;
    hit->out = io.out;
    hit->err = io.err;
    hit->last_use = ++clock_;
    // Every part's lead and fork first, then the graphs from the last part to the first: a
    // graph's kernels start only once most of its launch is done (about 30 µs of host time
    // for a part), so in a call that finds the device idle the part launched first starts
    // first.  Launched last, part 0 on st then ends last, and st's wait for the other
    // parts finds them done instead of taking a cross-queue wake-up after them.
    for (uint32_t k = 0; k < hit->nparts; k++) {
        const Part& pk = hit->parts[k];
        RDK_TRY(start_part(k));
        for (uint32_t i = 0; i < pk.lead; i++) RDK_TRY(launch_direct((*pk.launches)[i], stream_of(k)));
        RDK_TRY(after_lead(k));
    }
    for (uint32_t k = hit->nparts; k-- > 0;) RDK_TRY(hipGraphLaunch(hit->parts[k].exec, stream_of(k)));
    return join();
}

// Rwkv7State::reset (rwkv7/model.rs:135-140) for the listed slots: both token-shift
// inputs and the WKV matrices of every layer (each slot's block is contiguous).
hipError_t enqueue_reset_rwkv(const RDims& D, Pool& P, const uint32_t* d_slots, uint32_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t sd = (size_t)D.nl * D.d, sw = (size_t)D.nl * D.h * D.n * D.n;
    float* bases[3] = {P.x_att, P.x_ffn, P.wkv};
    const size_t strides[3] = {sd, sd, sw};
    for (int i = 0; i < 3; i++) {
        ZeroArgs z{bases[i], d_slots, P.cap, strides[i], 0, 1};
        k_zero_slots<<<dim3((unsigned)std::min<size_t>((strides[i] + kBlock - 1) / kBlock, 4096), n), kBlock, 0, st>>>(z);
        RDK_TRY(hipGetLastError());
    }
    return hipSuccess;
}

hipError_t enqueue_reset(const Dims& D, Pool& P, const uint32_t* d_slots, uint32_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t conv_stride = (size_t)D.di * (D.dc - 1), ssm_stride = (size_t)D.di * 16;
    ZeroArgs zc{P.conv, d_slots, P.cap, conv_stride, (size_t)P.scap * conv_stride, (int)D.nl};
    k_zero_slots<<<dim3((unsigned)((conv_stride + kBlock - 1) / kBlock), n), kBlock, 0, st>>>(zc);
    RDK_TRY(hipGetLastError());
    ZeroArgs zs{P.ssm, d_slots, P.cap, ssm_stride, (size_t)P.scap * ssm_stride, (int)D.nl};
    k_zero_slots<<<dim3((unsigned)((ssm_stride + kBlock - 1) / kBlock), n), kBlock, 0, st>>>(zs);
    return hipGetLastError();
}

}  // namespace rdk
