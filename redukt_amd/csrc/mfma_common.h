// mfma_common.h — device building blocks shared by the step kernels of libredukt_gpu.so:
// v_mfma_f32_16x16x32_bf16, the three-limb bf16 split of f32 activations, and the
// fragment loads of pre-tiled weights (layouts in model.h, TMat).
#pragma once
// No a*b+c in this file may be fused: the element-wise arithmetic follows the
// reference operation by operation (a header is compiled before its includer's pragmas).
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "model.h"
#include "portable_math.h"

namespace rdk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_u8;

constexpr int kWave = 64;
constexpr int kLimbBytes = 64 * 8 * 2;     // one B fragment of one limb: 1 KB

__device__ __forceinline__ f32x4 mma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

struct Limb3 {
    __bf16 h, m, l;
};

// v = h + m + l: h = bf16(v), m = bf16(v - h), l = bf16(v - h - m); both differences are
// exact in f32, so only the last rounding (below 2^-24 relative) is lost.
__device__ __forceinline__ Limb3 split3(float v) {
    Limb3 o;
    o.h = (__bf16)v;
    const float r = v - (float)o.h;
    o.m = (__bf16)r;
    o.l = (__bf16)(r - (float)o.m);
    return o;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// v moved between lanes by the DPP control word CTRL (within rows of 16 lanes; a lane
// without a source reads 0).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppRowShl4 = 0x104;     // lane i reads lane i + 4
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2, 3, 0, 1]: lane i reads lane i ^ 2
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1, 0, 3, 2]: lane i reads lane i ^ 1

// The horizontal sum ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) of lanes 8k .. 8k + 7
// (lane 8k + l holding a_l), complete in lane 8k: each add pairs the same two values as
// that expression (IEEE addition is commutative).  The other seven lanes end with values of
// no use.
__device__ __forceinline__ float hsum8_lane0(float v) {
    v = v + dpp_move<kDppRowShl4>(v);
    v = v + dpp_move<kDppQuadXor2>(v);
    v = v + dpp_move<kDppQuadXor1>(v);
    return v;
}

// The wave's index within its workgroup as a wave-uniform (scalar) value: indices derived
// from it stay in scalar registers instead of being recomputed per lane.
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave)); }

__device__ __forceinline__ uint32_t clamp_slot(uint32_t s, uint32_t cap) { return s < cap ? s : cap - 1; }

// The device argument check of batch entry b of a step of n entries, run by every thread
// of one workgroup: a token past the vocabulary (tok_ok false) or a slot past the pool
// (error bit 0), or a slot that another entry also names (error bit 1, set for each of
// them; the earliest keeps the slot), sends the entry to the scratch slot `cap`, which no
// caller can name.  Thread 0 stores the slot the step uses; without `check` (entries the
// host validated) the slot is only clamped.
__device__ __forceinline__ void check_entry(const uint32_t* __restrict__ slots_in, uint32_t* __restrict__ slots,
                                            uint32_t n, uint32_t b, bool tok_ok, uint32_t cap, int check,
                                            uint32_t* err) {
    const uint32_t s = slots_in[b];
    if (check) {
        __shared__ int earlier;
        if (threadIdx.x == 0) earlier = 0;
        __syncthreads();
        bool dup = false, first_dup = false;
        for (uint32_t c = threadIdx.x; c < n; c += blockDim.x)
            if (c != b && slots_in[c] == s) {
                dup = true;
                if (c < b) first_dup = true;
            }
        if (first_dup) earlier = 1;
        const bool bad = !tok_ok || s >= cap;
        if (threadIdx.x == 0 && bad) atomicOr(err, 1u);
        if (dup) atomicOr(err, 2u);
        __syncthreads();
        if (threadIdx.x == 0) slots[b] = bad || earlier ? cap : s;
    } else if (threadIdx.x == 0) {
        slots[b] = clamp_slot(s, cap);
    }
}

// Workgroups are dealt to the XCDs round-robin by linear index (starting from wherever the
// previous dispatch stopped, so within one launch linear indices L and L + kXcds share an
// XCD, whichever XCD that is), and each XCD has its own L2.  A grid of `units` work units,
// each split into `parts` workgroups that read the same operands, is laid out 1-D over
// parts x (units rounded up to a multiple of kXcds): linear index L takes part
// (L / kXcds) % parts of unit kXcds ((L / kXcds) / parts) + L % kXcds.  The parts of a unit
// are then workgroups of one XCD and share its L2.  `live` is false past the last unit.
constexpr uint32_t kXcds = 8;
struct XcdTile {
    uint32_t unit, part;
    bool live;
};
__device__ __forceinline__ XcdTile xcd_tile(uint32_t lin, uint32_t parts, uint32_t units) {
    const uint32_t xi = lin / kXcds;
    XcdTile t;
    t.unit = (xi / parts) * kXcds + lin % kXcds;
    t.part = xi % parts;
    t.live = t.unit < units;
    return t;
}
inline uint32_t xcd_grid(uint32_t parts, uint32_t units) { return parts * ((units + kXcds - 1) / kXcds * kXcds); }

// ---------------------------------------------------------------- weight fragments

// The A operand of one k-step: F32 weights as three limbs, Q8 weights as one exact one.
struct AFrag {
    bf16x8 h, m, l;
};

// Raw bytes of the fragments of k-steps [2p, 2p+2) of one lane: Q8 16 B, F32 64 B.
struct RawPair {
    int4 v[4];
};

template <bool Q8>
__device__ __forceinline__ RawPair load_pair(const TMat& w, int t, int p, int lane) {
    RawPair r;
    if (Q8) {
        r.v[0] = ((const int4*)w.w)[((size_t)t * (w.ks / 2) + p) * 64 + lane];
    } else {
        const int4* base = (const int4*)w.w;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const size_t f = (((size_t)t * w.ks + 2 * p + h) * 64 + lane) * 2;
            r.v[2 * h] = base[f];
            r.v[2 * h + 1] = base[f + 1];
        }
    }
    return r;
}

template <bool Q8>
__device__ __forceinline__ void decode_pair(const RawPair& r, AFrag& a0, AFrag& a1) {
    if (Q8) {
        const int w[4] = {r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            a0.h[j] = (__bf16)(float)(int8_t)(w[j / 4] >> (8 * (j % 4)));
            a1.h[j] = (__bf16)(float)(int8_t)(w[2 + j / 4] >> (8 * (j % 4)));
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            AFrag& a = h ? a1 : a0;
            const int4 lo = r.v[2 * h], hi = r.v[2 * h + 1];
            const int w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const Limb3 t = split3(bits_to_f((uint32_t)w[j]));
                a.h[j] = t.h;
                a.m[j] = t.m;
                a.l[j] = t.l;
            }
        }
    }
}

// acc += A * B for one k-step: Q8 three products (B limbs hi, mid, lo), F32 the six limb
// products hi*hi, hi*mid, mid*hi, hi*lo, mid*mid, lo*hi — always in this order.
template <bool Q8>
__device__ __forceinline__ f32x4 mma_step(const AFrag& a, const bf16x8& bh, const bf16x8& bm, const bf16x8& bl,
                                          f32x4 acc) {
    if (Q8) {
        acc = mma(a.h, bh, acc);
        acc = mma(a.h, bm, acc);
        acc = mma(a.h, bl, acc);
    } else {
        acc = mma(a.h, bh, acc);
        acc = mma(a.h, bm, acc);
        acc = mma(a.m, bh, acc);
        acc = mma(a.h, bl, acc);
        acc = mma(a.m, bm, acc);
        acc = mma(a.l, bh, acc);
    }
    return acc;
}

// Product j (j < kProds<Q8>) of mma_step's sequence alone, so that a caller can interleave
// the products of several independent accumulators (a dependent MFMA waits for the whole
// latency of the previous one) while each accumulator still sees mma_step's order.
template <bool Q8>
constexpr int kProds = Q8 ? 3 : 6;

template <bool Q8>
__device__ __forceinline__ f32x4 mma_prod(int j, const AFrag& a, const bf16x8& bh, const bf16x8& bm, const bf16x8& bl,
                                          const f32x4& acc) {
    if (Q8) return mma(a.h, j == 0 ? bh : j == 1 ? bm : bl, acc);
    switch (j) {
        case 0: return mma(a.h, bh, acc);
        case 1: return mma(a.h, bm, acc);
        case 2: return mma(a.m, bh, acc);
        case 3: return mma(a.h, bl, acc);
        case 4: return mma(a.m, bm, acc);
        default: return mma(a.l, bh, acc);
    }
}

__device__ __forceinline__ bf16x8 lds_frag(const __bf16* base) { return *(const bf16x8*)base; }

// Limbs of four consecutive rows r0 + i (i < 4) of one output tile t, held by one lane in
// the MFMA D layout (r0 = 16 t + 4 (lane / 16), stream b = column lane % 16), written as the
// B operand of a following product whose k runs over those rows: buffer
// [b / 16][k-step][3 limbs][64 lanes][8] with `ks` k-steps.
template <int AUX = 0>
__device__ __forceinline__ void write_limbs4(__bf16* __restrict__ buf, int ks, int t, uint32_t b, const float (&v)[4]) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x % kWave;
    bf16x4 h, m, l;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const Limb3 t3 = split3(v[i]);
        h[i] = t3.h;
        m[i] = t3.m;
        l[i] = t3.l;
    }
    const int rr = (t % 2) * kRowTile + (lane / 16) * 4;  // row within k-step t / 2
    const int ln = (int)(b % kRowTile) + kRowTile * (rr / 8);
    __bf16* dst = buf + ((((size_t)(b / kRowTile) * ks + t / 2) * 3) * 64 + ln) * 8 + rr % 8;
    if constexpr (AUX == 0) {
        *(bf16x4*)dst = h;
        *(bf16x4*)(dst + 512) = m;
        *(bf16x4*)(dst + 1024) = l;
    } else {
        // written through to the device's coherence point with cache policy AUX (the
        // persistent step kernel's hand-over); buf is uniform and the offset < 2 GiB
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const auto r = __builtin_amdgcn_make_buffer_rsrc(buf, (short)0, 0x7fffffff, 0x00020000);
        const int off = (int)((dst - buf) * 2);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, h), r, off, 0, AUX);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, m), r, off + 1024, 0, AUX);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, l), r, off + 2048, 0, AUX);
    }
}

// Limbs of one value (stream b, column k) into a B-fragment buffer with `ks` k-steps.
__device__ __forceinline__ void write_limb1(__bf16* __restrict__ buf, int ks, uint32_t b, int k, float v) {
    const Limb3 t3 = split3(v);
    const int ln = (int)(b % kRowTile) + kRowTile * ((k % kKStep) / 8);
    __bf16* dst = buf + ((((size_t)(b / kRowTile) * ks + k / kKStep) * 3) * 64 + ln) * 8 + k % 8;
    dst[0] = t3.h;
    dst[512] = t3.m;
    dst[1024] = t3.l;
}

}  // namespace
}  // namespace rdk
