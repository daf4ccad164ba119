// portable_math.h — the reference's portable f32 transcendentals, for host and device.
//
// redukt's CPU path computes exp and ln with its own IEEE-basic-operation routines
// (src/domain/tensor.rs:757-915: a Cephes degree-5 exp and the musl/FreeBSD logf) so
// that every platform produces the same bits.  Running the same algorithms on the GPU
// makes the element-wise phases (conv SiLU, softplus, selective scan, gate, softmax)
// bit-identical to the CPU path for identical inputs.  The constants are the published
// Cephes and musl coefficients the reference uses.  Floating-point contraction is off
// from here to the end of the including file: a fused a*b+c changes the last bit.
#pragma once
#pragma clang fp contract(off)

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define RDK_HD __host__ __device__ __forceinline__
#else
#define RDK_HD static inline
#endif

namespace rdk {

RDK_HD float bits_to_f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
RDK_HD uint32_t f_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// Round half to even with the 2^23 trick (tensor.rs:912-915).
RDK_HD float round_even(float x) {
    const float big = 8388608.0f;
    return x >= 0.0f ? (x + big) - big : (x - big) + big;
}

// exp(x): clamp to [-87.34, 88.38], n = round_even(x*log2e), two-constant Cody-Waite
// reduction, degree-5 polynomial, scale by 2^n built in the exponent field
// (tensor.rs:765-794).
RDK_HD float exp_f(float x) {
    const float lo = -87.3365447505531f, hi = 88.3762626647949f;
    x = x < lo ? lo : (x > hi ? hi : x);
    const float n_f = round_even(x * 1.44269504088896341f);
    const int32_t n = (n_f != n_f) ? 0 : (int32_t)n_f;
    const float r = (x - n_f * 6.93145751953125E-1f) - n_f * 1.42860682030941723212E-6f;
    const float r2 = r * r;
    float p = 1.9875691500E-4f;
    p = p * r + 1.3981999507E-3f;
    p = p * r + 8.3334519073E-3f;
    p = p * r + 4.1665795894E-2f;
    p = p * r + 1.6666665459E-1f;
    p = p * r + 5.0000001201E-1f;
    p = (p * r2 + r) + 1.0f;
    return p * bits_to_f((uint32_t)(n + 127) << 23);
}

// exp as one SIMD lane of the reference computes it: NaN becomes the lower clamp
// (tensor.rs:877-879).  lane_exp_arg is that argument rule alone, for callers that pick
// between the lane and the scalar form before one exp_f.
RDK_HD float lane_exp_arg(float x) { return x != x ? -87.3365447505531f : x; }
RDK_HD float lane_exp_f(float x) { return exp_f(lane_exp_arg(x)); }

// 1 / (1 + exp(0 - x)) (tensor.rs:883-885).
RDK_HD float lane_sigmoid_f(float x) { return 1.0f / (1.0f + lane_exp_f(0.0f - x)); }

// ln(x): reduce to [sqrt(2)/2, sqrt(2)], s = f/(2+f), even polynomial in s
// (tensor.rs:799-837).
RDK_HD float ln_f(float x) {
    uint32_t ix = f_to_bits(x);
    int32_t k = 0;
    if (ix < 0x00800000u || (ix >> 31) != 0) {
        if ((uint32_t)(ix << 1) == 0) return -bits_to_f(0x7f800000u);
        if ((ix >> 31) != 0) return bits_to_f(0x7fc00000u);
        k -= 25;
        ix = f_to_bits(x * bits_to_f(0x4c000000u));
    } else if (ix >= 0x7f800000u) {
        return x;
    } else if (ix == 0x3f800000u) {
        return 0.0f;
    }
    ix += 0x3f800000u - 0x3f3504f3u;
    k += (int32_t)(ix >> 23) - 0x7f;
    ix = (ix & 0x007fffffu) + 0x3f3504f3u;
    const float f = bits_to_f(ix) - 1.0f;
    const float s = f / (2.0f + f);
    const float dk = (float)k;
    const float z = s * s;
    const float w = z * z;
    const float t1 = w * (0.40000972152f + w * 0.24279078841f);
    const float t2 = z * (0.66666662693f + w * 0.28498786688f);
    const float hfsq = 0.5f * f * f;
    return s * (hfsq + (t2 + t1)) + dk * 9.0580006145e-06f - hfsq + f + dk * 6.9313812256e-01f;
}

// softplus with the reference's threshold of 20 (tensor.rs:859-861).
RDK_HD float softplus_f(float x) { return x > 20.0f ? x : ln_f(1.0f + exp_f(x)); }

}  // namespace rdk
