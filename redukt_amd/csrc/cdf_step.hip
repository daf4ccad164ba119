// Logits -> u32 CDF on the GPU, bit for bit the host coding path's cdf_from_logits
// (src/application/codec.rs:785-798 with Cdf::from_probs, src/domain/coder.rs:43-81, and
// the table-driven f64 exp of src/domain/fmath.rs:340-430).
//
// Every frequency depends on the last bit of every f64 operation, so the arithmetic is
// the host's operation for operation (contraction off below): the same exp (integer bit
// manipulation plus IEEE double adds and multiplies, one rounding each), the same
// products and conversions.  Three things are order-dependent and are kept in order:
//   * the two f64 sums (sum of exp, then sum of the f32 probabilities): each is one
//     sequential chain of adds in index order, run by one lane per row (k_cdf_sums);
//   * the argmax of the fix-up takes the last of equal maxima, a reduction whose result
//     does not depend on the order it is combined in;
//   * `used` and the cumulative frequencies are integer sums (exact in any order).
// Everything else is element-wise and runs on every lane.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "host/exp_table.h"
#include "step.h"

#pragma clang fp contract(off)

namespace rdk {
namespace {

constexpr uint32_t kCdfTotal = 1u << 24;   // REDUKT_CDF_TOTAL
constexpr int kCdfBlock = 256;

__device__ __forceinline__ double as_f64(uint64_t b) { return __longlong_as_double((long long)b); }
__device__ __forceinline__ uint64_t as_u64(double d) { return (uint64_t)__double_as_longlong(d); }

// The host's 2^(k/128) table (generated from decimal arithmetic), copied into constant
// memory at compile time.
template <size_t... I>
struct ExpTable {
    uint64_t v[sizeof...(I)];
};
template <size_t... I>
constexpr ExpTable<I...> exp_table(std::index_sequence<I...>) {
    return ExpTable<I...>{{redukt_exp::kTable[I]...}};
}
__constant__ const auto c_exp = exp_table(std::make_index_sequence<256>{});

// exp(x) in f64, the host's redukt_exp_f64 (fmath.rs:383-430): x = k ln2/128 + r,
// e^x = 2^(k/128) e^r with the 128-entry table, a degree-5 polynomial for e^r - 1 - r,
// and the host's paths for tiny, huge and subnormal results.
__device__ double exp_out_of_range(double x, uint32_t abstop) {
    if (as_u64(x) == 0xfff0000000000000ULL) return 0.0;   // -inf
    if (abstop >= 0x7ff) return 1.0 + x;                  // +inf stays +inf, NaN propagates
    return (as_u64(x) >> 63) ? 0.0 : __longlong_as_double(0x7ff0000000000000LL);
}

__device__ double exp_rescale(double tmp, uint64_t sbits, uint64_t ki) {
    if ((ki & 0x80000000ULL) == 0) {
        const double scale = as_f64(sbits - (1009ULL << 52));
        return as_f64(uint64_t(1009 + 1023) << 52) * (scale + scale * tmp);
    }
    const double scale = as_f64(sbits + (1022ULL << 52));
    double y = scale + scale * tmp;
    if (y < 1.0) {
        double lo = scale - y + scale * tmp;
        const double hi = 1.0 + y;
        lo = 1.0 - hi + y + lo;
        y = (hi + lo) - 1.0;
        if (y == 0.0) y = 0.0;
    }
    return as_f64(1ULL << 52) * y;
}

__device__ double exp_f64(double x, const uint64_t* __restrict__ table) {
    constexpr uint64_t kPoly[4] = {0x3fdffffffffffdbdULL, 0x3fc555555555543cULL, 0x3fa55555cf172b91ULL,
                                   0x3f81111167a4d017ULL};
    constexpr uint64_t kShiftBits = 0x4338000000000000ULL;
    uint32_t abstop = uint32_t(as_u64(x) >> 52) & 0x7ff;
    bool rescale = false;
    if (abstop - 0x3c9u >= 0x408u - 0x3c9u) {
        if (abstop - 0x3c9u >= 0x80000000u) return 1.0 + x;
        if (abstop >= 0x409u) return exp_out_of_range(x, abstop);
        rescale = true;
    }
    const double z = as_f64(redukt_exp::kInvLn2N) * x;
    double kd = z + as_f64(kShiftBits);
    const uint64_t ki = as_u64(kd);
    kd -= as_f64(kShiftBits);
    const double r = x + kd * as_f64(redukt_exp::kNegLn2HiN) + kd * as_f64(redukt_exp::kNegLn2LoN);
    const uint64_t idx = 2 * (ki & 127);
    const uint64_t top = ki << 45;
    const double tail = as_f64(table[idx]);
    const uint64_t sbits = table[idx + 1] + top;
    const double r2 = r * r;
    const double tmp = tail + r + r2 * (as_f64(kPoly[0]) + r * as_f64(kPoly[1])) +
                       r2 * r2 * (as_f64(kPoly[2]) + r * as_f64(kPoly[3]));
    if (rescale) return exp_rescale(tmp, sbits, ki);
    const double scale = as_f64(sbits);
    return scale + scale * tmp;
}

// Rust's `f as u64`: truncation toward zero, NaN -> 0, saturating at both ends.
__device__ __forceinline__ uint64_t sat_u64(double v) {
    if (!(v > 0.0)) return 0;
    if (v >= 18446744073709551616.0) return ~0ULL;
    return (uint64_t)v;
}

// One row's f32 probability, the host's p[i] = float(e[i] * inv_sum).
__device__ __forceinline__ float prob_of(double e, double inv_sum) { return (float)(e * inv_sum); }

struct CdfArgs {
    const float* logits;   // [rows][n]
    uint32_t rows, n;
    double* e;             // [rows][n] scratch: exp(logit - max)
    double* sums;          // [rows][2] scratch: sum of e, sum of the probabilities
    uint32_t* cdf;         // [rows][n + 1]
};

// Block-wide reductions over kCdfBlock threads (8 waves... 4 waves of 64).
template <class T, class F>
__device__ T block_reduce(T v, F op, T* sh) {
    const int lane = threadIdx.x % 64, w = threadIdx.x / 64;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const T u = __shfl_xor(v, o);
        v = op(v, u);
    }
    if (lane == 0) sh[w] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        T r = sh[0];
        for (int i = 1; i < kCdfBlock / 64; i++) r = op(r, sh[i]);
        sh[kCdfBlock / 64] = r;
    }
    __syncthreads();
    const T r = sh[kCdfBlock / 64];
    __syncthreads();
    return r;
}

// Phase 1 (one workgroup per row): max over the row (f64::max, NaN loses; -inf if every
// entry is NaN, as the host's fold), then e[i] = exp(logit[i] - max).
__global__ __launch_bounds__(kCdfBlock) void k_cdf_exp(CdfArgs a) {
    __shared__ double sh[kCdfBlock / 64 + 1];
    const uint32_t row = blockIdx.x, n = a.n;
    const float* l = a.logits + (size_t)row * n;
    double m = -__longlong_as_double(0x7ff0000000000000LL);
    for (uint32_t i = threadIdx.x; i < n; i += kCdfBlock) {
        const double v = (double)l[i];
        if (!isnan(v) && !(v <= m)) m = v;
    }
    // every partial is -inf or a number, so the combination order does not matter
    m = block_reduce<double>(m, [](double x, double y) { return (y <= x) ? x : y; }, sh);
    double* e = a.e + (size_t)row * n;
    for (uint32_t i = threadIdx.x; i < n; i += kCdfBlock) e[i] = exp_f64((double)l[i] - m, c_exp.v);
}

// Phase 2 (one workgroup per row): the two sequential f64 sums, in index order:
// sum = 0.0 + e[0] + e[1] + ... (codec.rs:791-794), then sum_p = -0.0 + p[0] + p[1] + ...
// (coder.rs:45-46) with p[i] = float(e[i] * (1 / sum)).  Each is one dependent chain of adds,
// run by wave 0 (every lane the same chain, lane 0's result kept) out of an LDS ring that
// waves 1-3 fill from HBM kLead chunks ahead, so the chain waits on LDS (about a hundred
// cycles, reads returned in order) instead of on memory.
constexpr uint32_t kChunk = 1024;   // doubles per ring slot (8 KB)
constexpr uint32_t kSlots = 4;
constexpr uint32_t kLead = 2;       // chunks the producers run ahead of the chain

template <class F>
__device__ double ring_sum(const double* __restrict__ e, uint32_t n, double s, F f, double* ring) {
    const uint32_t chunks = (n + kChunk - 1) / kChunk;
    const uint32_t wave = threadIdx.x / 64, pt = threadIdx.x - 64;   // producer thread index (waves 1-3)
    // a producer thread's share of a chunk: every load issued before the first store
    constexpr uint32_t kProducers = kCdfBlock - 64;
    constexpr uint32_t kPer = (kChunk + kProducers - 1) / kProducers;
    auto produce = [&](uint32_t c) {
        double* slot = ring + (c % kSlots) * kChunk;
        const uint32_t base = c * kChunk, len = min(kChunk, n - base);
        double t[kPer];
#pragma unroll
        for (uint32_t j = 0; j < kPer; j++) {
            const uint32_t i = pt + j * kProducers;
            t[j] = e[base + min(i, len - 1)];
        }
#pragma unroll
        for (uint32_t j = 0; j < kPer; j++) {
            const uint32_t i = pt + j * kProducers;
            if (i < len) slot[i] = t[j];
        }
    };
    if (wave != 0)
        for (uint32_t c = 0; c < kLead && c < chunks; c++) produce(c);
    __syncthreads();
    for (uint32_t c = 0; c < chunks; c++) {
        if (wave != 0) {
            if (c + kLead < chunks) produce(c + kLead);
        } else {
            const double* slot = ring + (c % kSlots) * kChunk;
            const uint32_t len = min(kChunk, n - c * kChunk);
            uint32_t i = 0;
            for (; i + 32 <= len; i += 32) {
                double v[32];
#pragma unroll
                for (int j = 0; j < 32; j++) v[j] = slot[i + j];
#pragma unroll
                for (int j = 0; j < 32; j++) s += f(v[j]);
            }
            for (; i < len; i++) s += f(slot[i]);
        }
        __syncthreads();
    }
    return s;
}

__global__ __launch_bounds__(kCdfBlock) void k_cdf_sums(CdfArgs a) {
    __shared__ double ring[kSlots * kChunk];
    static_assert(kLead < kSlots, "a slot is refilled only after the chain has left it");
    const uint32_t row = blockIdx.x, n = a.n;
    const double* e = a.e + (size_t)row * n;
    const double s = ring_sum(e, n, 0.0, [](double v) { return v; }, ring);
    const double inv_sum = 1.0 / s;
    const double sp = ring_sum(e, n, -0.0, [inv_sum](double v) { return (double)prob_of(v, inv_sum); }, ring);
    if (threadIdx.x == 0) {
        a.sums[2 * row] = s;
        a.sums[2 * row + 1] = sp;
    }
}

// Phase 3 (one workgroup per row): Cdf::from_probs (coder.rs:43-81) from the two sums:
// extra[i] = (u64)(p[i] * inv * rem + 0.5), freq[i] = 1 + extra[i]; the surplus or deficit
// goes to the last of the largest frequencies; then the cumulative frequencies.  Thread t
// owns the contiguous span [t * per, (t + 1) * per) for the prefix sums.
__global__ __launch_bounds__(kCdfBlock) void k_cdf_freq(CdfArgs a) {
    __shared__ uint64_t sh64[kCdfBlock / 64 + 1];
    __shared__ uint32_t shu[kCdfBlock];
    const uint32_t row = blockIdx.x, n = a.n;
    const double* e = a.e + (size_t)row * n;
    uint32_t* cdf = a.cdf + (size_t)row * (n + 1);
    const double s = a.sums[2 * row], sum_p = a.sums[2 * row + 1];
    const double inv_sum = 1.0 / s;
    const uint64_t remaining = (uint64_t)kCdfTotal - n;
    const double inv = sum_p > 0.0 ? 1.0 / sum_p : 0.0;
    const double rem = (double)remaining;
    auto extra_of = [&](uint32_t i) {
        return sat_u64((double)prob_of(e[i], inv_sum) * inv * rem + 0.5);
    };
    // used (exact integer sum) and the fix-up position: the largest frequency, last index
    // among equals; both reductions are order-independent.
    uint64_t used = 0;
    uint64_t best = 0;   // (freq << 32) | index: the larger freq, then the larger index
    for (uint32_t i = threadIdx.x; i < n; i += kCdfBlock) {
        const uint64_t x = extra_of(i);
        used += x;
        const uint64_t key = ((uint64_t)(uint32_t)(1u + (uint32_t)x) << 32) | i;
        best = key > best ? key : best;
    }
    used = block_reduce<uint64_t>(used, [](uint64_t x, uint64_t y) { return x + y; }, sh64);
    best = block_reduce<uint64_t>(best, [](uint64_t x, uint64_t y) { return x > y ? x : y; }, sh64);
    const int64_t diff = (int64_t)remaining - (int64_t)used;
    const uint32_t at = (uint32_t)best;
    auto freq_of = [&](uint32_t i) {
        uint32_t f = 1u + (uint32_t)extra_of(i);
        if (diff != 0 && i == at) f = (uint32_t)((int64_t)f + diff);
        return f;
    };
    // prefix sums over contiguous spans (u32, wrapping like the host's)
    const uint32_t per = (n + kCdfBlock - 1) / kCdfBlock;
    const uint32_t i0 = min(n, threadIdx.x * per), i1 = min(n, i0 + per);
    uint32_t tot = 0;
    for (uint32_t i = i0; i < i1; i++) tot += freq_of(i);
    shu[threadIdx.x] = tot;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int t = 0; t < kCdfBlock; t++) {
            const uint32_t v = shu[t];
            shu[t] = run;
            run += v;
        }
        cdf[0] = 0;
    }
    __syncthreads();
    uint32_t cum = shu[threadIdx.x];
    for (uint32_t i = i0; i < i1; i++) {
        cum += freq_of(i);
        cdf[i + 1] = cum;
    }
}

}  // namespace

size_t cdf_scratch_bytes(uint32_t rows, uint32_t n) { return (size_t)rows * n * 8 + (size_t)rows * 16; }

hipError_t cdf_launch(const float* logits, uint32_t rows, uint32_t n, void* scratch, uint32_t* cdf, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    CdfArgs a{logits, rows, n, (double*)scratch, (double*)scratch + (size_t)rows * n, cdf};
    k_cdf_exp<<<dim3(rows), dim3(kCdfBlock), 0, st>>>(a);
    k_cdf_sums<<<dim3(rows), dim3(kCdfBlock), 0, st>>>(a);
    k_cdf_freq<<<dim3(rows), dim3(kCdfBlock), 0, st>>>(a);
    return hipGetLastError();
}

}  // namespace rdk
