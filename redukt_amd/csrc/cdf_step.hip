// Logits -> u32 CDF on the GPU, bit for bit the host coding path's cdf_from_logits
// (src/application/codec.rs:785-798 with Cdf::from_probs, src/domain/coder.rs:43-81, and
// the table-driven f64 exp of src/domain/fmath.rs:340-430).
//
// Every frequency depends on the last bit of every f64 operation, so the arithmetic is
// the host's operation for operation (contraction off below): the same exp (integer bit
// manipulation plus IEEE double adds and multiplies, one rounding each), the same
// products and conversions.  Three things are order-dependent and are kept in order:
//   * the two f64 sums (sum of exp, then sum of the f32 probabilities): each is one
//     sequential chain of adds in index order, formed exactly by one workgroup per row in
//     integer rounds on the running sum's grid (k_cdf_sums);
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

constexpr uint32_t kSpan = 16;                      // consecutive elements per thread in a chunk
constexpr uint32_t kChunk = kSpan * kCdfBlock;      // elements per chunk workgroup

struct ChunkPart {
    double max;        // the chunk's max (NaN loses; -inf if none)
    uint64_t used;     // sum of the chunk's extra frequencies
    uint64_t best;     // (largest frequency << 32) | its last index
    uint32_t total;    // sum of the chunk's frequencies before the fix-up (u32, wrapping)
    uint32_t pad;
};

struct CdfArgs {
    const float* logits;   // [rows][n]
    uint32_t rows, n, chunks;
    double* e;             // [rows][n] scratch: exp(logit - max)
    double* sums;          // [rows][2] scratch: sum of e, sum of the probabilities
    ChunkPart* part;       // [rows][chunks] scratch
    uint32_t* cdf;         // [rows][n + 1]
};

// Block-wide reductions over kCdfBlock threads (four waves of 64).
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
    T r = sh[0];
#pragma unroll
    for (int i = 1; i < kCdfBlock / 64; i++) r = op(r, sh[i]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ double max_nan_loses(double m, double v) { return (!isnan(v) && !(v <= m)) ? v : m; }

// A row whose logits start on 16 bytes: its chunks are read four elements a lane.
__device__ __forceinline__ bool vec_row(const float* l) { return ((uintptr_t)l & 15) == 0; }

// Phase 1a (chunk c of row r): the chunk's max (f64::max folding, NaN loses).
__global__ __launch_bounds__(kCdfBlock) void k_cdf_max(CdfArgs a) {
    __shared__ double sh[kCdfBlock / 64];
    const uint32_t c = blockIdx.x, row = blockIdx.y, n = a.n;
    const float* l = a.logits + (size_t)row * n;
    double m = -__longlong_as_double(0x7ff0000000000000LL);
    const uint32_t i0 = c * kChunk, i1 = min(n, (c + 1) * kChunk);
    if (vec_row(l)) {
        // four consecutive elements a lane (chunks start at multiples of 4)
        for (uint32_t i = i0 + 4 * threadIdx.x; i < i1; i += 4 * kCdfBlock) {
            if (i + 4 <= i1) {
                const float4 v = *(const float4*)(l + i);
                m = max_nan_loses(max_nan_loses(m, (double)v.x), (double)v.y);
                m = max_nan_loses(max_nan_loses(m, (double)v.z), (double)v.w);
            } else {
                for (uint32_t k = i; k < i1; k++) m = max_nan_loses(m, (double)l[k]);
            }
        }
    } else {
        for (uint32_t i = i0 + threadIdx.x; i < i1; i += kCdfBlock) m = max_nan_loses(m, (double)l[i]);
    }
    // every partial is -inf or a number, so the combination order does not matter
    m = block_reduce<double>(m, [](double x, double y) { return (y <= x) ? x : y; }, sh);
    if (threadIdx.x == 0) a.part[(size_t)row * a.chunks + c].max = m;
}

// Phase 1b (chunk c of row r): the row's max from the chunk maxima, then e = exp(logit - max).
__global__ __launch_bounds__(kCdfBlock) void k_cdf_exp(CdfArgs a) {
    const uint32_t c = blockIdx.x, row = blockIdx.y, n = a.n;
    const ChunkPart* pr = a.part + (size_t)row * a.chunks;
    double m = pr[0].max;
    for (uint32_t i = 1; i < a.chunks; i++) m = (pr[i].max <= m) ? m : pr[i].max;
    const float* l = a.logits + (size_t)row * n;
    double* e = a.e + (size_t)row * n;
    const uint32_t i0 = c * kChunk, i1 = min(n, (c + 1) * kChunk);
    if (vec_row(l) && ((uintptr_t)e & 15) == 0) {
        for (uint32_t i = i0 + 4 * threadIdx.x; i < i1; i += 4 * kCdfBlock) {
            if (i + 4 <= i1) {
                const float4 v = *(const float4*)(l + i);
                *(double2*)(e + i) = make_double2(exp_f64((double)v.x - m, c_exp.v), exp_f64((double)v.y - m, c_exp.v));
                *(double2*)(e + i + 2) =
                    make_double2(exp_f64((double)v.z - m, c_exp.v), exp_f64((double)v.w - m, c_exp.v));
            } else {
                for (uint32_t k = i; k < i1; k++) e[k] = exp_f64((double)l[k] - m, c_exp.v);
            }
        }
    } else {
        for (uint32_t i = i0 + threadIdx.x; i < i1; i += kCdfBlock) e[i] = exp_f64((double)l[i] - m, c_exp.v);
    }
}

// Phase 2 (one workgroup per row): the two sequential f64 sums, in index order:
// sum = 0.0 + e[0] + e[1] + ... (codec.rs:791-794), then sum_p = -0.0 + p[0] + p[1] + ...
// (coder.rs:45-46) with p[i] = float(e[i] * (1 / sum)).  Every term is >= +0 or NaN.
//
// A sequential sum of non-negative terms can be computed exactly in parallel between binade
// changes of the running sum s.  While s stays in [2^E, 2^(E+1)), every double there is a
// multiple of u = 2^(E-52), s = T u with T < 2^53, and fl(s + x) = (T + a) u with
// a = round(x / u), as long as x / u is not a tie (fractional part exactly 1/2: then the
// result depends on the parity of T) and T + a < 2^53 (else the result leaves the binade
// and rounds on a coarser grid).  So a round takes 4096 terms, each thread forms a for 4
// of them, a block-wide prefix sum gives every T, and the first term that is a tie, a NaN,
// or takes T to 2^53 or beyond is an event: the terms before it are added as the integer
// sum, the event itself with one real f64 add, and the next round starts after it (on the
// new s's grid).  Below 2^-1022 the grid is the subnormal spacing 2^-1074 with the same
// rule.  A round without an event adds all its terms.  The result is the sequential sum
// bit for bit (an event changes s exactly as the sequential add does; between events the
// integer sum is exact).  The running sum of these rows stays below 2^24 (each term <= 1,
// n < 2^24), so the grid is always finer than 1.  The grid counts are integer-valued f64
// (no integer conversion is a single instruction for 64 bits): a sum of non-negative
// integers is exact whenever its result is below 2^53, and rounding is monotone, so a sum
// that reaches 2^53 still reads as >= 2^53 - the crossing test needs no more.  Prefixes
// are formed by adding, never by subtracting, so that this holds for each of them.
//
// The running sum of a row doubles about once per binade, and most of those crossings (and
// most ties, when the terms are still close to the sum) fall in the row's first few hundred
// terms: a round each.  So the first kHead terms are added one by one, in order, by one
// wave, from the registers of the lanes that loaded them (real f64 adds, the sequential sum
// itself), and the rounds start after them.
constexpr uint32_t kSumBlock = 1024;                 // threads of a row's workgroup
constexpr uint32_t kSumWaves = kSumBlock / 64;
constexpr uint32_t kTerms = 4;                       // terms per thread per round
constexpr uint32_t kRound = kTerms * kSumBlock;      // terms per round
constexpr uint32_t kHeadLanes = 64;                  // lanes of wave 0 whose terms form the head
constexpr uint32_t kHead = kHeadLanes * kTerms;      // terms added one by one
constexpr uint32_t kNoEvent = 0xffffffffu;
static_assert(kHeadLanes <= 64 && kHead <= kRound, "the head lies in wave 0's terms of the first window");

// A 64-bit value moved across lanes by DPP (each 32-bit half; lanes without a source
// read 0): a few cycles, against an LDS round trip for a lane permute.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = as_u64(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWS, 0xf, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWS, 0xf, true);
    return as_f64(((uint64_t)hi << 32) | lo);
}
// The same value in every lane, made visibly uniform (scalar registers): the round loop's
// control values come from LDS, and without this the compiler treats the loop as divergent
// (exec masking, and copies of the prefetched terms that wait for their loads every round).
__device__ __forceinline__ uint32_t uni(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ double uni(double v) {
    const uint64_t b = as_u64(v);
    const uint32_t lo = uni((uint32_t)b), hi = uni((uint32_t)(b >> 32));
    return as_f64(((uint64_t)hi << 32) | lo);
}

// Lane L's copy of v, in every lane (a constant lane: two scalar reads).
__device__ __forceinline__ double lane_f64(double v, int L) {
    const uint64_t b = as_u64(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, L);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), L);
    return as_f64(((uint64_t)hi << 32) | lo);
}

// Inclusive prefix sum over the wave's 64 lanes: shifts by 1, 2, 4, 8 within each row of
// 16 lanes, then the last lane of row 0 / 2 into rows 1 / 3 and lane 31 into rows 2 and 3.
__device__ __forceinline__ double wave_incl_sum(double v) {
    v += dpp_f64<0x111>(v);          // row_shr:1
    v += dpp_f64<0x112>(v);          // row_shr:2
    v += dpp_f64<0x114>(v);          // row_shr:4
    v += dpp_f64<0x118>(v);          // row_shr:8
    v += dpp_f64<0x142, 0xa>(v);     // row_bcast:15 into rows 1 and 3
    v += dpp_f64<0x143, 0xc>(v);     // row_bcast:31 into rows 2 and 3
    return v;
}

// LDS of a round, double-buffered by round parity so that a round's writes never meet the
// previous round's reads (two barriers per round).
struct SumShared {
    double part[2][kSumWaves];     // per-wave totals
    uint32_t first[2][kSumWaves];  // per-wave first event
    double t_ev[2][kSumWaves];     // the grid count before that event
    double x_ev[2][kSumWaves];     // that event's term
    double s;                      // the head's or the fallback's result
    double head[kHead];            // the head's terms in order
};

// A barrier for the rounds' LDS traffic only: LDS operations complete (lgkmcnt 0), then
// s_barrier.  __syncthreads would also wait for every global load in flight (vmcnt 0), and
// the next window's terms are loaded while this window's rounds run.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);   // vmcnt and expcnt at their maxima, lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <class F>
__device__ double exact_seq_sum(const double* __restrict__ e, uint32_t n, double s, F f, SumShared& sh) {
    const uint32_t t = threadIdx.x;
    const int lane = t % 64, w = t / 64;
    // The window's terms stay in registers (thread t: terms t kTerms .. + kTerms - 1).
    // The next window's terms are requested before this window's first round and arrive
    // while its rounds run; the rounds wait only for LDS.
    uint32_t par = 0;
    double nx[kTerms];
#pragma unroll
    for (uint32_t j = 0; j < kTerms; j++) nx[j] = e[min(t * kTerms + j, n - 1)];
    for (uint32_t k0 = 0; k0 < n; k0 += kRound) {
        double fx[kTerms];
        __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
        for (uint32_t j = 0; j < kTerms; j++) fx[j] = f(nx[j]);
        if (k0 + kRound < n) {
#pragma unroll
            for (uint32_t j = 0; j < kTerms; j++) nx[j] = e[min(k0 + kRound + t * kTerms + j, n - 1)];
        }
        // rounds over this window: after an event the rest of the window is re-gridded
        uint32_t from = 0;   // first term of the window not yet in s
        if (k0 == 0 && n >= kHead) {
            // the head: terms 0 .. kHead - 1 in order.  Wave 0 holds them (lane L: terms
            // L kTerms ..); it stores them to LDS in order and every lane reads them back
            // (same address: a broadcast) into one chain of adds.
            if (w == 0) {
#pragma unroll
                for (uint32_t j = 0; j < kTerms; j++)
                    if (lane < (int)kHeadLanes) sh.head[lane * kTerms + j] = fx[j];
                __builtin_amdgcn_s_waitcnt(0xc07f);   // this wave's LDS stores done
                __builtin_amdgcn_wave_barrier();
                double acc = s;
#pragma unroll 2
                for (uint32_t i = 0; i < kHead; i += 16) {
                    double v[16];
#pragma unroll
                    for (uint32_t k = 0; k < 16; k++) v[k] = sh.head[i + k];
#pragma unroll
                    for (uint32_t k = 0; k < 16; k++) acc += v[k];
                }
                if (lane == 0) sh.s = acc;
            }
            lds_barrier();
            s = uni(sh.s);
            from = kHead;
            lds_barrier();   // sh.s and sh.head are read before any later write to them
        }
        while (from < kRound && k0 + from < n) {
            if (isnan(s)) return s;   // stays NaN (only NaN-ness is used downstream)
            if (!(s < 0x1p52)) {
                // a grid of 1 or coarser (not reached by these rows): finish in order on one thread
                __syncthreads();
                if (t == 0) {
                    for (uint32_t i = k0 + from; i < n; i++) s += f(e[i]);
                    sh.s = s;
                }
                __syncthreads();
                return uni(sh.s);
            }
            // the grid of the current binade: terms scale by 2^ks into units of it
            int ks;
            double top;
            if (s < 0x1p-1022) {
                ks = 1074;
                top = 0x1p52;
            } else {
                ks = 52 - ilogb(s);
                top = 0x1p53;
            }
            const double T0 = ldexp(s, ks);   // exact and integer-valued: s is on the grid
            double a[kTerms];   // grid counts; 0 for events and for terms outside the round
            double c[kTerms];   // this thread's inclusive prefix of them
            bool live[kTerms];
            uint32_t ev = kNoEvent;   // this thread's first tie or NaN (index within the window)
            double mine = 0.0;
            // (straight-line: selects, no branches per term)
#pragma unroll
            for (uint32_t j = 0; j < kTerms; j++) {
                const uint32_t r = t * kTerms + j;
                live[j] = r >= from && k0 + r < n;
                const double q = ldexp(fx[j], ks);     // exact, or +inf past the double range
                // round half to even: every non-tie rounds as fl(s + x) does; q - m is exact
                const double m = rint(q);
                // NaN, inf or certainly past the binade; or a tie
                const bool bad = !(q < 0x1p53) || fabs(q - m) == 0.5;
                ev = (live[j] && bad && ev == kNoEvent) ? r : ev;
                a[j] = (live[j] && !bad) ? m : 0.0;
                mine += a[j];
                c[j] = mine;
            }
            // workgroup prefix of the grid counts: the lane's exclusive prefix in its wave
            // (the inclusive prefix of the lane before it), then the waves before it
            const double incl = wave_incl_sum(mine);
            if (lane == 63) sh.part[par][w] = incl;
            const double before = dpp_f64<0x138>(incl);   // wave_shr:1 (lane 0 reads 0)
            lds_barrier();
            // lanes 0 .. kSumWaves - 1 read one wave's total each; their inclusive prefix gives
            // the waves before this one and the workgroup's total
            double wp = lane < (int)kSumWaves ? sh.part[par][lane] : 0.0;
            wp += dpp_f64<0x111>(wp);   // row_shr:1, 2, 4, 8 within lanes 0 .. 15
            wp += dpp_f64<0x112>(wp);
            wp += dpp_f64<0x114>(wp);
            wp += dpp_f64<0x118>(wp);
            static_assert(kSumWaves <= 16, "the wave totals fit one DPP row");
            const double waves = w > 0 ? lane_f64(wp, (int)uni((uint32_t)(w - 1))) : 0.0;
            const double total = lane_f64(wp, (int)kSumWaves - 1);
            // crossings: the first term whose add takes T to the top of the binade, or this
            // thread's first tie or NaN, whichever comes first (lowest j wins)
            const double base = (T0 + waves) + before;
            uint32_t evn = kNoEvent;
            double T_ev = 0.0, x_ev = 0.0;
#pragma unroll
            for (int j = (int)kTerms - 1; j >= 0; j--) {
                const uint32_t r = t * kTerms + (uint32_t)j;
                const bool hit = live[j] && (r == ev || (r < ev && base + c[j] >= top));
                evn = hit ? r : evn;
                T_ev = hit ? (j > 0 ? base + c[j - 1] : base) : T_ev;
                x_ev = hit ? fx[j] : x_ev;
            }
            ev = evn;
            // the wave's first event sits in its lowest lane that has one (lanes hold
            // consecutive terms)
            const uint64_t has = __ballot(ev != kNoEvent);
            if (lane == 0) sh.first[par][w] = kNoEvent;
            if (has != 0) {
                const int src = __builtin_ctzll(has);
                if (lane == src) {
                    sh.first[par][w] = ev;
                    sh.t_ev[par][w] = T_ev;
                    sh.x_ev[par][w] = x_ev;
                }
            }
            lds_barrier();
            // the round's first event is the first event of the lowest wave that has one
            const uint32_t fv = lane < (int)kSumWaves ? sh.first[par][lane] : kNoEvent;
            const uint64_t hasw = __ballot(fv != kNoEvent);
            if (hasw == 0) {
                // no event: the window's remaining terms are the grid sum (T0 + total < 2^53)
                s = uni(ldexp(T0 + total, -ks));
                from = kRound;
            } else {
                // the event's add, done by every thread on the same operands
                const int fw = (int)uni((uint32_t)__builtin_ctzll(hasw));
                const double tv = lane < (int)kSumWaves ? sh.t_ev[par][lane] : 0.0;
                const double xv = lane < (int)kSumWaves ? sh.x_ev[par][lane] : 0.0;
                s = uni(ldexp(lane_f64(tv, fw), -ks) + lane_f64(xv, fw));
                from = (uint32_t)__builtin_amdgcn_readlane((int)fv, fw) + 1;
            }
            par ^= 1u;
        }
    }
    return s;
}

__global__ __launch_bounds__(kSumBlock) void k_cdf_sums(CdfArgs a) {
    __shared__ SumShared sh;
    const uint32_t row = blockIdx.x, n = a.n;
    const double* e = a.e + (size_t)row * n;
    const double s = uni(exact_seq_sum(e, n, 0.0, [](double v) { return v; }, sh));
    const double inv_sum = 1.0 / s;
    const double sp = exact_seq_sum(e, n, -0.0, [inv_sum](double v) { return (double)prob_of(v, inv_sum); }, sh);
    if (threadIdx.x == 0) {
        a.sums[2 * row] = s;
        a.sums[2 * row + 1] = sp;
    }
}

// Phase 3, Cdf::from_probs (coder.rs:43-81) from the two sums: extra[i] =
// (u64)(p[i] * inv * rem + 0.5) and freq[i] = 1 + extra[i]; the surplus or deficit goes to
// the last of the largest frequencies; then the cumulative frequencies.  3a gathers each
// chunk's used sum, its largest (frequency, last index) and its frequency total; 3b writes
// the chunk's cumulative frequencies from those.  Every combination here is an integer sum
// or a max, exact in any order.
struct FreqRow {
    double inv_sum, inv, rem;
    uint64_t remaining;
};
__device__ __forceinline__ FreqRow freq_row(const CdfArgs& a, uint32_t row) {
    FreqRow f;
    const double s = a.sums[2 * row], sum_p = a.sums[2 * row + 1];
    f.inv_sum = 1.0 / s;
    f.remaining = (uint64_t)kCdfTotal - a.n;
    f.inv = sum_p > 0.0 ? 1.0 / sum_p : 0.0;
    f.rem = (double)f.remaining;
    return f;
}
__device__ __forceinline__ uint64_t extra_of(double e, const FreqRow& f) {
    return sat_u64((double)prob_of(e, f.inv_sum) * f.inv * f.rem + 0.5);
}

__global__ __launch_bounds__(kCdfBlock) void k_cdf_freq_parts(CdfArgs a) {
    __shared__ uint64_t sh64[kCdfBlock / 64];
    __shared__ uint32_t sh32[kCdfBlock / 64];
    const uint32_t c = blockIdx.x, row = blockIdx.y, n = a.n;
    const FreqRow f = freq_row(a, row);
    const double* e = a.e + (size_t)row * n;
    uint64_t used = 0, best = 0;
    uint32_t total = 0;
    auto take = [&](double v, uint32_t i) {
        const uint64_t x = extra_of(v, f);
        const uint32_t fr = 1u + (uint32_t)x;
        used += x;
        total += fr;
        const uint64_t key = ((uint64_t)fr << 32) | i;
        best = key > best ? key : best;
    };
    const uint32_t i0 = c * kChunk, i1 = min(n, (c + 1) * kChunk);
    if (((uintptr_t)e & 15) == 0) {
        // two consecutive elements a lane (chunks start at even positions)
        for (uint32_t i = i0 + 2 * threadIdx.x; i < i1; i += 2 * kCdfBlock) {
            if (i + 2 <= i1) {
                const double2 v = *(const double2*)(e + i);
                take(v.x, i);
                take(v.y, i + 1);
            } else {
                take(e[i], i);
            }
        }
    } else {
        for (uint32_t i = i0 + threadIdx.x; i < i1; i += kCdfBlock) take(e[i], i);
    }
    used = block_reduce<uint64_t>(used, [](uint64_t x, uint64_t y) { return x + y; }, sh64);
    best = block_reduce<uint64_t>(best, [](uint64_t x, uint64_t y) { return x > y ? x : y; }, sh64);
    total = block_reduce<uint32_t>(total, [](uint32_t x, uint32_t y) { return x + y; }, sh32);
    if (threadIdx.x == 0) {
        ChunkPart& p = a.part[(size_t)row * a.chunks + c];
        p.used = used;
        p.best = best;
        p.total = total;
    }
}

// LDS index of a chunk position: one pad word per 32, so that both the coalesced pass
// (thread t at t + 256 j) and the per-thread pass (thread t at 16 t + j) meet no bank
// conflicts.
__device__ __forceinline__ uint32_t pad_ix(uint32_t p) { return p + p / 32; }

__global__ __launch_bounds__(kCdfBlock) void k_cdf_freq_write(CdfArgs a) {
    __shared__ uint32_t sh[kCdfBlock / 64];
    __shared__ uint32_t lfq[kChunk + kChunk / 32];   // the chunk's frequencies, then its cumulative ones
    const uint32_t c = blockIdx.x, row = blockIdx.y, n = a.n;
    const FreqRow f = freq_row(a, row);
    const ChunkPart* pr = a.part + (size_t)row * a.chunks;
    uint64_t used = 0, best = 0;
    uint32_t offset = 0;
    for (uint32_t i = 0; i < a.chunks; i++) {
        used += pr[i].used;
        best = pr[i].best > best ? pr[i].best : best;
        if (i < c) offset += pr[i].total;
    }
    const int64_t diff = (int64_t)f.remaining - (int64_t)used;
    const uint32_t at = (uint32_t)best;
    const uint32_t c0 = c * kChunk;
    if (diff != 0 && at < c0) offset = (uint32_t)((int64_t)offset + diff);   // u32 wrap, as the host's sum
    const double* e = a.e + (size_t)row * n;
    uint32_t* cdf = a.cdf + (size_t)row * (n + 1);
    // the chunk's frequencies, read coalesced (element c0 + t + 256 j)
#pragma unroll
    for (uint32_t j = 0; j < kSpan; j++) {
        const uint32_t p = threadIdx.x + kCdfBlock * j, i = c0 + p;
        uint32_t v = 0;
        if (i < n) {
            v = 1u + (uint32_t)extra_of(e[i], f);
            if (diff != 0 && i == at) v = (uint32_t)((int64_t)v + diff);
        }
        lfq[pad_ix(p)] = v;
    }
    __syncthreads();
    // thread t: kSpan consecutive elements; exclusive scan of the thread totals
    uint32_t fq[kSpan];
    uint32_t mine = 0;
#pragma unroll
    for (uint32_t j = 0; j < kSpan; j++) {
        fq[j] = lfq[pad_ix(threadIdx.x * kSpan + j)];
        mine += fq[j];
    }
    const int lane = threadIdx.x % 64, w = threadIdx.x / 64;
    uint32_t incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t up = __shfl_up(incl, o);
        if (lane >= o) incl += up;
    }
    if (lane == 63) sh[w] = incl;
    __syncthreads();
    uint32_t cum = offset + incl - mine;
#pragma unroll
    for (int i = 0; i < kCdfBlock / 64; i++)
        if (i < w) cum += sh[i];
    if (c == 0 && threadIdx.x == 0) cdf[0] = 0;
#pragma unroll
    for (uint32_t j = 0; j < kSpan; j++) {
        cum += fq[j];
        lfq[pad_ix(threadIdx.x * kSpan + j)] = cum;   // each thread rewrites only its own positions
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < kChunk && c0 + r < n; r += kCdfBlock) cdf[c0 + r + 1] = lfq[pad_ix(r)];
}

}  // namespace

namespace {
uint32_t cdf_chunks(uint32_t n) { return (n + kChunk - 1) / kChunk; }
}  // namespace

size_t cdf_scratch_bytes(uint32_t rows, uint32_t n) {
    return (size_t)rows * n * 8 + (size_t)rows * 16 + (size_t)rows * cdf_chunks(n) * sizeof(ChunkPart);
}

hipError_t cdf_launch(const float* logits, uint32_t rows, uint32_t n, void* scratch, uint32_t* cdf, hipStream_t st) {
    if (rows == 0) return hipSuccess;
    const uint32_t chunks = cdf_chunks(n);
    double* e = (double*)scratch;
    double* sums = e + (size_t)rows * n;
    ChunkPart* part = (ChunkPart*)(sums + 2 * (size_t)rows);
    CdfArgs a{logits, rows, n, chunks, e, sums, part, cdf};
    const dim3 grid(chunks, rows);
    k_cdf_max<<<grid, dim3(kCdfBlock), 0, st>>>(a);
    k_cdf_exp<<<grid, dim3(kCdfBlock), 0, st>>>(a);
    k_cdf_sums<<<dim3(rows), dim3(kSumBlock), 0, st>>>(a);
    k_cdf_freq_parts<<<grid, dim3(kCdfBlock), 0, st>>>(a);
    k_cdf_freq_write<<<grid, dim3(kCdfBlock), 0, st>>>(a);
    return hipGetLastError();
}

namespace {
// What the range coder reads of row r when its next symbol is known (coder.rs:163-177 via
// encode_symbol): out[3r] = cdf[r][sym[r]], out[3r + 1] = cdf[r][sym[r] + 1], out[3r + 2] =
// cdf[r][n], the total.  The host checked sym[r] < n; the clamp keeps every read inside
// the row whatever it holds.
__global__ __launch_bounds__(256) void k_cdf_pick(const uint32_t* __restrict__ cdf, uint32_t rows, uint32_t n,
                                                  const uint32_t* __restrict__ sym, uint32_t* __restrict__ out) {
    const uint32_t r = blockIdx.x * 256u + threadIdx.x;
    if (r >= rows) return;
    const uint32_t s = min(sym[r], n - 1);
    const uint32_t* row = cdf + (size_t)r * (n + 1);
    out[3 * (size_t)r] = row[s];
    out[3 * (size_t)r + 1] = row[s + 1];
    out[3 * (size_t)r + 2] = row[n];
}
}  // namespace

hipError_t cdf_pick_launch(const uint32_t* cdf, uint32_t rows, uint32_t n, const uint32_t* sym, uint32_t* out,
                           hipStream_t st) {
    if (rows == 0) return hipSuccess;
    k_cdf_pick<<<dim3((rows + 255) / 256), dim3(256), 0, st>>>(cdf, rows, n, sym, out);
    return hipGetLastError();
}

namespace {
// The symbol the range decoder finds in row r for its target cum[r] (coder.rs:100-115, the
// binary search of decode_symbol) with what it reads next: out[4r] = s, out[4r + 1] =
// cdf[r][s], out[4r + 2] = cdf[r][s + 1], out[4r + 3] = cdf[r][n]; s = n (both bounds
// cdf[r][n]) when cum[r] >= cdf[r][n].  One wave a row takes six levels of the search
// per round trip to memory: lane k (1..63) is node k of those levels' tree in heap order
// (children 2k: hi = mid, 2k + 1: lo = mid + 1), works out its node's interval from the
// bits of k and evaluates the node's test; the wave then walks the tree from the ballot.
// Every decision is the host search's own (the same mid of the same interval), so the
// result equals it for any row contents, monotone or not.
constexpr uint32_t kFindRows = 4;   // rows (waves) a workgroup

__global__ __launch_bounds__(64 * kFindRows) void k_cdf_find(const uint32_t* __restrict__ cdf, uint32_t rows,
                                                              uint32_t n, const uint32_t* __restrict__ cum,
                                                              uint32_t* __restrict__ out) {
    const uint32_t r = blockIdx.x * kFindRows + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (r >= rows) return;   // whole waves
    const uint32_t* row = cdf + (size_t)r * (n + 1);
    const uint32_t t = cum[r];
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        bool right = false;
        if (lane > 0) {
            uint32_t a = lo, b = hi;
            for (int d = 30 - __clz(lane); d >= 0 && a < b; d--) {   // path bits below the leading one
                const uint32_t m = a + (b - a) / 2;
                if ((lane >> d) & 1)
                    a = m + 1;
                else
                    b = m;
            }
            if (a < b) right = row[a + (b - a) / 2 + 1] <= t;
        }
        const uint64_t bits = __ballot(right);
        for (uint32_t level = 0, node = 1; level < 6 && lo < hi; level++) {
            const uint32_t m = lo + (hi - lo) / 2;
            if ((bits >> node) & 1) {
                lo = m + 1;
                node = 2 * node + 1;
            } else {
                hi = m;
                node = 2 * node;
            }
        }
    }
    if (lane == 0) {
        const uint32_t total = row[n];
        uint32_t* o = out + 4 * (size_t)r;
        o[0] = lo;
        o[1] = lo < n ? row[lo] : total;
        o[2] = lo < n ? row[lo + 1] : total;
        o[3] = total;
    }
}
}  // namespace

hipError_t cdf_find_launch(const uint32_t* cdf, uint32_t rows, uint32_t n, const uint32_t* cum, uint32_t* out,
                           hipStream_t st) {
    if (rows == 0) return hipSuccess;
    k_cdf_find<<<dim3((rows + kFindRows - 1) / kFindRows), dim3(64 * kFindRows), 0, st>>>(cdf, rows, n, cum, out);
    return hipGetLastError();
}

}  // namespace rdk
