// Host coding path: table-driven double exp, logits -> CDF, and the carry range coder.
//
// Bit compatibility with the reference host is the point of this file, so three things
// are kept exactly as the reference computes them (each cited below):
//   * the exp algorithm: 7-bit table of 2^(k/128), range reduction by ln2/128 split in a
//     hi/lo pair, degree-5 polynomial, special paths for tiny, huge and subnormal results;
//   * the order of every floating-point operation of the softmax and of Cdf::from_probs
//     (sequential f64 sums, left-to-right products), which fixes the rounding of each
//     frequency;
//   * the coder's integer state machine (u64 low with carry cache, 32-bit range, byte-wise
//     renormalisation below 2^24).
// This translation unit must be built without FP contraction (-ffp-contract=off): a fused
// multiply-add changes the last bit of exp and of the frequencies.
#include "redukt_codec.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <new>
#include <vector>

#include "coder.h"
#include "exp_table.h"
#include "host_pool.h"

namespace {

inline double as_f64(uint64_t b) {
    double d;
    std::memcpy(&d, &b, sizeof d);
    return d;
}
inline uint64_t as_u64(double d) {
    uint64_t b;
    std::memcpy(&b, &d, sizeof b);
    return b;
}

// Polynomial of exp(r) - 1 - r on |r| <= ln2/256 (orders 2..5): the published minimax
// coefficients of the musl / ARM optimized-routines exp (EXP_POLY_ORDER 5), which the
// reference uses (src/domain/fmath.rs:113-118).  They are data of the algorithm and must
// match bit for bit.
constexpr uint64_t kPoly[4] = {0x3fdffffffffffdbdULL, 0x3fc555555555543cULL, 0x3fa55555cf172b91ULL,
                               0x3f81111167a4d017ULL};
constexpr uint64_t kShiftBits = 0x4338000000000000ULL;  // 1.5 * 2^52: rounds z to an integer

// |x| >= 1024, infinities and NaN (fmath.rs:421-430).
double exp_out_of_range(double x, uint32_t abstop) {
    if (as_u64(x) == as_u64(-std::numeric_limits<double>::infinity())) return 0.0;
    if (abstop >= 0x7ff) return 1.0 + x;  // +inf stays +inf, NaN propagates
    return (as_u64(x) >> 63) ? 0.0 : std::numeric_limits<double>::infinity();
}

// Result whose exponent left the normal range during reconstruction: scale * (1 + tmp)
// with one final rounding, including the subnormal band (fmath.rs:352-379).
double exp_rescale(double tmp, uint64_t sbits, uint64_t ki) {
    if ((ki & 0x80000000ULL) == 0) {
        // k > 0: scale carries up to 2^460 too much; take 2^1009 out and put it back.
        const double scale = as_f64(sbits - (1009ULL << 52));
        return as_f64(uint64_t(1009 + 1023) << 52) * (scale + scale * tmp);
    }
    // k < 0: compute at 2^1022 above the final scale, then scale down once.
    const double scale = as_f64(sbits + (1022ULL << 52));
    double y = scale + scale * tmp;
    if (y < 1.0) {
        // Round to the subnormal precision in two steps that cannot double-round.
        double lo = scale - y + scale * tmp;
        const double hi = 1.0 + y;
        lo = 1.0 - hi + y + lo;
        y = (hi + lo) - 1.0;
        if (y == 0.0) y = 0.0;  // no -0
    }
    return as_f64(1ULL << 52) * y;  // 2^-1022
}

}  // namespace

extern "C" double redukt_exp_f64(double x) {
    // src/domain/fmath.rs:383-416.  Exponent field bounds: 2^-54 -> 0x3c9, 512 -> 0x408,
    // 1024 -> 0x409, inf -> 0x7ff.
    uint32_t abstop = uint32_t(as_u64(x) >> 52) & 0x7ff;
    bool rescale = false;
    if (abstop - 0x3c9u >= 0x408u - 0x3c9u) {
        if (abstop - 0x3c9u >= 0x80000000u) return 1.0 + x;  // |x| < 2^-54
        if (abstop >= 0x409u) return exp_out_of_range(x, abstop);
        rescale = true;  // 512 <= |x| < 1024: the result may leave the normal range
    }
    // x = k*ln2/128 + r with |r| <= ln2/256; e^x = 2^(k/128) * e^r.
    const double z = as_f64(redukt_exp::kInvLn2N) * x;
    double kd = z + as_f64(kShiftBits);
    const uint64_t ki = as_u64(kd);
    kd -= as_f64(kShiftBits);
    const double r = x + kd * as_f64(redukt_exp::kNegLn2HiN) + kd * as_f64(redukt_exp::kNegLn2LoN);
    const uint64_t idx = 2 * (ki & 127);
    const uint64_t top = ki << 45;  // k/128 of the exponent, in place
    const double tail = as_f64(redukt_exp::kTable[idx]);
    const uint64_t sbits = redukt_exp::kTable[idx + 1] + top;
    const double r2 = r * r;
    const double tmp = tail + r + r2 * (as_f64(kPoly[0]) + r * as_f64(kPoly[1])) +
                       r2 * r2 * (as_f64(kPoly[2]) + r * as_f64(kPoly[3]));
    if (rescale) return exp_rescale(tmp, sbits, ki);
    const double scale = as_f64(sbits);
    return scale + scale * tmp;
}

namespace {

// Rust's `f as u64`: truncation toward zero, NaN -> 0, saturating at both ends.
inline uint64_t sat_u64(double v) {
    if (!(v > 0.0)) return 0;
    if (v >= 18446744073709551616.0) return ~0ULL;
    return uint64_t(v);
}

}  // namespace

int32_t redukt_host::cdf_from_probs_impl(const float* probs, uint32_t n, uint32_t* cdf, uint32_t* freqs) {
    // src/domain/coder.rs:43-81.
    const uint64_t remaining = uint64_t(REDUKT_CDF_TOTAL) - n;
    double sum_p = -0.0;
    for (uint32_t i = 0; i < n; ++i) sum_p += double(probs[i]);
    const double inv = sum_p > 0.0 ? 1.0 / sum_p : 0.0;
    const double rem = double(remaining);
    uint64_t used = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const uint64_t extra = sat_u64(double(probs[i]) * inv * rem + 0.5);  // round to nearest
        freqs[i] = 1u + uint32_t(extra);
        used += extra;
    }
    const int64_t diff = int64_t(remaining) - int64_t(used);
    if (diff != 0) {
        // The rounding surplus or deficit goes to the largest frequency; among equal
        // maxima the last one (Iterator::max_by_key).
        uint32_t at = 0;
        for (uint32_t i = 1; i < n; ++i)
            if (freqs[i] >= freqs[at]) at = i;
        freqs[at] = uint32_t(int64_t(freqs[at]) + diff);
    }
    uint32_t cum = 0;
    cdf[0] = 0;
    for (uint32_t i = 0; i < n; ++i) {
        cum += freqs[i];
        cdf[i + 1] = cum;
    }
    return REDUKT_CODEC_OK;
}

// One logits row (src/application/codec.rs:785-798); e, p and f are n-element scratch.
int32_t redukt_host::cdf_from_logits_impl(const float* logits, uint32_t n, uint32_t* cdf, double* e, float* p, uint32_t* f) {
    double max_l = -std::numeric_limits<double>::infinity();
    for (uint32_t i = 0; i < n; ++i) {
        const double l = double(logits[i]);
        if (!std::isnan(l) && !(l <= max_l)) max_l = l;  // f64::max: NaN loses
    }
    double sum = 0.0;
    for (uint32_t i = 0; i < n; ++i) {
        e[i] = redukt_exp_f64(double(logits[i]) - max_l);
        sum += e[i];
    }
    const double inv_sum = 1.0 / sum;
    for (uint32_t i = 0; i < n; ++i) p[i] = float(e[i] * inv_sum);
    return cdf_from_probs_impl(p, n, cdf, f);
}

namespace {

inline bool valid_n(uint32_t n) { return n >= 1 && n < REDUKT_CDF_TOTAL; }

// Per-thread scratch of the row functions (grows to the largest vocabulary seen).
struct RowScratch {
    std::vector<double> e;
    std::vector<float> p;
    std::vector<uint32_t> f;
    void fit(uint32_t n) {
        if (e.size() < n) {
            e.resize(n);
            p.resize(n);
            f.resize(n);
        }
    }
};
thread_local RowScratch t_scratch;

}  // namespace

void redukt_host::cdf_from_logits_row(const float* logits, uint32_t n, uint32_t* cdf) {
    t_scratch.fit(n);
    cdf_from_logits_impl(logits, n, cdf, t_scratch.e.data(), t_scratch.p.data(), t_scratch.f.data());
}

extern "C" int32_t redukt_cdf_from_probs(const float* probs, uint32_t n, uint32_t* cdf) {
    if (!probs || !cdf || !valid_n(n)) return REDUKT_CODEC_INVALID_ARG;
    t_scratch.fit(n);
    return redukt_host::cdf_from_probs_impl(probs, n, cdf, t_scratch.f.data());
}

extern "C" int32_t redukt_cdf_uniform(uint32_t n, uint32_t* cdf) {
    // src/domain/coder.rs:83-93 (n <= 2^24 keeps every frequency >= 1).
    if (!cdf || n == 0 || n > REDUKT_CDF_TOTAL) return REDUKT_CODEC_INVALID_ARG;
    const uint32_t each = REDUKT_CDF_TOTAL / n;
    for (uint32_t i = 0; i <= n; ++i) cdf[i] = i * each;
    return REDUKT_CODEC_OK;
}

extern "C" int32_t redukt_cdf_from_logits(const float* logits, uint32_t n, uint32_t* cdf) {
    if (!logits || !cdf || !valid_n(n)) return REDUKT_CODEC_INVALID_ARG;
    t_scratch.fit(n);
    redukt_host::cdf_from_logits_row(logits, n, cdf);
    return REDUKT_CODEC_OK;
}

extern "C" int32_t redukt_cdf_from_logits_batch(const float* logits, uint32_t rows, uint32_t n, uint32_t* cdf,
                                                uint32_t threads) {
    if (!valid_n(n)) return REDUKT_CODEC_INVALID_ARG;
    if (rows == 0) return REDUKT_CODEC_OK;
    if (!logits || !cdf) return REDUKT_CODEC_INVALID_ARG;
    redukt_host::parallel_for(rows, threads, [&](size_t r) {
        redukt_host::cdf_from_logits_row(logits + size_t(r) * n, n, cdf + size_t(r) * (size_t(n) + 1));
    });
    return REDUKT_CODEC_OK;
}

extern "C" uint32_t redukt_cdf_lookup(const uint32_t* cdf, uint32_t n, uint32_t cum_freq) {
    // src/domain/coder.rs:100-115; returns n when cum_freq >= cdf[n].
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (cdf[mid + 1] <= cum_freq)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

// ---- range coder C API (the state machines live in coder.h) ---------------------------

extern "C" redukt_rc_encoder* redukt_rc_encoder_new(void) { return new (std::nothrow) redukt_rc_encoder(); }

extern "C" void redukt_rc_encoder_free(redukt_rc_encoder* enc) { delete enc; }

extern "C" int32_t redukt_rc_encode(redukt_rc_encoder* enc, uint32_t lo, uint32_t hi, uint32_t total) {
    if (!enc) return REDUKT_CODEC_INVALID_ARG;
    return enc->encode(lo, hi, total);
}

extern "C" int32_t redukt_rc_encode_symbol(redukt_rc_encoder* enc, uint32_t sym, const uint32_t* cdf, uint32_t n) {
    if (!enc || !cdf) return REDUKT_CODEC_INVALID_ARG;
    return enc->encode_symbol(sym, cdf, n);
}

extern "C" size_t redukt_rc_encoder_size(const redukt_rc_encoder* enc) { return enc ? enc->size() : 0; }

extern "C" size_t redukt_rc_finish(redukt_rc_encoder* enc, uint8_t* out, size_t cap) {
    if (!enc) return 0;
    enc->finish();
    const size_t len = enc->out.size();
    if (out && cap) std::memcpy(out, enc->out.data(), std::min(len, cap));
    return len;
}

extern "C" redukt_rc_decoder* redukt_rc_decoder_new(const uint8_t* data, size_t len) {
    if (!data && len) return nullptr;
    auto* dec = new (std::nothrow) redukt_rc_decoder();
    if (!dec) return nullptr;
    dec->start(data, len);
    return dec;
}

extern "C" void redukt_rc_decoder_free(redukt_rc_decoder* dec) { delete dec; }

extern "C" int32_t redukt_rc_decode_symbol(redukt_rc_decoder* dec, const uint32_t* cdf, uint32_t n, uint32_t vocab,
                                           uint32_t* sym) {
    if (!dec || !cdf || !sym || n == 0) return REDUKT_CODEC_INVALID_ARG;
    return dec->decode(cdf, n, vocab, sym);
}
