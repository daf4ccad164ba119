// Range coder state machines and CDF builders shared by the C API (codec.cpp) and the
// lockstep driver (lockstep.cpp).  src/domain/coder.rs:118-296: u64 low with a carry
// cache and a run of pending 0xFF bytes, a 32-bit range renormalised byte-wise below
// 2^24, the last symbol of a CDF taking the remainder of the range.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <vector>

#include "redukt_codec.h"

namespace redukt_host {

// Frequencies -> cdf[n + 1] from f32 probabilities (freqs: n-element scratch).
int32_t cdf_from_probs_impl(const float* probs, uint32_t n, uint32_t* cdf, uint32_t* freqs);
// One logits row -> cdf[n + 1] (e, p, f: n-element scratch).
int32_t cdf_from_logits_impl(const float* logits, uint32_t n, uint32_t* cdf, double* e, float* p, uint32_t* f);
// Same with the calling thread's own scratch; 1 <= n < 2^24 is the caller's check.
void cdf_from_logits_row(const float* logits, uint32_t n, uint32_t* cdf);

constexpr uint32_t kRenorm = 1u << 24;  // range is kept >= 2^24 between symbols

}  // namespace redukt_host

struct redukt_rc_encoder {
    uint64_t low = 0;
    uint32_t range = 0xFFFFFFFFu;
    uint8_t cache = 0;
    uint64_t ff_run = 0;  // pending 0xFF bytes whose value waits on a carry
    bool first = true;    // the first shifted byte is a placeholder, never written
    bool finished = false;
    std::vector<uint8_t> out;

    // Emits the byte above bit 24 of low once its carry is known (coder.rs:140-160).
    void shift_low() {
        const uint32_t low32 = uint32_t(low);
        if (low32 < 0xFF000000u || (low >> 32) != 0) {
            const uint8_t carry = uint8_t(low >> 32);
            if (!first) out.push_back(uint8_t(cache + carry));
            first = false;
            out.insert(out.end(), ff_run, uint8_t(0xFF + carry));
            ff_run = 0;
            cache = uint8_t((low >> 24) & 0xFF);
        } else {
            ++ff_run;
        }
        low = (low & 0x00FFFFFFULL) << 8;
    }

    // Checked interval coding (coder.rs:163-177); INVALID_ARG for an empty or
    // out-of-total interval or a total the range cannot divide.
    int32_t encode(uint32_t lo, uint32_t hi, uint32_t total) {
        if (finished || total == 0 || lo >= hi || hi > total || range / total == 0) return REDUKT_CODEC_INVALID_ARG;
        const uint64_t r = range / total;
        low += uint64_t(lo) * r;
        range = hi < total ? uint32_t(r * uint64_t(hi - lo)) : range - uint32_t(r * uint64_t(lo));
        while (range < redukt_host::kRenorm) {
            shift_low();
            range <<= 8;
        }
        return REDUKT_CODEC_OK;
    }

    int32_t encode_symbol(uint32_t sym, const uint32_t* cdf, uint32_t n) {
        if (sym >= n) return REDUKT_CODEC_INVALID_ARG;
        return encode(cdf[sym], cdf[sym + 1], cdf[n]);
    }

    // coder.rs:185-196: five shifts push low out, then the cached byte and its run.
    void finish() {
        if (finished) return;
        for (int i = 0; i < 5; ++i) shift_low();
        if (!first) {
            out.push_back(cache);
            out.insert(out.end(), ff_run, uint8_t(0xFF));
        }
        finished = true;
    }

    size_t size() const { return finished ? out.size() : out.size() + (first ? 0 : 1) + size_t(ff_run); }
};

struct redukt_rc_decoder {
    uint32_t low = 0;
    uint32_t range = 0xFFFFFFFFu;
    uint32_t code = 0;
    std::vector<uint8_t> in;
    size_t pos = 0;

    uint8_t next_byte() { return pos < in.size() ? in[pos++] : uint8_t(0); }

    void start(const uint8_t* data, size_t len) {
        in.assign(data, data + len);
        pos = 0;
        low = 0;
        range = 0xFFFFFFFFu;
        code = 0;
        for (int i = 0; i < 4; ++i) code = (code << 8) | next_byte();
    }

    // get_freq (coder.rs:249-262): the cumulative frequency to look up in a CDF of this
    // total.  The state is unchanged.
    int32_t target(uint32_t total, uint32_t* cum) const {
        if (total == 0) return REDUKT_CODEC_INVALID_ARG;
        const uint32_t r = range / total;
        if (r == 0) return REDUKT_CODEC_RANGE_UNDERFLOW;
        *cum = std::min((code - low) / r, total - 1);
        return REDUKT_CODEC_OK;
    }

    // update (coder.rs:264-286) with the symbol s the lookup found for target()'s value
    // and its bounds lo = cdf[s], hi = cdf[s + 1] (read only when s < n), after target()
    // returned OK for this total; vocab > 0 also rejects symbols >= vocab after the update,
    // as decode_symbol_checked does.
    int32_t finish(uint32_t s, uint32_t lo, uint32_t hi, uint32_t total, uint32_t n, uint32_t vocab, uint32_t* sym) {
        if (s >= n) return REDUKT_CODEC_INVALID_ARG;  // cdf does not end at its total
        const uint32_t r = range / total;
        low += r * lo;
        range = hi < total ? r * (hi - lo) : range - r * lo;
        while (range < redukt_host::kRenorm) {
            code = (code << 8) | next_byte();
            low <<= 8;
            range <<= 8;
        }
        if (vocab && s >= vocab) return REDUKT_CODEC_SYMBOL_OUT_OF_RANGE;
        *sym = s;
        return REDUKT_CODEC_OK;
    }

    // get_freq + lookup + update (coder.rs:249-286).
    int32_t decode(const uint32_t* cdf, uint32_t n, uint32_t vocab, uint32_t* sym) {
        const uint32_t total = cdf[n];
        uint32_t cum = 0;
        const int32_t st = target(total, &cum);
        if (st != REDUKT_CODEC_OK) return st;
        const uint32_t s = redukt_cdf_lookup(cdf, n, cum);
        return s < n ? finish(s, cdf[s], cdf[s + 1], total, n, vocab, sym) : REDUKT_CODEC_INVALID_ARG;
    }
};
