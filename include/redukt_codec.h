/* Host-side coding path of redukt: logits -> quantized CDF -> range coder, and back.
 *
 * This is the CPU half of compress/decompress that sits on top of the GPU backend
 * (redukt_backend.h): each step the backend returns one row of logits per stream; the
 * host turns every row into a 2^24-total CDF and codes that stream's next token with it.
 * Every function here is bit-compatible with the reference host, so archives and CDFs
 * are interchangeable with it:
 *
 *   redukt_exp_f64            src/domain/fmath.rs:340-430   (exp_f64 + its special cases)
 *   redukt_cdf_from_logits    src/application/codec.rs:785-798 (cdf_from_logits_with, fmath-v1)
 *   redukt_cdf_from_probs     src/domain/coder.rs:43-81      (Cdf::from_probs)
 *   redukt_cdf_uniform        src/domain/coder.rs:83-93      (Cdf::uniform)
 *   redukt_cdf_lookup         src/domain/coder.rs:100-115    (Cdf::lookup)
 *   redukt_rc_encoder_*       src/domain/coder.rs:118-204    (RangeEncoder)
 *   redukt_rc_decoder_*       src/domain/coder.rs:206-296    (RangeDecoder)
 *
 * CDF layout: uint32_t cdf[n + 1], cdf[0] = 0, cdf[i + 1] - cdf[i] = frequency of symbol
 * i (>= 1), cdf[n] = total (2^24 for the probability-built CDFs, floor(2^24/n)*n for the
 * uniform one).  The total is always read from cdf[n].
 *
 * Threading: encoders and decoders are independent objects; one object must not be used
 * from two threads at once.  redukt_cdf_from_logits_batch runs rows on a pool of host
 * threads; a row's result does not depend on the thread count.
 */
#ifndef REDUKT_CODEC_H
#define REDUKT_CODEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    REDUKT_CODEC_OK = 0,
    REDUKT_CODEC_INVALID_ARG = 1,
    /* range / total == 0 in the decoder: corrupted stream or CDF mismatch
     * (DecodeError::RangeUnderflow, coder.rs:17-18) */
    REDUKT_CODEC_RANGE_UNDERFLOW = 2,
    /* decoded symbol >= vocab (DecodeError::SymbolOutOfRange, coder.rs:19-20) */
    REDUKT_CODEC_SYMBOL_OUT_OF_RANGE = 3,
    REDUKT_CODEC_BUFFER_TOO_SMALL = 4,
    /* the file was not finished: the backbone failed (forward / reset) while it was in
     * flight or before it was admitted; its output is not valid (length 0) */
    REDUKT_CODEC_INCOMPLETE = 5,
} redukt_codec_status;

/* Cumulative total of every probability-built CDF (coder.rs:12). */
#define REDUKT_CDF_TOTAL (1u << 24)

/* e^x, correctly rounded except within 0.52 ulp; the exact double of the reference's
 * portable exp for every input (including subnormal results, +-inf and NaN). */
double redukt_exp_f64(double x);

/* CDF from a probability vector (need not be normalised; negative or NaN entries are the
 * caller's problem exactly as in the reference).  Requires 1 <= n < 2^24. */
int32_t redukt_cdf_from_probs(const float* probs, uint32_t n, uint32_t* cdf);

/* Uniform CDF over n symbols (the first token of every stream is coded with it). */
int32_t redukt_cdf_uniform(uint32_t n, uint32_t* cdf);

/* f64 softmax of one logits row with redukt_exp_f64, rounded to f32 probabilities, then
 * redukt_cdf_from_probs.  Requires 1 <= n < 2^24. */
int32_t redukt_cdf_from_logits(const float* logits, uint32_t n, uint32_t* cdf);

/* rows independent redukt_cdf_from_logits calls: logits [rows x n] -> cdf [rows x (n+1)].
 * threads = 0 uses every host thread.  Bit-identical to calling the row function. */
int32_t redukt_cdf_from_logits_batch(const float* logits, uint32_t rows, uint32_t n, uint32_t* cdf,
                                     uint32_t threads);

/* Symbol whose interval [cdf[s], cdf[s+1]) holds cum_freq (binary search). */
uint32_t redukt_cdf_lookup(const uint32_t* cdf, uint32_t n, uint32_t cum_freq);

/* ---- range encoder ---------------------------------------------------------------- */
typedef struct redukt_rc_encoder redukt_rc_encoder;

redukt_rc_encoder* redukt_rc_encoder_new(void);
void redukt_rc_encoder_free(redukt_rc_encoder* enc);
/* Codes the interval [lo, hi) of total (RangeEncoder::encode). */
int32_t redukt_rc_encode(redukt_rc_encoder* enc, uint32_t lo, uint32_t hi, uint32_t total);
/* Codes symbol sym < n with cdf[n + 1] (RangeEncoder::encode_symbol). */
int32_t redukt_rc_encode_symbol(redukt_rc_encoder* enc, uint32_t sym, const uint32_t* cdf, uint32_t n);
/* Bytes the stream would have if finished now (RangeEncoder::size). */
size_t redukt_rc_encoder_size(const redukt_rc_encoder* enc);
/* Flushes and returns the stream length; copies min(len, cap) bytes to out (out may be
 * NULL with cap 0 to ask the length).  The encoder is left finished: a second call
 * returns the same bytes; further encode calls return INVALID_ARG. */
size_t redukt_rc_finish(redukt_rc_encoder* enc, uint8_t* out, size_t cap);

/* ---- range decoder ---------------------------------------------------------------- */
typedef struct redukt_rc_decoder redukt_rc_decoder;

/* Copies data[0..len); bytes past the end read as zero (RangeDecoder::next_byte). */
redukt_rc_decoder* redukt_rc_decoder_new(const uint8_t* data, size_t len);
void redukt_rc_decoder_free(redukt_rc_decoder* dec);
/* Decodes one symbol of cdf[n + 1]; *sym is written on OK.  vocab > 0 additionally
 * rejects symbols >= vocab with SYMBOL_OUT_OF_RANGE after the state update, as
 * RangeDecoder::decode_symbol_checked does; vocab = 0 skips that check. */
int32_t redukt_rc_decode_symbol(redukt_rc_decoder* dec, const uint32_t* cdf, uint32_t n, uint32_t vocab,
                                uint32_t* sym);

#ifdef __cplusplus
}
#endif
#endif /* REDUKT_CODEC_H */
