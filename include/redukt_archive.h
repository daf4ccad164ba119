/* RDKT archive container: header writer / reader and CRC-32, byte-compatible with the
 * reference host (src/application/codec.rs:16-68 constants, 177-243 validate_magic and
 * the PROFILE byte, 250-440 parse_header, 540-560 extract_stream_and_crc_v, 581-680
 * build_v4_header / build_header_with; src/domain/crc32.rs).
 *
 * File layout (v3+):  HEADER | STREAM (range-coded tokens) | CRC-32 of the original
 * bytes, little-endian.  The writer always emits v5 with the "RDKT" magic:
 *
 *   0  "RDKT" 05 00 00 00      magic + version
 *   8  u32 TOTAL_BYTES         original length
 *  12  u8  FLAGS               0x01 custom HP, 0x02 emb surgery, 0x04 E8E9, 0x08 shuffle,
 *                              0x10 delta, 0x20 adaptive skip, 0x40 backbone, 0x80 enhanced CM
 *  13  u8  PROFILE             bits 0-3 quant (0 F32, 1 Q8), bits 4-5 numeric contract
 *                              (0 legacy libm, 1 fmath-v1, 2 fma-v1), bit 6 RESET_LOG2 follows
 *  [u8 RESET_LOG2] [3 x f32 HP] [u8 method + f32 alpha] [u8 shuffle] [u8 delta] [u8 skip]
 *  [u8 BACKBONE: 0 RWKV, 1 Mamba, 2 MambaByte, 3 GPU plugin]      (each only when flagged)
 *
 * The reader also accepts the legacy "AZTH" magic (v2-v5); v2/v3 carry a 28-byte header
 * with a token count and the three hyperparameters, v2 has no CRC.
 */
#ifndef REDUKT_ARCHIVE_H
#define REDUKT_ARCHIVE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define REDUKT_RDKT_BACKBONE_RWKV 0u
#define REDUKT_RDKT_BACKBONE_MAMBA 1u
#define REDUKT_RDKT_BACKBONE_MAMBA_BYTE 2u
#define REDUKT_RDKT_BACKBONE_PLUGIN 3u
#define REDUKT_RDKT_DEFAULT_RESET_LOG2 12u /* 4096 forwards, codec.rs:42 */

typedef struct {
    uint8_t version;         /* 2..5 (parse); the writer always writes 5 */
    uint8_t legacy_magic;    /* 1 = "AZTH" (read only) */
    uint8_t has_token_count; /* v2/v3 */
    uint8_t has_crc;         /* v3+ */
    uint32_t total_bytes;
    uint32_t token_count;
    float bias_lr, ngram_scale, mix_eta; /* defaults 0.30 / 0.50 / 0.01 */
    uint8_t emb_method;                  /* 0 none, 1 center, 2 norm, 3 spread */
    float emb_alpha;
    uint8_t e8e9;
    uint8_t shuffle_stride; /* 0 or 1 = none */
    uint8_t delta_stride;   /* 0 = none */
    uint8_t skip_threshold; /* 0 = none */
    uint8_t backbone;       /* REDUKT_RDKT_BACKBONE_* */
    uint8_t enhanced_cm;
    uint8_t quant;          /* 0 F32, 1 Q8 */
    uint8_t contract;       /* 0 legacy libm, 1 fmath-v1, 2 fma-v1 (Mamba family only) */
    uint8_t reset_log2;     /* 0 = never, else 8..20 */
    uint32_t header_size;   /* parse: bytes of the header */
} redukt_rdkt_header;

/* CRC-32 (IEEE 802.3, reflected 0xEDB88320): crc32 = finalize(update(INIT, data)). */
#define REDUKT_CRC32_INIT 0xFFFFFFFFu
uint32_t redukt_crc32_update(uint32_t state, const uint8_t* data, size_t len);
uint32_t redukt_crc32(const uint8_t* data, size_t len);

/* Fills *h with the reference writer's defaults: v5, fmath-v1, default hyperparameters,
 * no preprocessing, the given backbone, quant and reset period, resolved as the reference
 * compressor resolves them (codec.rs:140-147, 694-717): quant is kept for the Mamba family
 * only (RWKV and the GPU plugin write F32: a plugin's own quantisation is part of its
 * configuration, not of the archive), and RWKV gets no reset period. */
void redukt_rdkt_default_header(redukt_rdkt_header* h, uint32_t total_bytes, uint8_t backbone, uint8_t quant,
                                uint8_t reset_log2);

/* Writes the v5 header of *h into out (capacity cap); *len receives its size (also when
 * it does not fit, with REDUKT_CODEC_BUFFER_TOO_SMALL).  INVALID_ARG, with a message in
 * err, for an unknown quant / contract / backbone, a RESET_LOG2 outside 8..20, the
 * fma-v1 contract on a backbone outside the Mamba family, a non-F32 quant outside the
 * Mamba family, or a reset period on RWKV: headers the reference decoder would refuse or
 * that its compressor never writes. */
int32_t redukt_rdkt_build_header(const redukt_rdkt_header* h, uint8_t* out, size_t cap, size_t* len, char* err,
                                 size_t err_cap);

/* Checks the magic and the minimum size (validate_magic); *version receives 2..5. */
int32_t redukt_rdkt_validate_magic(const uint8_t* data, size_t len, uint8_t* version, char* err, size_t err_cap);

/* validate_magic + parse_header: every reference rejection (reserved flag or PROFILE
 * bits, unknown contract / quant / backbone, RESET_LOG2 out of range, truncated fields,
 * non-finite hyperparameters) returns INVALID_ARG with the reason in err. */
int32_t redukt_rdkt_parse_header(const uint8_t* data, size_t len, redukt_rdkt_header* h, char* err,
                                 size_t err_cap);

/* resolve_decompress_profile (codec.rs:719-741) without a --quant override: the weight
 * profile a decoder takes from the header.  INVALID_ARG for a non-F32 profile on any
 * backbone outside the Mamba family (RWKV, the GPU plugin), as the reference refuses it
 * ("only Mamba supports profiles"); else *quant receives the header's quant. */
int32_t redukt_rdkt_decode_profile(const redukt_rdkt_header* h, uint8_t* quant, char* err, size_t err_cap);

/* extract_stream_and_crc_v: the stream is data[*stream_off .. *stream_off + *stream_len);
 * for v3+ the trailing 4 bytes are the stored CRC (*has_crc = 1). */
int32_t redukt_rdkt_split(const uint8_t* data, size_t len, uint32_t header_size, uint8_t version,
                          size_t* stream_off, size_t* stream_len, uint32_t* crc, uint8_t* has_crc);

#ifdef __cplusplus
}
#endif
#endif /* REDUKT_ARCHIVE_H */
