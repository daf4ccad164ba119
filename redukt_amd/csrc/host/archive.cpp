// RDKT container: CRC-32 and the v2-v5 header reader / v5 writer (src/application/codec.rs,
// src/domain/crc32.rs).  Field order, flag bits and every rejection follow the reference
// reader so an archive is accepted or refused identically by both.
#include "redukt_archive.h"

#include <array>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#include "redukt_codec.h"

namespace {

// Byte-wise table of the reflected IEEE polynomial.
constexpr std::array<uint32_t, 256> crc_table() {
    std::array<uint32_t, 256> t{};
    for (uint32_t i = 0; i < 256; ++i) {
        uint32_t c = i;
        for (int k = 0; k < 8; ++k) c = (c & 1u) ? (c >> 1) ^ 0xEDB88320u : c >> 1;
        t[i] = c;
    }
    return t;
}
constexpr std::array<uint32_t, 256> kCrc = crc_table();

constexpr uint8_t kFlagCustomHp = 0x01, kFlagEmb = 0x02, kFlagE8e9 = 0x04, kFlagShuffle = 0x08,
                  kFlagDelta = 0x10, kFlagSkip = 0x20, kFlagBackbone = 0x40, kFlagEnhancedCm = 0x80;
constexpr uint8_t kProfileQuantMask = 0x0F, kProfileContractMask = 0x30, kProfileResetFlag = 0x40;
constexpr size_t kV23Header = 28, kV4Base = 13, kV5Base = 14;
constexpr uint8_t kResetMin = 8, kResetMax = 20;
constexpr float kDefaultBiasLr = 0.30f, kDefaultNgramScale = 0.50f, kDefaultMixEta = 0.01f;

int32_t fail(char* err, size_t cap, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int32_t fail(char* err, size_t cap, const char* fmt, ...) {
    if (err && cap) {
        va_list ap;
        va_start(ap, fmt);
        std::vsnprintf(err, cap, fmt, ap);
        va_end(ap);
    }
    return REDUKT_CODEC_INVALID_ARG;
}

uint32_t rd_u32(const uint8_t* p) { return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24; }
float rd_f32(const uint8_t* p) {
    const uint32_t b = rd_u32(p);
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}
uint32_t f32_bits(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}
void put_u32(std::vector<uint8_t>& v, uint32_t x) {
    for (int i = 0; i < 4; ++i) v.push_back(uint8_t(x >> (8 * i)));
}

bool mamba_family(uint8_t backbone) {
    return backbone == REDUKT_RDKT_BACKBONE_MAMBA || backbone == REDUKT_RDKT_BACKBONE_MAMBA_BYTE;
}

// check_contract_backbone (codec.rs:448-457): fma-v1 exists for the Mamba family only.
int32_t check_contract(uint8_t contract, uint8_t backbone, char* err, size_t cap) {
    if (contract == 2 && !mamba_family(backbone))
        return fail(err, cap,
                    "archive asks for numeric contract 2 (fma-v1), which only Mamba backbones have; "
                    "backbone byte is %u",
                    backbone);
    return REDUKT_CODEC_OK;
}

// parse_profile_byte (codec.rs:216-243).
int32_t parse_profile(uint8_t b, uint8_t* quant, uint8_t* contract, char* err, size_t cap) {
    if (b & ~(kProfileQuantMask | kProfileContractMask | kProfileResetFlag))
        return fail(err, cap, "archive PROFILE byte 0x%02X uses reserved bits", b);
    const uint8_t c = (b & kProfileContractMask) >> 4;
    if (c > 2)
        return fail(err, cap, "archive numeric contract %u is unknown here (this reader knows 0 legacy libm, "
                    "1 fmath-v1, 2 fma-v1)", c);
    const uint8_t q = b & kProfileQuantMask;
    if (q > 1)
        return fail(err, cap, "archive weight profile code %u (%s) has no decoder here", q,
                    q == 2 ? "Q6 (reserved)" : "unknown");
    *quant = q;
    *contract = c;
    return REDUKT_CODEC_OK;
}

void defaults(redukt_rdkt_header* h) {
    std::memset(h, 0, sizeof *h);
    h->bias_lr = kDefaultBiasLr;
    h->ngram_scale = kDefaultNgramScale;
    h->mix_eta = kDefaultMixEta;
}

}  // namespace

extern "C" uint32_t redukt_crc32_update(uint32_t state, const uint8_t* data, size_t len) {
    for (size_t i = 0; i < len; ++i) state = (state >> 8) ^ kCrc[(state ^ data[i]) & 0xFFu];
    return state;
}

extern "C" uint32_t redukt_crc32(const uint8_t* data, size_t len) {
    return redukt_crc32_update(REDUKT_CRC32_INIT, data, len) ^ 0xFFFFFFFFu;
}

extern "C" void redukt_rdkt_default_header(redukt_rdkt_header* h, uint32_t total_bytes, uint8_t backbone,
                                           uint8_t quant, uint8_t reset_log2) {
    if (!h) return;
    defaults(h);
    h->version = 5;
    h->has_crc = 1;
    h->total_bytes = total_bytes;
    h->backbone = backbone;
    // resolve_compress_profile (codec.rs:706-717): only the Mamba family records a weight
    // profile; RWKV and the GPU plugin always write F32, whatever their own quantisation.
    h->quant = mamba_family(backbone) ? quant : 0;
    h->contract = 1;  // fmath-v1: the exp of every CDF (NumericContract::CURRENT)
    // resolve_reset_log2 (codec.rs:140-147, 694-703): RWKV never resets.
    h->reset_log2 = backbone == REDUKT_RDKT_BACKBONE_RWKV ? 0 : reset_log2;
}

extern "C" int32_t redukt_rdkt_build_header(const redukt_rdkt_header* h, uint8_t* out, size_t cap, size_t* len,
                                            char* err, size_t err_cap) {
    // build_v4_header + set_v5_profile (codec.rs:581-665).
    if (!h || !len) return fail(err, err_cap, "null argument");
    if (h->quant > 1) return fail(err, err_cap, "unknown quant code %u", h->quant);
    if (h->contract > 2) return fail(err, err_cap, "unknown numeric contract %u", h->contract);
    if (h->backbone > REDUKT_RDKT_BACKBONE_PLUGIN) return fail(err, err_cap, "unknown backbone %u", h->backbone);
    if (h->reset_log2 && (h->reset_log2 < kResetMin || h->reset_log2 > kResetMax))
        return fail(err, err_cap, "reset period exponent %u lies outside %u..%u", h->reset_log2, kResetMin,
                    kResetMax);
    if (h->emb_method > 3) return fail(err, err_cap, "unknown emb-surgery method %u", h->emb_method);
    if (int32_t rc = check_contract(h->contract, h->backbone, err, err_cap)) return rc;
    if (h->quant && !mamba_family(h->backbone))
        return fail(err, err_cap,
                    "backbone %u records no weight profile (only the Mamba family does); its archives carry F32",
                    h->backbone);
    if (h->reset_log2 && h->backbone == REDUKT_RDKT_BACKBONE_RWKV)
        return fail(err, err_cap, "RWKV archives carry no reset period (RWKV never resets its state)");

    const bool custom_hp = f32_bits(h->bias_lr) != f32_bits(kDefaultBiasLr) ||
                           f32_bits(h->ngram_scale) != f32_bits(kDefaultNgramScale) ||
                           f32_bits(h->mix_eta) != f32_bits(kDefaultMixEta);
    const bool has_emb = h->emb_method != 0, has_shuffle = h->shuffle_stride > 1, has_delta = h->delta_stride > 0,
               has_skip = h->skip_threshold > 0, has_backbone = h->backbone != REDUKT_RDKT_BACKBONE_RWKV;
    uint8_t flags = 0;
    if (custom_hp) flags |= kFlagCustomHp;
    if (has_emb) flags |= kFlagEmb;
    if (h->e8e9) flags |= kFlagE8e9;
    if (has_shuffle) flags |= kFlagShuffle;
    if (has_delta) flags |= kFlagDelta;
    if (has_skip) flags |= kFlagSkip;
    if (has_backbone) flags |= kFlagBackbone;
    if (h->enhanced_cm) flags |= kFlagEnhancedCm;

    std::vector<uint8_t> v;
    v.reserve(40);
    const uint8_t magic[8] = {'R', 'D', 'K', 'T', 5, 0, 0, 0};
    v.insert(v.end(), magic, magic + 8);
    put_u32(v, h->total_bytes);
    v.push_back(flags);
    v.push_back(uint8_t(h->quant | h->contract << 4 | (h->reset_log2 ? kProfileResetFlag : 0)));
    if (h->reset_log2) v.push_back(h->reset_log2);
    if (custom_hp) {
        put_u32(v, f32_bits(h->bias_lr));
        put_u32(v, f32_bits(h->ngram_scale));
        put_u32(v, f32_bits(h->mix_eta));
    }
    if (has_emb) {
        v.push_back(h->emb_method);
        put_u32(v, f32_bits(h->emb_alpha));
    }
    if (has_shuffle) v.push_back(h->shuffle_stride);
    if (has_delta) v.push_back(h->delta_stride);
    if (has_skip) v.push_back(h->skip_threshold);
    if (has_backbone) v.push_back(h->backbone);
    *len = v.size();
    if (!out || cap < v.size()) return REDUKT_CODEC_BUFFER_TOO_SMALL;
    std::memcpy(out, v.data(), v.size());
    return REDUKT_CODEC_OK;
}

extern "C" int32_t redukt_rdkt_validate_magic(const uint8_t* data, size_t len, uint8_t* version, char* err,
                                              size_t err_cap) {
    // codec.rs:177-210.
    if (!data && len) return fail(err, err_cap, "null data");
    if (len < 8) return fail(err, err_cap, "%zu bytes cannot hold an archive header", len);
    const bool legacy = std::memcmp(data, "AZTH", 4) == 0;
    if (!legacy && std::memcmp(data, "RDKT", 4) != 0)
        return fail(err, err_cap, "not an archive: the first four bytes are neither RDKT nor AZTH");
    const uint8_t ver = data[4];
    if (!legacy && ver < 5)
        return fail(err, err_cap, "RDKT archives begin at version 5; version %u "
                    "is only valid under the legacy AZTH magic", ver);
    size_t min_size;
    switch (ver) {
        case 2:
        case 3: min_size = kV23Header; break;
        case 4: min_size = kV4Base; break;
        case 5: min_size = kV5Base; break;
        default: return fail(err, err_cap, "archive version %u is not one of 2, 3, 4, 5", ver);
    }
    if (len < min_size)
        return fail(err, err_cap, "version-%u header needs more bytes than the %zu given (at least %zu)", ver, len,
                    min_size);
    if (version) *version = ver;
    return REDUKT_CODEC_OK;
}

extern "C" int32_t redukt_rdkt_parse_header(const uint8_t* data, size_t len, redukt_rdkt_header* h, char* err,
                                            size_t err_cap) {
    // codec.rs:250-440.
    if (!h) return fail(err, err_cap, "null header");
    uint8_t ver = 0;
    if (int32_t rc = redukt_rdkt_validate_magic(data, len, &ver, err, err_cap)) return rc;
    redukt_rdkt_header r;
    defaults(&r);
    r.version = ver;
    r.legacy_magic = std::memcmp(data, "AZTH", 4) == 0;
    r.has_crc = ver >= 3;
    r.total_bytes = rd_u32(data + 8);
    if (ver <= 3) {
        r.has_token_count = 1;
        r.token_count = rd_u32(data + 12);
        const float hp[3] = {rd_f32(data + 16), rd_f32(data + 20), rd_f32(data + 24)};
        for (float x : hp)
            if (!std::isfinite(x)) return fail(err, err_cap, "archive hyperparameter is not finite");
        r.bias_lr = hp[0];
        r.ngram_scale = hp[1];
        r.mix_eta = hp[2];
        r.backbone = REDUKT_RDKT_BACKBONE_RWKV;
        r.header_size = uint32_t(kV23Header);
        *h = r;
        return REDUKT_CODEC_OK;
    }
    const uint8_t flags = data[12];  // all eight bits are defined
    size_t off = kV4Base;
    if (ver == 5) {
        if (int32_t rc = parse_profile(data[13], &r.quant, &r.contract, err, err_cap)) return rc;
        off = kV5Base;
        if (data[13] & kProfileResetFlag) {
            if (len < off + 1)
                return fail(err, err_cap, "archive ends inside its reset-period byte (%zu bytes, %zu needed)", len,
                            off + 1);
            const uint8_t l = data[off];
            if (l < kResetMin || l > kResetMax)
                return fail(err, err_cap, "archive reset period exponent %u lies outside %u..%u", l, kResetMin,
                            kResetMax);
            r.reset_log2 = l;
            off += 1;
        }
    }
    auto need = [&](size_t n, const char* what) {
        if (len < off + n)
            return fail(err, err_cap, "version-%u archive ends inside its %s (%zu bytes, %zu needed)", ver, what, len,
                        off + n);
        return int32_t(REDUKT_CODEC_OK);
    };
    if (flags & kFlagCustomHp) {
        if (int32_t rc = need(12, "custom HP")) return rc;
        const float hp[3] = {rd_f32(data + off), rd_f32(data + off + 4), rd_f32(data + off + 8)};
        for (float x : hp)
            if (!std::isfinite(x)) return fail(err, err_cap, "archive hyperparameter is not finite");
        r.bias_lr = hp[0];
        r.ngram_scale = hp[1];
        r.mix_eta = hp[2];
        off += 12;
    }
    if (flags & kFlagEmb) {
        if (int32_t rc = need(5, "emb-surgery")) return rc;
        r.emb_method = data[off];
        r.emb_alpha = rd_f32(data + off + 1);
        off += 5;
    }
    r.e8e9 = (flags & kFlagE8e9) != 0;
    if (flags & kFlagShuffle) {
        if (int32_t rc = need(1, "shuffle")) return rc;
        r.shuffle_stride = data[off++];
    }
    if (flags & kFlagDelta) {
        if (int32_t rc = need(1, "delta")) return rc;
        r.delta_stride = data[off++];
    }
    if (flags & kFlagSkip) {
        if (int32_t rc = need(1, "adaptive-skip")) return rc;
        r.skip_threshold = data[off++];
    }
    r.backbone = REDUKT_RDKT_BACKBONE_RWKV;
    if (flags & kFlagBackbone) {
        if (int32_t rc = need(1, "backbone")) return rc;
        const uint8_t b = data[off++];
        if (b > REDUKT_RDKT_BACKBONE_PLUGIN)
            return fail(err, err_cap, "version-%u archive names backbone %u, which this reader does not know", ver, b);
        r.backbone = b;
    }
    r.enhanced_cm = (flags & kFlagEnhancedCm) != 0;
    if (int32_t rc = check_contract(r.contract, r.backbone, err, err_cap)) return rc;
    r.header_size = uint32_t(off);
    *h = r;
    return REDUKT_CODEC_OK;
}

extern "C" int32_t redukt_rdkt_split(const uint8_t* data, size_t len, uint32_t header_size, uint8_t version,
                                     size_t* stream_off, size_t* stream_len, uint32_t* crc, uint8_t* has_crc) {
    // extract_stream_and_crc_v (codec.rs:540-560).
    if (!stream_off || !stream_len || (!data && len)) return REDUKT_CODEC_INVALID_ARG;
    if (len < header_size) return REDUKT_CODEC_INVALID_ARG;  // truncated: the header alone does not fit
    const size_t payload = len - header_size;
    *stream_off = header_size;
    if (version < 3) {
        *stream_len = payload;
        if (has_crc) *has_crc = 0;
        return REDUKT_CODEC_OK;
    }
    if (payload < 4) return REDUKT_CODEC_INVALID_ARG;  // no room for the CRC-32
    *stream_len = payload - 4;
    if (crc) *crc = rd_u32(data + len - 4);
    if (has_crc) *has_crc = 1;
    return REDUKT_CODEC_OK;
}

extern "C" int32_t redukt_rdkt_decode_profile(const redukt_rdkt_header* h, uint8_t* quant, char* err, size_t err_cap) {
    // resolve_decompress_profile with no --quant override (codec.rs:719-741).
    if (!h) return fail(err, err_cap, "null header");
    if (!mamba_family(h->backbone) && h->quant != 0)
        return fail(err, err_cap,
                    "version-%u archive gives backbone %u the weight profile %s; only Mamba backbones carry a "
                    "profile other than F32",
                    h->version, h->backbone, h->quant == 1 ? "Q8" : "?");
    if (quant) *quant = h->quant;
    return REDUKT_CODEC_OK;
}
