"""RDKT container (libredukt_host.so) against the reference's own header and CRC tests
(src/application/codec.rs:2250-2600, 2700-2860, 2890-3190; src/domain/crc32.rs tests)
and the plugin archive layout of docs FORMAT-SPEC.md:224-226 (BACKBONE 3, PROFILE 0x50,
RESET_LOG2 12).  Legacy files are built byte by byte here, as the reference's test helpers
build them."""
import struct

import numpy as np
import pytest

from redukt_amd import archive as A

MAGIC_V4 = b"AZTH\x04\x00\x00\x00"
MAGIC_V5 = b"RDKT\x05\x00\x00\x00"


def f32(x):
    return struct.pack("<f", x)


def make_v2(total, tokens, stream):
    return b"AZTH\x02\x00\x00\x00" + struct.pack("<II", total, tokens) + f32(0.30) + f32(0.50) + f32(0.01) + stream


def make_v3(total, tokens, stream, crc):
    return (b"AZTH\x03\x00\x00\x00" + struct.pack("<II", total, tokens) + f32(0.30) + f32(0.50) + f32(0.01) + stream
            + struct.pack("<I", crc))


def make_v4_default(total, stream, crc):
    return MAGIC_V4 + struct.pack("<I", total) + b"\x00" + stream + struct.pack("<I", crc)


def make_v4_custom(total, lr, scale, eta, stream, crc):
    return MAGIC_V4 + struct.pack("<I", total) + b"\x01" + f32(lr) + f32(scale) + f32(eta) + stream + struct.pack("<I", crc)


def with_payload(hdr):
    return hdr + b"\xab" * 16 + struct.pack("<I", 0xDEADBEEF)


def v4_layout(total, lr, scale, eta, emb, alpha, e8e9, shuffle, delta, skip, backbone, enhanced):
    """The v4 field order of build_v4_header (codec.rs:581-631), written out by hand."""
    custom = struct.pack("<fff", lr, scale, eta) != struct.pack("<fff", 0.30, 0.50, 0.01)
    flags = ((0x01 if custom else 0) | (0x02 if emb else 0) | (0x04 if e8e9 else 0) | (0x08 if shuffle > 1 else 0)
             | (0x10 if delta else 0) | (0x20 if skip else 0) | (0x40 if backbone != 0 else 0)
             | (0x80 if enhanced else 0))
    b = MAGIC_V4 + struct.pack("<I", total) + bytes([flags])
    if custom:
        b += struct.pack("<fff", lr, scale, eta)
    if emb:
        b += bytes([emb]) + f32(alpha)
    if shuffle > 1:
        b += bytes([shuffle])
    if delta:
        b += bytes([delta])
    if skip:
        b += bytes([skip])
    if backbone != 0:
        b += bytes([backbone])
    return b


def all_fields(quant, reset_log2=0, contract=1):
    return A.Header(total_bytes=4321, bias_lr=0.25, ngram_scale=0.6, mix_eta=0.02, emb_method=1, emb_alpha=0.3,
                    e8e9=True, shuffle_stride=4, delta_stride=1, skip_threshold=50, backbone=A.BACKBONE_MAMBA,
                    enhanced_cm=True, quant=quant, contract=contract, reset_log2=reset_log2)


# ---- CRC-32 (crc32.rs tests) ---------------------------------------------------------------

def test_crc32_known_vectors():
    assert A.crc32(b"123456789") == 0xCBF43926
    assert A.crc32(b"") == 0
    assert A.crc32(b"a") == 0xE8B7BE43


def test_crc32_incremental_and_against_zlib():
    import zlib

    data = np.random.default_rng(0).integers(0, 256, 10000, dtype=np.uint8).tobytes()
    s = 0xFFFFFFFF
    for i in range(0, len(data), 777):
        s = A.crc32(data[i:i + 777], s)
    assert s ^ 0xFFFFFFFF == A.crc32(data) == zlib.crc32(data)


# ---- validate_magic (codec.rs:2313-2386) ---------------------------------------------------

def test_validate_magic_versions():
    assert A.validate_magic(make_v2(100, 10, bytes(16))) == 2
    assert A.validate_magic(make_v3(100, 10, bytes(16), 0)) == 3
    assert A.validate_magic(make_v4_default(100, bytes(16), 0)) == 4
    assert A.validate_magic(make_v4_custom(100, 0.5, 0.5, 0.5, bytes(8), 0)) == 4
    with pytest.raises(A.ArchiveError):
        A.validate_magic(bytes(7))
    with pytest.raises(A.ArchiveError):
        A.validate_magic(MAGIC_V4 + bytes(4))  # 12 bytes: v4 needs 13
    with pytest.raises(A.ArchiveError):
        A.validate_magic(b"NOPE" + bytes(28))
    bad = bytearray(make_v3(100, 10, bytes(8), 0))
    bad[4] = 99
    with pytest.raises(A.ArchiveError):
        A.validate_magic(bytes(bad))


def test_validate_magic_rdkt_and_legacy():
    data = bytearray(32)
    data[:8] = MAGIC_V5
    assert A.validate_magic(bytes(data)) == 5
    data[:4] = b"AZTH"
    assert A.validate_magic(bytes(data)) == 5
    for v in (2, 3, 4):
        data[4] = v
        assert A.validate_magic(bytes(data)) == v
        data[:4] = b"RDKT"
        with pytest.raises(A.ArchiveError):
            A.validate_magic(bytes(data))
        data[:4] = b"AZTH"
    v5 = MAGIC_V5 + bytes(6)
    assert A.validate_magic(v5) == 5
    with pytest.raises(A.ArchiveError):
        A.validate_magic(v5[:13])


# ---- parse_header (codec.rs:2387-2453, 2735-2860) -----------------------------------------

def test_parse_header_legacy():
    h = A.parse_header(make_v3(500, 42, bytes(8), 0))
    assert (h.version, h.total_bytes, h.token_count, h.has_token_count, h.header_size) == (3, 500, 42, True, 28)
    assert abs(h.bias_lr - 0.30) < 1e-6 and h.backbone == A.BACKBONE_RWKV and h.legacy_magic
    h = A.parse_header(make_v4_default(1234, bytes(8), 0))
    assert (h.version, h.total_bytes, h.has_token_count, h.header_size) == (4, 1234, False, 13)
    assert f32(h.bias_lr) == f32(0.30) and f32(h.ngram_scale) == f32(0.50) and f32(h.mix_eta) == f32(0.01)
    assert (h.quant, h.contract) == (0, 0)  # v4: F32, legacy libm
    h = A.parse_header(make_v4_custom(999, 0.5, 0.7, 0.02, bytes(8), 0))
    assert (h.total_bytes, h.header_size) == (999, 25)
    assert abs(h.ngram_scale - 0.7) < 1e-6 and abs(h.mix_eta - 0.02) < 1e-6
    f = bytearray(make_v4_default(100, bytes(8), 0))
    f[12] = 0x80  # enhanced CM: every flag bit is known
    assert A.parse_header(bytes(f)).enhanced_cm


def test_parse_header_rejects_non_finite_hp():
    with pytest.raises(A.ArchiveError, match="not finite"):
        A.parse_header(make_v4_custom(100, float("nan"), 0.5, 0.01, b"", 0))
    f = bytearray(make_v3(100, 10, b"", 0))
    f[20:24] = f32(float("inf"))
    with pytest.raises(A.ArchiveError):
        A.parse_header(bytes(f))


# ---- the v5 writer (codec.rs:2455-2470, 2711-2730, 2890-3010, 3116-3190) -------------------

def test_header_is_v4_layout_plus_profile_byte():
    v4 = v4_layout(4321, 0.25, 0.6, 0.02, 1, 0.3, True, 4, 1, 50, A.BACKBONE_MAMBA, True)
    for quant, byte in ((0, 0x10), (1, 0x11)):
        v5 = A.build_header(all_fields(quant))
        assert v5[:8] == MAGIC_V5 and len(v5) == len(v4) + 1
        assert v5[8:13] == v4[8:13] and v5[13] == byte and v5[14:] == v4[13:]


def test_header_default_and_custom_sizes():
    h = A.build_header(A.Header(total_bytes=1000, backbone=A.BACKBONE_RWKV, reset_log2=0))
    assert len(h) == 14 and struct.unpack("<I", h[8:12])[0] == 1000 and h[12] == 0 and h[13] == 0x10
    h = A.build_header(A.Header(total_bytes=2000, bias_lr=0.5, ngram_scale=0.7, mix_eta=0.02,
                                backbone=A.BACKBONE_RWKV, reset_log2=0))
    assert len(h) == 26 and h[12] == 0x01 and abs(struct.unpack("<f", h[14:18])[0] - 0.5) < 1e-6
    h = A.build_header(A.Header(total_bytes=1000, emb_method=1, emb_alpha=0.3, backbone=A.BACKBONE_RWKV,
                                reset_log2=0))
    assert len(h) == 19 and h[12] == 0x02 and h[14] == 1
    h = A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_MAMBA, quant=1, reset_log2=0))
    assert len(h) == 15 and A.parse_header(with_payload(h)).backbone == A.BACKBONE_MAMBA


def test_reset_period_roundtrips_through_header():
    base = A.build_header(all_fields(1))
    with_ = A.build_header(all_fields(1, reset_log2=12))
    assert len(with_) == len(base) + 1 and with_[13] == 0x51 and with_[14] == 12 and with_[15:] == base[14:]
    h = A.parse_header(with_payload(with_))
    assert (h.reset_log2, h.reset_every, h.header_size) == (12, 4096, len(with_))
    assert (h.quant, h.contract) == (1, 1)
    assert A.parse_header(with_payload(base)).reset_every == 0


@pytest.mark.parametrize("bad", [0, 7, 21, 255])
def test_reset_log2_out_of_range_is_rejected(bad):
    h = bytearray(A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_MAMBA, reset_log2=12, enhanced_cm=True)))
    h[14] = bad
    with pytest.raises(A.ArchiveError, match="reset period exponent"):
        A.parse_header(with_payload(bytes(h)))
    if bad:  # 0 is "never" for the writer; the rest are refused there too
        with pytest.raises(A.ArchiveError, match="reset period exponent"):
            A.build_header(A.Header(total_bytes=10, reset_log2=bad))


def test_reset_flag_without_its_byte_is_truncated():
    h = bytearray(A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_RWKV, reset_log2=0, enhanced_cm=True)))
    h[13] |= 0x40
    with pytest.raises(A.ArchiveError, match="ends inside"):
        A.parse_header(bytes(h))


def test_numeric_contracts():
    assert A.parse_header(with_payload(A.build_header(all_fields(0)))).contract == 1
    v4 = A.parse_header(with_payload(v4_layout(4321, 0.25, 0.6, 0.02, 1, 0.3, True, 4, 1, 50, 1, True)))
    assert (v4.version, v4.contract) == (4, 0)
    r099 = bytearray(A.build_header(all_fields(1)))
    r099[13] = 0x01
    old = A.parse_header(with_payload(bytes(r099)))
    assert (old.quant, old.contract) == (1, 0)
    for byte in (0x31, 0x30):
        r099[13] = byte
        with pytest.raises(A.ArchiveError, match="numeric contract"):
            A.parse_header(with_payload(bytes(r099)))


def test_fma_contract_is_mamba_only():
    for quant, byte in ((0, 0x20), (1, 0x21)):
        h = A.build_header(all_fields(quant, contract=2))
        assert h[13] == byte and A.parse_header(with_payload(h)).contract == 2
    with pytest.raises(A.ArchiveError, match="only Mamba backbones"):
        A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_RWKV, contract=2, reset_log2=0))
    h = bytearray(A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_RWKV, reset_log2=0)))
    h[13] = 0x20
    with pytest.raises(A.ArchiveError, match="only Mamba backbones"):
        A.parse_header(with_payload(bytes(h)))


@pytest.mark.parametrize("byte,ok,quant,contract", [(0x00, True, 0, 0), (0x01, True, 1, 0), (0x10, True, 0, 1),
                                                    (0x11, True, 1, 1), (0x02, False, 0, 0), (0x07, False, 0, 0),
                                                    (0x22, False, 0, 0), (0x30, False, 0, 0), (0x81, False, 0, 0)])
def test_profile_byte(byte, ok, quant, contract):
    h = bytearray(A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_MAMBA, reset_log2=0)))
    h[13] = byte
    if ok:
        p = A.parse_header(with_payload(bytes(h)))
        assert (p.quant, p.contract) == (quant, contract)
    else:
        with pytest.raises(A.ArchiveError, match="Q6" if byte == 0x02 else "."):
            A.parse_header(with_payload(bytes(h)))


def test_profile_reset_bit_is_known():
    h = A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_MAMBA, quant=1, reset_log2=12))
    assert h[13] == 0x51 and A.parse_header(with_payload(h)).quant == 1


def test_all_fields_roundtrip_and_split():
    hdr = A.build_header(all_fields(1))
    f = with_payload(hdr)
    assert A.validate_magic(f) == 5
    h = A.parse_header(f)
    assert (h.version, h.quant, h.header_size, h.total_bytes) == (5, 1, len(hdr), 4321)
    assert (h.bias_lr, h.ngram_scale, h.mix_eta) == pytest.approx((0.25, 0.6, 0.02))
    assert h.e8e9 and h.enhanced_cm and (h.shuffle_stride, h.delta_stride, h.skip_threshold) == (4, 1, 50)
    assert h.emb_method == 1 and abs(h.emb_alpha - 0.3) < 1e-6 and h.backbone == A.BACKBONE_MAMBA
    stream, crc = A.split(f, h.header_size, h.version)
    assert stream == b"\xab" * 16 and crc == 0xDEADBEEF


# ---- extract_stream_and_crc_v (codec.rs:2480-2575) -----------------------------------------

def test_split_legacy_and_v4():
    assert A.split(make_v4_default(100, b"\xaa\xbb\xcc", 0xCAFEBABE), 13, 4) == (b"\xaa\xbb\xcc", 0xCAFEBABE)
    assert A.split(make_v4_custom(50, 0.5, 0.5, 0.5, b"\x11\x22", 0x12345678), 25, 4) == (b"\x11\x22", 0x12345678)
    short = bytes(13) + b"\x01\x02\x03"
    with pytest.raises(A.ArchiveError):
        A.split(short, 13, 4)
    with pytest.raises(A.ArchiveError):
        A.split(short[:5], 13, 4)
    assert A.split(short, 13, 2) == (b"\x01\x02\x03", None)
    assert A.split(make_v3(100, 10, b"\xaa\xbb\xcc\xdd\xee", 0xDEADBEEF), 28, 3) == (b"\xaa\xbb\xcc\xdd\xee", 0xDEADBEEF)
    assert A.split(make_v2(100, 10, b"\xaa\xbb\xcc"), 28, 2) == (b"\xaa\xbb\xcc", None)
    assert A.split(make_v3(0, 0, b"", 0x12345678), 28, 3) == (b"", 0x12345678)


def test_crc_detects_corruption():
    orig = b"Hello, Redukt!"
    f = make_v3(len(orig), 5, b"\xaa" * 20, A.crc32(orig))
    assert A.split(f, 28, 3)[1] != A.crc32(b"Hello, Redakt!")
    f = bytearray(make_v3(17, 3, b"\x55" * 10, A.crc32(b"test data for CRC")))
    f[28] ^= 1
    assert A.split(bytes(f), 28, 3)[1] == A.crc32(b"test data for CRC")


# ---- plugin archives (FORMAT-SPEC.md:224-226) ----------------------------------------------

def test_plugin_archive_defaults_and_pack():
    h = A.default_header(1234, A.BACKBONE_PLUGIN, 0, 12)
    raw = A.build_header(h)
    assert raw == MAGIC_V5 + struct.pack("<I", 1234) + bytes([0x40, 0x50, 12, 3])
    payload = b"some original bytes"
    file = A.pack(h, b"\x01\x02\x03", payload)
    hh, stream, crc = A.unpack(file)
    assert stream == b"\x01\x02\x03" and crc == A.crc32(payload)
    assert (hh.backbone, hh.quant, hh.contract, hh.reset_every, hh.header_size) == (3, 0, 1, 4096, len(raw))
    # resolve_compress_profile (codec.rs:706-717): the plugin's own int8 weights are part of
    # its configuration, not of the archive; asking for Q8 still writes PROFILE 0x50
    q8 = A.build_header(A.default_header(1, A.BACKBONE_PLUGIN, 1, 12))
    assert q8 == MAGIC_V5 + struct.pack("<I", 1) + bytes([0x40, 0x50, 12, 3])
    assert A.build_header(A.default_header(1, A.BACKBONE_PLUGIN, 0, 0))[13] == 0x10
    # RWKV: PROFILE 0x10, no reset byte, no backbone byte (FORMAT-SPEC.md:224-226)
    rw = A.build_header(A.default_header(77, A.BACKBONE_RWKV, 1, 12))
    assert rw == MAGIC_V5 + struct.pack("<I", 77) + bytes([0x00, 0x10])
    assert A.unpack(A.pack(A.default_header(77, A.BACKBONE_RWKV, 1, 12), b"", b"x"))[0].reset_every == 0
    # the Mamba family keeps its profile
    assert A.build_header(A.default_header(1, A.BACKBONE_MAMBA, 1, 12))[13] == 0x51


def test_writer_refuses_what_the_reference_never_writes():
    with pytest.raises(A.ArchiveError, match="no weight profile"):
        A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_PLUGIN, quant=1, reset_log2=12))
    with pytest.raises(A.ArchiveError, match="no weight profile"):
        A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_RWKV, quant=1, reset_log2=0))
    with pytest.raises(A.ArchiveError, match="no reset period"):
        A.build_header(A.Header(total_bytes=10, backbone=A.BACKBONE_RWKV, reset_log2=12))


@pytest.mark.parametrize("backbone,byte", [(A.BACKBONE_PLUGIN, 0x51), (A.BACKBONE_PLUGIN, 0x11),
                                           (A.BACKBONE_RWKV, 0x11), (A.BACKBONE_RWKV, 0x01)])
def test_non_f32_profile_outside_mamba_is_refused_on_decode(backbone, byte):
    """resolve_decompress_profile (codec.rs:719-741, test at :3202-3212): a Q8 PROFILE on the
    plugin or RWKV backbone parses but is refused before decoding."""
    reset = 12 if byte & 0x40 else 0
    h = bytearray(A.build_header(A.default_header(10, backbone, 0, reset)))
    h[13] = byte  # what a writer outside these rules would put there
    f = with_payload(bytes(h))
    hp = A.parse_header(f)  # the header itself is well formed
    assert (hp.backbone, hp.quant) == (backbone, 1)
    with pytest.raises(A.ArchiveError, match="only Mamba backbones carry a profile"):
        A.decode_profile(hp)
    with pytest.raises(A.ArchiveError, match="only Mamba backbones carry a profile"):
        A.unpack(f)
    # the same byte on a Mamba backbone decodes as Q8
    m = bytearray(A.build_header(A.default_header(10, A.BACKBONE_MAMBA, 1, 12)))
    assert A.decode_profile(A.parse_header(with_payload(bytes(m)))) == 1
