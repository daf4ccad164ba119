"""ctypes binding of the RDKT container in libredukt_host.so (include/redukt_archive.h):
CRC-32, the v5 header writer and the v2-v5 reader of the reference host
(src/application/codec.rs, src/domain/crc32.rs), plus pack/unpack of whole archives."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields
from typing import Optional, Tuple

import numpy as np

from . import codec

BACKBONE_RWKV, BACKBONE_MAMBA, BACKBONE_MAMBA_BYTE, BACKBONE_PLUGIN = 0, 1, 2, 3
DEFAULT_RESET_LOG2 = 12


class _Header(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint8), ("legacy_magic", ctypes.c_uint8), ("has_token_count", ctypes.c_uint8),
                ("has_crc", ctypes.c_uint8), ("total_bytes", ctypes.c_uint32), ("token_count", ctypes.c_uint32),
                ("bias_lr", ctypes.c_float), ("ngram_scale", ctypes.c_float), ("mix_eta", ctypes.c_float),
                ("emb_method", ctypes.c_uint8), ("emb_alpha", ctypes.c_float), ("e8e9", ctypes.c_uint8),
                ("shuffle_stride", ctypes.c_uint8), ("delta_stride", ctypes.c_uint8),
                ("skip_threshold", ctypes.c_uint8), ("backbone", ctypes.c_uint8), ("enhanced_cm", ctypes.c_uint8),
                ("quant", ctypes.c_uint8), ("contract", ctypes.c_uint8), ("reset_log2", ctypes.c_uint8),
                ("header_size", ctypes.c_uint32)]


@dataclass
class Header:
    total_bytes: int = 0
    backbone: int = BACKBONE_PLUGIN
    quant: int = 0
    contract: int = 1
    reset_log2: int = DEFAULT_RESET_LOG2
    bias_lr: float = 0.30
    ngram_scale: float = 0.50
    mix_eta: float = 0.01
    emb_method: int = 0
    emb_alpha: float = 0.0
    e8e9: bool = False
    shuffle_stride: int = 0
    delta_stride: int = 0
    skip_threshold: int = 0
    enhanced_cm: bool = False
    # filled by parse_header
    version: int = 5
    legacy_magic: bool = False
    has_token_count: bool = False
    token_count: int = 0
    has_crc: bool = True
    header_size: int = 0

    @property
    def reset_every(self) -> int:
        """The period a decoder replays: RWKV ignores any period (model_loader.rs:121-128)."""
        if self.reset_log2 == 0 or self.backbone == BACKBONE_RWKV:
            return 0
        return 1 << self.reset_log2

    def _to_c(self) -> _Header:
        c = _Header()
        for f in fields(self):
            setattr(c, f.name, int(getattr(self, f.name)) if not isinstance(getattr(self, f.name), float)
                    else getattr(self, f.name))
        return c

    @classmethod
    def _from_c(cls, c: _Header) -> "Header":
        h = cls()
        for f in fields(cls):
            v = getattr(c, f.name)
            setattr(h, f.name, bool(v) if isinstance(f.default, bool) else v)
        return h


class ArchiveError(ValueError):
    pass


def _lib():
    lib = codec.load()
    if not getattr(lib, "_archive_bound", False):
        u8p, hp = ctypes.POINTER(ctypes.c_uint8), ctypes.POINTER(_Header)
        sig = {
            "redukt_crc32": (ctypes.c_uint32, [u8p, ctypes.c_size_t]),
            "redukt_crc32_update": (ctypes.c_uint32, [ctypes.c_uint32, u8p, ctypes.c_size_t]),
            "redukt_rdkt_default_header": (None, [hp, ctypes.c_uint32, ctypes.c_uint8, ctypes.c_uint8, ctypes.c_uint8]),
            "redukt_rdkt_build_header": (ctypes.c_int32, [hp, u8p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t),
                                                          ctypes.c_char_p, ctypes.c_size_t]),
            "redukt_rdkt_validate_magic": (ctypes.c_int32, [u8p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint8),
                                                            ctypes.c_char_p, ctypes.c_size_t]),
            "redukt_rdkt_parse_header": (ctypes.c_int32, [u8p, ctypes.c_size_t, hp, ctypes.c_char_p, ctypes.c_size_t]),
            "redukt_rdkt_decode_profile": (ctypes.c_int32, [hp, ctypes.POINTER(ctypes.c_uint8), ctypes.c_char_p,
                                                            ctypes.c_size_t]),
            "redukt_rdkt_split": (ctypes.c_int32, [u8p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint8,
                                                   ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t),
                                                   ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint8)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        lib._archive_bound = True
    return lib


def _buf(data: bytes):
    a = np.frombuffer(bytes(data), np.uint8)
    return a, (a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)) if a.size else None)


def crc32(data: bytes, state: Optional[int] = None) -> int:
    a, p = _buf(data)
    if state is None:
        return int(_lib().redukt_crc32(p, a.size))
    return int(_lib().redukt_crc32_update(state, p, a.size))


def default_header(total_bytes: int, backbone: int = BACKBONE_PLUGIN, quant: int = 0,
                   reset_log2: int = DEFAULT_RESET_LOG2) -> Header:
    c = _Header()
    _lib().redukt_rdkt_default_header(ctypes.byref(c), total_bytes, backbone, quant, reset_log2)
    return Header._from_c(c)


def build_header(h: Header) -> bytes:
    c = h._to_c()
    out = (ctypes.c_uint8 * 64)()
    n = ctypes.c_size_t(0)
    err = ctypes.create_string_buffer(256)
    rc = _lib().redukt_rdkt_build_header(ctypes.byref(c), out, 64, ctypes.byref(n), err, 256)
    if rc != 0:
        raise ArchiveError(err.value.decode() or f"build_header: status {rc}")
    return bytes(out[: n.value])


def validate_magic(data: bytes) -> int:
    a, p = _buf(data)
    v = ctypes.c_uint8(0)
    err = ctypes.create_string_buffer(256)
    if _lib().redukt_rdkt_validate_magic(p, a.size, ctypes.byref(v), err, 256) != 0:
        raise ArchiveError(err.value.decode())
    return int(v.value)


def parse_header(data: bytes) -> Header:
    a, p = _buf(data)
    c = _Header()
    err = ctypes.create_string_buffer(256)
    if _lib().redukt_rdkt_parse_header(p, a.size, ctypes.byref(c), err, 256) != 0:
        raise ArchiveError(err.value.decode())
    return Header._from_c(c)


def decode_profile(h: Header) -> int:
    """The weight profile a decoder takes from the header (resolve_decompress_profile,
    codec.rs:719-741): refuses a non-F32 profile outside the Mamba family."""
    c = h._to_c()
    q = ctypes.c_uint8(0)
    err = ctypes.create_string_buffer(256)
    if _lib().redukt_rdkt_decode_profile(ctypes.byref(c), ctypes.byref(q), err, 256) != 0:
        raise ArchiveError(err.value.decode())
    return int(q.value)


def split(data: bytes, header_size: int, version: int) -> Tuple[bytes, Optional[int]]:
    """(stream, stored CRC or None for v2)."""
    a, p = _buf(data)
    off, n, crc, has = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_uint32(), ctypes.c_uint8()
    if _lib().redukt_rdkt_split(p, a.size, header_size, version, ctypes.byref(off), ctypes.byref(n),
                                ctypes.byref(crc), ctypes.byref(has)) != 0:
        raise ArchiveError(f"truncated RDKT file: {a.size} bytes, header {header_size}")
    return bytes(data[off.value: off.value + n.value]), (int(crc.value) if has.value else None)


def pack(header: Header, stream: bytes, payload: bytes) -> bytes:
    """HEADER | STREAM | CRC-32(payload), the layout of the reference's archives."""
    return build_header(header) + bytes(stream) + crc32(payload).to_bytes(4, "little")


def unpack(data: bytes) -> Tuple[Header, bytes, Optional[int]]:
    """Header, stream and stored CRC of an archive a decoder accepts: the header parsed,
    its weight profile resolved for decoding (non-F32 outside the Mamba family refused)."""
    h = parse_header(data)
    decode_profile(h)
    stream, crc = split(data, h.header_size, h.version)
    return h, stream, crc
