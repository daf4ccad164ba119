"""ctypes binding of libredukt_host.so's coding path (include/redukt_codec.h).

Mirrors the reference host's coder API: `Cdf` construction from probabilities, logits or a
uniform distribution (src/domain/coder.rs:43-115, src/application/codec.rs:785-798) and the
carry range coder (src/domain/coder.rs:118-296).  A CDF is a uint32 array of n + 1 entries
whose last entry is the total.  Everything here runs on the host CPU, as in the reference;
the library must be built (make -C redukt_amd/csrc/host) and there is no Python fallback.
"""
from __future__ import annotations

import ctypes
import enum
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(HERE, "libredukt_host.so")
CDF_TOTAL = 1 << 24

_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)


class CodecStatus(enum.IntEnum):
    OK = 0
    INVALID_ARG = 1
    RANGE_UNDERFLOW = 2
    SYMBOL_OUT_OF_RANGE = 3
    BUFFER_TOO_SMALL = 4
    INCOMPLETE = 5


class CodecError(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = CodecStatus(status)
        super().__init__(f"{what}: {self.status.name}")


def _check(code: int, what: str) -> None:
    if code != CodecStatus.OK:
        raise CodecError(code, what)


_LIB: Optional[ctypes.CDLL] = None


def load(path: str = DEFAULT_LIB) -> ctypes.CDLL:
    """Loads the host library once; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (make -C redukt_amd/csrc/host)")
    lib = ctypes.CDLL(path)
    sig = {
        "redukt_exp_f64": (ctypes.c_double, [ctypes.c_double]),
        "redukt_cdf_from_probs": (ctypes.c_int32, [_f32p, ctypes.c_uint32, _u32p]),
        "redukt_cdf_uniform": (ctypes.c_int32, [ctypes.c_uint32, _u32p]),
        "redukt_cdf_from_logits": (ctypes.c_int32, [_f32p, ctypes.c_uint32, _u32p]),
        "redukt_cdf_from_logits_batch": (ctypes.c_int32, [_f32p, ctypes.c_uint32, ctypes.c_uint32, _u32p,
                                                          ctypes.c_uint32]),
        "redukt_cdf_lookup": (ctypes.c_uint32, [_u32p, ctypes.c_uint32, ctypes.c_uint32]),
        "redukt_rc_encoder_new": (ctypes.c_void_p, []),
        "redukt_rc_encoder_free": (None, [ctypes.c_void_p]),
        "redukt_rc_encode": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]),
        "redukt_rc_encode_symbol": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_uint32, _u32p, ctypes.c_uint32]),
        "redukt_rc_encoder_size": (ctypes.c_size_t, [ctypes.c_void_p]),
        "redukt_rc_finish": (ctypes.c_size_t, [ctypes.c_void_p, _u8p, ctypes.c_size_t]),
        "redukt_rc_decoder_new": (ctypes.c_void_p, [_u8p, ctypes.c_size_t]),
        "redukt_rc_decoder_free": (None, [ctypes.c_void_p]),
        "redukt_rc_decode_symbol": (ctypes.c_int32, [ctypes.c_void_p, _u32p, ctypes.c_uint32, ctypes.c_uint32,
                                                     _u32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    _LIB = lib
    return lib


def _p(a: np.ndarray, ct):
    return a.ctypes.data_as(ct)


def exp_f64(x: float) -> float:
    return load().redukt_exp_f64(float(x))


def cdf_from_probs(probs) -> np.ndarray:
    p = np.ascontiguousarray(probs, np.float32)
    out = np.empty(p.size + 1, np.uint32)
    _check(load().redukt_cdf_from_probs(_p(p, _f32p), p.size, _p(out, _u32p)), "cdf_from_probs")
    return out


def cdf_uniform(n: int) -> np.ndarray:
    out = np.empty(n + 1, np.uint32)
    _check(load().redukt_cdf_uniform(n, _p(out, _u32p)), "cdf_uniform")
    return out


def cdf_from_logits(logits) -> np.ndarray:
    lg = np.ascontiguousarray(logits, np.float32)
    out = np.empty(lg.size + 1, np.uint32)
    _check(load().redukt_cdf_from_logits(_p(lg, _f32p), lg.size, _p(out, _u32p)), "cdf_from_logits")
    return out


def cdf_from_logits_batch(logits: np.ndarray, threads: int = 0, out: Optional[np.ndarray] = None) -> np.ndarray:
    """logits [rows, n] -> cdf [rows, n + 1], rows on the host thread pool."""
    lg = np.ascontiguousarray(logits, np.float32)
    rows, n = lg.shape
    if out is None:
        out = np.empty((rows, n + 1), np.uint32)
    assert out.shape == (rows, n + 1) and out.dtype == np.uint32 and out.flags.c_contiguous
    _check(load().redukt_cdf_from_logits_batch(_p(lg, _f32p), rows, n, _p(out, _u32p), threads),
           "cdf_from_logits_batch")
    return out


def lookup(cdf: np.ndarray, cum: int) -> int:
    c = np.ascontiguousarray(cdf, np.uint32)
    return int(load().redukt_cdf_lookup(_p(c, _u32p), c.size - 1, cum))


class RangeEncoder:
    def __init__(self):
        self._lib = load()
        self._h = self._lib.redukt_rc_encoder_new()
        if not self._h:
            raise MemoryError("redukt_rc_encoder_new")

    def encode(self, lo: int, hi: int, total: int) -> None:
        _check(self._lib.redukt_rc_encode(self._h, lo, hi, total), "encode")

    def encode_symbol(self, sym: int, cdf: np.ndarray) -> None:
        c = np.ascontiguousarray(cdf, np.uint32)
        _check(self._lib.redukt_rc_encode_symbol(self._h, sym, _p(c, _u32p), c.size - 1), "encode_symbol")

    def size(self) -> int:
        return int(self._lib.redukt_rc_encoder_size(self._h))

    def finish(self) -> bytes:
        n = self._lib.redukt_rc_finish(self._h, None, 0)
        buf = np.empty(max(n, 1), np.uint8)
        self._lib.redukt_rc_finish(self._h, _p(buf, _u8p), n)
        return buf[:n].tobytes()

    def __del__(self):
        if getattr(self, "_h", None):
            self._lib.redukt_rc_encoder_free(self._h)
            self._h = None


class RangeDecoder:
    def __init__(self, data: bytes):
        self._lib = load()
        buf = np.frombuffer(bytes(data), np.uint8)
        self._h = self._lib.redukt_rc_decoder_new(_p(buf, _u8p) if buf.size else None, buf.size)
        if not self._h:
            raise MemoryError("redukt_rc_decoder_new")

    def decode_symbol(self, cdf: np.ndarray, vocab: int = 0) -> int:
        """vocab > 0 checks the symbol against it (decode_symbol_checked)."""
        c = np.ascontiguousarray(cdf, np.uint32)
        s = ctypes.c_uint32(0)
        _check(self._lib.redukt_rc_decode_symbol(self._h, _p(c, _u32p), c.size - 1, vocab, ctypes.byref(s)),
               "decode_symbol")
        return int(s.value)

    def __del__(self):
        if getattr(self, "_h", None):
            self._lib.redukt_rc_decoder_free(self._h)
            self._h = None
