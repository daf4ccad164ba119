"""ctypes binding of the lockstep driver in libredukt_host.so (include/redukt_lockstep.h).

`Lockstep` loads a backend plugin (libredukt_gpu.so by default) through the C++ driver
and compresses / decompresses token files with it, N streams per step
(src/application/lockstep.rs), or one file at a time on the plugin's v1 state when
slots=0 (the reference's `compress --input` path)."""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import codec

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_PLUGIN = os.path.join(HERE, "libredukt_gpu.so")
DEFAULT_RESET_EVERY = 4096  # 2^12, the Mamba family default (src/application/codec.rs:42)


class LockstepStatus(enum.IntEnum):
    OK = 0
    INVALID_ARG = 1
    PLUGIN_LOAD = 2
    PLUGIN_INIT = 3
    FORWARD = 4
    CODER = 5
    BUFFER_TOO_SMALL = 6
    NEEDS_V2 = 7


class LockstepError(RuntimeError):
    def __init__(self, status: int, what: str, file_status: Optional[List[int]] = None):
        self.status = LockstepStatus(status)
        self.file_status = [codec.CodecStatus(s) for s in file_status] if file_status is not None else None
        super().__init__(f"{what}: {self.status.name}" + (f" {self.file_status}" if file_status is not None else ""))


class _Stats(ctypes.Structure):
    _fields_ = [("steps", ctypes.c_uint64), ("tokens", ctypes.c_uint64), ("files", ctypes.c_uint64),
                ("secs", ctypes.c_double), ("code_secs", ctypes.c_double), ("forward_secs", ctypes.c_double)]


@dataclass
class Stats:
    steps: int
    tokens: int
    files: int
    secs: float
    code_secs: float
    forward_secs: float

    @property
    def tok_per_s(self) -> float:
        return self.tokens / self.secs if self.secs > 0 else 0.0


_u64p = ctypes.POINTER(ctypes.c_uint64)
_i32p = ctypes.POINTER(ctypes.c_int32)


def _bind(lib: ctypes.CDLL) -> None:
    if getattr(lib, "_lockstep_bound", False):
        return
    vp, pp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
    sig = {
        "redukt_lockstep_open": (ctypes.c_int32, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32,
                                                  ctypes.c_uint32, ctypes.c_uint32, pp]),
        "redukt_lockstep_close": (None, [vp]),
        "redukt_lockstep_vocab": (ctypes.c_uint32, [vp]),
        "redukt_lockstep_backend_name": (ctypes.c_char_p, [vp]),
        "redukt_lockstep_stream_bound": (ctypes.c_uint64, [ctypes.c_uint64]),
        "redukt_lockstep_set_device_cdf": (ctypes.c_int32, [vp, ctypes.c_int32]),
        "redukt_lockstep_device_cdf": (ctypes.c_int32, [vp]),
        "redukt_lockstep_compress": (ctypes.c_int32, [vp, ctypes.c_uint32, pp, _u64p, ctypes.c_uint64, pp, _u64p,
                                                      _u64p, _i32p, ctypes.POINTER(_Stats)]),
        "redukt_lockstep_decompress": (ctypes.c_int32, [vp, ctypes.c_uint32, pp, _u64p, _u64p, ctypes.c_uint64, pp,
                                                        _i32p, ctypes.POINTER(_Stats)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    lib._lockstep_bound = True


def _ptrs(arrays: Sequence[np.ndarray]):
    arr = (ctypes.c_void_p * max(len(arrays), 1))()
    for i, a in enumerate(arrays):
        arr[i] = a.ctypes.data if a.size else None
    return ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p)), arr


def stream_bound(n_tokens: int) -> int:
    lib = codec.load()
    _bind(lib)
    return int(lib.redukt_lockstep_stream_bound(n_tokens))


class Lockstep:
    def __init__(self, weights_path: str, plugin_path: str = DEFAULT_PLUGIN, device_id: int = 0,
                 profile: Optional[int] = None, slots: int = 0, threads: int = 0,
                 device_cdf: Optional[bool] = None):
        self._lib = codec.load()
        _bind(self._lib)
        h = ctypes.c_void_p()
        rc = self._lib.redukt_lockstep_open(plugin_path.encode(), weights_path.encode(), device_id,
                                            -1 if profile is None else int(profile), slots, threads, ctypes.byref(h))
        if rc != 0:
            raise LockstepError(rc, f"open({plugin_path}, {weights_path}, slots={slots})")
        self._h = h
        if device_cdf is not None:   # None: the driver's default (device CDFs where the plugin has them)
            rc = self._lib.redukt_lockstep_set_device_cdf(h, 1 if device_cdf else 0)
            if rc != 0:
                self.close()
                raise LockstepError(rc, "set_device_cdf (the plugin has no forward_batch_cdf, or slots = 0)")
        self.slots = slots
        self.vocab = int(self._lib.redukt_lockstep_vocab(h))
        self.name = self._lib.redukt_lockstep_backend_name(h).decode()

    @property
    def device_cdf(self) -> bool:
        return bool(self._lib.redukt_lockstep_device_cdf(self._h))

    def compress(self, files: Sequence[Sequence[int]], reset_every: int = DEFAULT_RESET_EVERY
                 ) -> Tuple[List[bytes], Stats]:
        toks = [np.ascontiguousarray(f, np.uint32) for f in files]
        n = len(toks)
        lens = np.array([t.size for t in toks] or [0], np.uint64)
        outs = [np.empty(stream_bound(t.size), np.uint8) for t in toks]
        caps = np.array([o.size for o in outs] or [0], np.uint64)
        out_len = np.zeros(max(n, 1), np.uint64)
        status = np.zeros(max(n, 1), np.int32)
        tp, _k1 = _ptrs(toks)
        op, _k2 = _ptrs(outs)
        st = _Stats()
        rc = self._lib.redukt_lockstep_compress(self._h, n, tp, lens.ctypes.data_as(_u64p), reset_every, op,
                                                caps.ctypes.data_as(_u64p), out_len.ctypes.data_as(_u64p),
                                                status.ctypes.data_as(_i32p), ctypes.byref(st))
        if rc != 0:
            raise LockstepError(rc, "compress", list(status[:n]))
        return [outs[i][: int(out_len[i])].tobytes() for i in range(n)], Stats(*[getattr(st, f) for f, _ in st._fields_])

    def decompress(self, streams: Sequence[bytes], n_tokens: Sequence[int], reset_every: int = DEFAULT_RESET_EVERY
                   ) -> Tuple[List[np.ndarray], Stats]:
        n = len(streams)
        if len(n_tokens) != n:
            raise ValueError(f"decompress: {n} streams but {len(n_tokens)} token counts")
        data = [np.frombuffer(bytes(s), np.uint8).copy() for s in streams]
        slen = np.array([d.size for d in data] or [0], np.uint64)
        ntok = np.array(list(n_tokens) or [0], np.uint64)
        outs = [np.zeros(int(k), np.uint32) for k in n_tokens]
        status = np.zeros(max(n, 1), np.int32)
        sp, _k1 = _ptrs(data)
        op, _k2 = _ptrs(outs)
        st = _Stats()
        rc = self._lib.redukt_lockstep_decompress(self._h, n, sp, slen.ctypes.data_as(_u64p),
                                                  ntok.ctypes.data_as(_u64p), reset_every, op,
                                                  status.ctypes.data_as(_i32p), ctypes.byref(st))
        if rc != 0:
            raise LockstepError(rc, "decompress", list(status[:n]))
        return outs, Stats(*[getattr(st, f) for f, _ in st._fields_])

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.redukt_lockstep_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()
