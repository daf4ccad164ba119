"""Host side of the plugin boundary, mirroring redukt's Rust host over ctypes.

`PluginLibrary` follows src/infrastructure/plugin_backend/loader.rs:128-253 (dlopen,
four required v1 symbols, optional v2 table enabled only when every v2 symbol resolves
and abi_version() >= 2, ffi_version == 1 check after init, free on drop).
`validate_batch_args` is backend_ffi.rs:182-202.  `PluginBackend`, `PluginState` and
`SlotPool` follow plugin_backend/model.rs:32-103, 249-452: slot hand-out, the periodic
reset `tick`, one `forward_batch` per lockstep step.  The v3 extensions of
include/redukt_backend.h are exposed when abi_version() >= 3.

The library is loaded from this package directory; a missing library raises — there
is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import enum
import os
from typing import List, Optional, Sequence

import numpy as np

LIB_NAME = "libredukt_gpu.so"
PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(PACKAGE_DIR, LIB_NAME)

BACKEND_FFI_VERSION = 1
BACKEND_ABI_V2 = 2
BACKEND_ABI_V3 = 3
BACKEND_NAME_MAX = 64

PROFILE_F32 = 0
PROFILE_Q8_G64 = 1
PROFILE_Q8_ROW = 2
PROFILE_Q8_SMALL = 4
PROFILE_EXACT_SCAN = 8  # Mamba scan decay by the portable exp instead of the hardware exp2
PROFILE_GEMV = 16       # Mamba projections on the wavefront-GEMV kernels (the small-batch tier)
PROFILE_W8A8 = 32       # RWKV-7 in the reference's own W8A8 arithmetic (with PROFILE_Q8_ROW), bit-exact
PROFILE_EXACT = 64      # the reference GEMV orders, numeric contract 1: logits bit-exact to the CPU path (Mamba; RWKV-7 F32)
PROFILE_FMA = 128       # the same in numeric contract 2 (fma-v1); implies PROFILE_EXACT

V1_SYMBOLS = ("redukt_backend_init", "redukt_backend_forward", "redukt_backend_reset_state", "redukt_backend_free")
V2_SYMBOLS = ("redukt_backend_abi_version", "redukt_backend_batch_init", "redukt_backend_batch_reset",
              "redukt_backend_forward_batch")
V3_SYMBOLS = ("redukt_backend_init_ex", "redukt_backend_forward_batch_probs", "redukt_backend_forward_batch_device",
              "redukt_backend_device_status", "redukt_backend_stream", "redukt_backend_get_state",
              "redukt_backend_probe_kernel", "redukt_backend_probe_used", "redukt_backend_get_rwkv_state",
              "redukt_backend_eval_math", "redukt_backend_forward_batch_device_noalloc",
              "redukt_backend_forward_batch_cdf", "redukt_backend_cdf_from_logits_device",
              "redukt_backend_copy_probe", "redukt_backend_forward_batch_cdf_sym",
              "redukt_backend_forward_batch_cdf_find",
              "redukt_backend_forward_batch_cdf_sym_submit", "redukt_backend_forward_batch_cdf_sym_wait")
# redukt_backend_eval_math function codes: the portable element-wise functions
MATH_FNS = {"exp": 0, "lane_exp": 1, "ln": 2, "softplus": 3, "lane_sigmoid": 4, "sigmoid": 5}

# Kernel classes of redukt_backend_probe_kernel, and the flag that makes a probed step
# launch only the kernels of that class (REDUKT_PROBE_CLASS_ONLY).
KERNEL_CLASSES = {"embed": 1, "mix_in": 2, "scan": 3, "mix_out": 4, "head": 5, "softmax": 6}
RWKV_KERNEL_CLASSES = {"embed": 1, "shift": 7, "proj": 8, "wkv": 9, "head": 5, "softmax": 6}
PROBE_CLASS_ONLY = 0x100
KC_FLOW = 10  # the persistent step kernel (REDUKT_GPU_FLOW), probed without PROBE_CLASS_ONLY


class BackendResult(enum.IntEnum):
    """backend_ffi.rs:27-41."""
    OK = 0
    INIT_FAILED = 1
    FORWARD_FAILED = 2
    VERSION_MISMATCH = 3
    WEIGHTS_NOT_FOUND = 4
    INVALID_ARGUMENT = 5

    @classmethod
    def from_code(cls, code: int) -> "BackendResult":
        """backend_ffi.rs:48-57: unknown codes map to FORWARD_FAILED."""
        return {0: cls.OK, 1: cls.INIT_FAILED, 3: cls.VERSION_MISMATCH, 4: cls.WEIGHTS_NOT_FOUND,
                5: cls.INVALID_ARGUMENT}.get(int(code), cls.FORWARD_FAILED)


class BackendError(RuntimeError):
    def __init__(self, result: BackendResult, what: str = ""):
        super().__init__(f"{what}: {result.name}" if what else result.name)
        self.result = result


class BackendInfo(ctypes.Structure):
    """76-byte repr(C) struct, backend_ffi.rs:63-72."""
    _fields_ = [("ffi_version", ctypes.c_uint32), ("vocab_size", ctypes.c_uint32),
                ("hidden_dim", ctypes.c_uint32), ("name", ctypes.c_uint8 * BACKEND_NAME_MAX)]

    def name_str(self) -> str:
        raw = bytes(self.name)
        end = raw.find(b"\0")
        try:
            return raw[: end if end >= 0 else BACKEND_NAME_MAX].decode()
        except UnicodeDecodeError:
            return "unknown"


def validate_batch_args(slots: Sequence[int], tokens: Sequence[int], out_len: int, vocab_size: int,
                        max_streams: int, seen: List[bool]) -> Optional[BackendResult]:
    """backend_ffi.rs:182-202: None when valid, else INVALID_ARGUMENT."""
    n = len(slots)
    if not (len(tokens) == n and n <= max_streams and len(seen) >= max_streams and out_len == n * vocab_size):
        return BackendResult.INVALID_ARGUMENT
    for i in range(len(seen)):
        seen[i] = False
    for slot, tok in zip(slots, tokens):
        if slot >= max_streams or tok >= vocab_size or seen[slot]:
            return BackendResult.INVALID_ARGUMENT
        seen[slot] = True
    return None


_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)


def _ptr(a: np.ndarray, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


class PluginLibrary:
    """A loaded plugin with its v1 table and, when available, the v2/v3 tables."""

    def __init__(self, path: str = DEFAULT_LIB):
        if not os.path.isfile(path):
            raise FileNotFoundError(f"{path} is not built (run __graft_entry__.build())")
        self.path = path
        self.lib = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
        for s in V1_SYMBOLS:
            if not hasattr(self.lib, s):
                raise OSError(f"{path}: missing required symbol {s}")
        L = self.lib
        L.redukt_backend_init.argtypes = [ctypes.c_char_p, ctypes.c_int32, ctypes.POINTER(BackendInfo)]
        L.redukt_backend_init.restype = ctypes.c_int
        L.redukt_backend_forward.argtypes = [ctypes.c_uint32, _f32p, ctypes.c_uint32]
        L.redukt_backend_forward.restype = ctypes.c_int
        L.redukt_backend_reset_state.argtypes = []
        L.redukt_backend_reset_state.restype = None
        L.redukt_backend_free.argtypes = []
        L.redukt_backend_free.restype = None
        self.abi_version = self._resolve_v2()
        self.has_v3 = self.abi_version is not None and self.abi_version >= BACKEND_ABI_V3 and all(
            hasattr(L, s) for s in V3_SYMBOLS)
        if self.has_v3:
            L.redukt_backend_init_ex.argtypes = [ctypes.c_char_p, ctypes.c_int32, ctypes.c_uint32,
                                                 ctypes.POINTER(BackendInfo)]
            L.redukt_backend_init_ex.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_probs.argtypes = [ctypes.c_uint32, _u32p, _u32p, _f32p, ctypes.c_uint32]
            L.redukt_backend_forward_batch_probs.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_device.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p,
                                                              ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32]
            L.redukt_backend_forward_batch_device.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_device_noalloc.argtypes = L.redukt_backend_forward_batch_device.argtypes
            L.redukt_backend_forward_batch_device_noalloc.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_cdf.argtypes = [ctypes.c_uint32, _u32p, _u32p, _u32p, ctypes.c_uint32]
            L.redukt_backend_forward_batch_cdf.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_cdf_sym.argtypes = [ctypes.c_uint32, _u32p, _u32p, _u32p, _u32p,
                                                               ctypes.c_uint32]
            L.redukt_backend_forward_batch_cdf_sym.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_cdf_find.argtypes = [ctypes.c_uint32, _u32p, _u32p, _u32p, _u32p,
                                                                ctypes.c_uint32]
            L.redukt_backend_forward_batch_cdf_find.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_cdf_sym_submit.argtypes = [ctypes.c_uint32, _u32p, _u32p, _u32p,
                                                                      ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint64)]
            L.redukt_backend_forward_batch_cdf_sym_submit.restype = ctypes.c_int32
            L.redukt_backend_forward_batch_cdf_sym_wait.argtypes = [ctypes.c_uint64, _u32p, ctypes.c_uint32]
            L.redukt_backend_forward_batch_cdf_sym_wait.restype = ctypes.c_int32
            L.redukt_backend_cdf_from_logits_device.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                                ctypes.c_void_p]
            L.redukt_backend_cdf_from_logits_device.restype = ctypes.c_int32
            L.redukt_backend_device_status.argtypes = []
            L.redukt_backend_device_status.restype = ctypes.c_int32
            L.redukt_backend_stream.argtypes = []
            L.redukt_backend_stream.restype = ctypes.c_void_p
            L.redukt_backend_get_state.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p]
            L.redukt_backend_get_state.restype = ctypes.c_int32
            L.redukt_backend_get_rwkv_state.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p, _f32p]
            L.redukt_backend_get_rwkv_state.restype = ctypes.c_int32
            L.redukt_backend_probe_kernel.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32]
            L.redukt_backend_probe_kernel.restype = ctypes.c_int32
            L.redukt_backend_probe_used.argtypes = []
            L.redukt_backend_probe_used.restype = ctypes.c_uint32
            L.redukt_backend_eval_math.argtypes = [ctypes.c_uint32, _f32p, _f32p, ctypes.c_uint32]
            L.redukt_backend_eval_math.restype = ctypes.c_int32
            L.redukt_backend_copy_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32]
            L.redukt_backend_copy_probe.restype = ctypes.c_int32

    def eval_math(self, fn: str, x: np.ndarray) -> np.ndarray:
        """One portable element-wise function evaluated on the device (test hook)."""
        xi = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(xi)
        res = BackendResult.from_code(self.lib.redukt_backend_eval_math(MATH_FNS[fn], _ptr(xi, ctypes.c_float),
                                                                         _ptr(y, ctypes.c_float), xi.size))
        if res != BackendResult.OK:
            raise BackendError(res, f"eval_math({fn})")
        return y

    def _resolve_v2(self) -> Optional[int]:
        """loader.rs:196-216: all four symbols and abi >= 2, else v1 only."""
        L = self.lib
        if not all(hasattr(L, s) for s in V2_SYMBOLS):
            return None
        L.redukt_backend_abi_version.argtypes = []
        L.redukt_backend_abi_version.restype = ctypes.c_uint32
        abi = int(L.redukt_backend_abi_version())
        if abi < BACKEND_ABI_V2:
            return None
        L.redukt_backend_batch_init.argtypes = [ctypes.c_uint32]
        L.redukt_backend_batch_init.restype = ctypes.c_int32
        L.redukt_backend_batch_reset.argtypes = [_u32p, ctypes.c_uint32]
        L.redukt_backend_batch_reset.restype = ctypes.c_int32
        L.redukt_backend_forward_batch.argtypes = [ctypes.c_uint32, _u32p, _u32p, _f32p, ctypes.c_uint32]
        L.redukt_backend_forward_batch.restype = ctypes.c_int32
        return abi

    def init(self, weights_path: str, device_id: int = 0, profile: Optional[int] = None) -> BackendInfo:
        """loader.rs:219-245; `profile` selects the v3 init_ex."""
        info = BackendInfo()
        raw = weights_path.encode()
        if profile is None:
            res = BackendResult(self.lib.redukt_backend_init(raw, device_id, ctypes.byref(info)))
        else:
            if not self.has_v3:
                raise BackendError(BackendResult.VERSION_MISMATCH, "init_ex")
            res = BackendResult.from_code(self.lib.redukt_backend_init_ex(raw, device_id, profile, ctypes.byref(info)))
        if res != BackendResult.OK:
            raise BackendError(res, "init")
        if info.ffi_version != BACKEND_FFI_VERSION:
            raise BackendError(BackendResult.VERSION_MISMATCH, "init")
        return info

    def free(self) -> None:
        self.lib.redukt_backend_free()


class SlotPool:
    """plugin_backend/model.rs:81-103."""

    def __init__(self):
        self.cap = 0
        self.next = 0
        self.seen: List[bool] = []

    def init(self, cap: int) -> None:
        self.cap, self.next, self.seen = cap, 0, [False] * cap

    def take(self) -> Optional[int]:
        if self.next < self.cap:
            self.next += 1
            return self.next - 1
        return None


class PluginState:
    """plugin_backend/model.rs:32-76: a slot (or the v1 global state) plus the
    periodic-reset schedule."""

    def __init__(self, backend: "PluginBackend", slot: Optional[int]):
        self.backend = backend
        self.slot = slot
        self.reset_every = 0
        self.since_reset = 0

    def set_reset_every(self, every: int) -> None:
        self.reset_every = every

    def tick(self) -> None:
        if self.reset_every > 0 and self.since_reset >= self.reset_every:
            self.reset()
        self.since_reset += 1

    def reset(self) -> None:
        self.since_reset = 0
        if self.slot is not None and self.backend.lib.abi_version is not None:
            self.backend.batch_reset([self.slot])
        else:
            self.backend.lib.lib.redukt_backend_reset_state()


class PluginBackend:
    """plugin_backend/model.rs:249-452 over a loaded `PluginLibrary`."""

    def __init__(self, weights_path: str, device_id: int = 0, profile: Optional[int] = None,
                 lib_path: str = DEFAULT_LIB):
        self.lib = PluginLibrary(lib_path)
        self.info = self.lib.init(weights_path, device_id, profile)
        self.vocab = int(self.info.vocab_size)
        self.pool = SlotPool()
        self._closed = False

    # ---- v2 batch API (model.rs:303-354) ----
    def batch_abi(self) -> Optional[int]:
        return self.lib.abi_version

    def batch_init(self, max_streams: int) -> None:
        if self.lib.abi_version is None:
            raise BackendError(BackendResult.VERSION_MISMATCH, "batch_init")
        res = BackendResult.from_code(self.lib.lib.redukt_backend_batch_init(max_streams))
        if res != BackendResult.OK:
            raise BackendError(res, f"batch_init({max_streams})")
        self.pool.init(max_streams)

    def batch_reset(self, slots: Optional[Sequence[int]] = None) -> None:
        if self.lib.abi_version is None:
            raise BackendError(BackendResult.VERSION_MISMATCH, "batch_reset")
        if slots is None:
            code = self.lib.lib.redukt_backend_batch_reset(None, 0)
        else:
            s = np.ascontiguousarray(slots, dtype=np.uint32)
            code = self.lib.lib.redukt_backend_batch_reset(_ptr(s, ctypes.c_uint32), len(s))
        res = BackendResult.from_code(code)
        if res != BackendResult.OK:
            raise BackendError(res, "batch_reset")

    def forward_batch(self, slots: Sequence[int], tokens: Sequence[int], out: np.ndarray,
                      probs: bool = False) -> None:
        if self.lib.abi_version is None:
            raise BackendError(BackendResult.VERSION_MISMATCH, "forward_batch")
        err = validate_batch_args(list(slots), list(tokens), out.size, self.vocab, self.pool.cap, self.pool.seen)
        if err is not None:
            raise BackendError(err, "forward_batch")
        if len(slots) == 0:
            return
        assert out.dtype == np.float32 and out.flags.c_contiguous
        s = np.ascontiguousarray(slots, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        fn = self.lib.lib.redukt_backend_forward_batch_probs if probs else self.lib.lib.redukt_backend_forward_batch
        res = BackendResult.from_code(fn(len(s), _ptr(s, ctypes.c_uint32), _ptr(t, ctypes.c_uint32),
                                         _ptr(out, ctypes.c_float), self.vocab))
        if res != BackendResult.OK:
            raise BackendError(res, "forward_batch")

    # ---- Backbone trait (model.rs:357-452) ----
    def create_state(self) -> PluginState:
        slot = self.pool.take() if self.lib.abi_version is not None else None
        return PluginState(self, slot)

    def prepare_streams(self, n: int) -> None:
        if self.lib.abi_version is None:
            if n > 1:
                raise RuntimeError(f"the GPU plugin implements FFI v1 only: --jobs {n} needs the v2 batch API")
            return
        self.batch_init(n)

    def forward_into(self, token: int, state: PluginState, out: np.ndarray) -> None:
        state.tick()
        if state.slot is not None:
            self.forward_batch([state.slot], [token], out)
            return
        res = BackendResult(self.lib.lib.redukt_backend_forward(token, _ptr(out, ctypes.c_float), out.size))
        if res != BackendResult.OK:
            raise BackendError(res, "forward")

    def forward_multi(self, tokens: Sequence[int], states: Sequence[PluginState], out: np.ndarray) -> None:
        """One forward_batch for every slot state; `out` is [n, vocab]."""
        n = len(tokens)
        slots = [s.slot for s in states]
        if n == 0:
            return
        if any(s is None for s in slots):
            for i in range(n):
                self.forward_into(tokens[i], states[i], out[i])
            return
        for s in states:
            s.tick()
        self.forward_batch(slots, tokens, out)

    # ---- v3 ----
    def forward_batch_device(self, n: int, d_slots: int, d_tokens: int, d_out: int, probs: bool = False) -> None:
        res = BackendResult.from_code(self.lib.lib.redukt_backend_forward_batch_device(
            n, d_slots, d_tokens, d_out, self.vocab, 1 if probs else 0))
        if res != BackendResult.OK:
            raise BackendError(res, "forward_batch_device")

    def forward_batch_device_noalloc(self, n: int, d_slots: int, d_tokens: int, d_out: int,
                                     probs: bool = False) -> BackendResult:
        """The allocation-free device step; returns the result code (INVALID_ARGUMENT when n
        does not fit the library's scratch)."""
        return BackendResult.from_code(self.lib.lib.redukt_backend_forward_batch_device_noalloc(
            n, d_slots, d_tokens, d_out, self.vocab, 1 if probs else 0))

    def forward_batch_cdf(self, slots: Sequence[int], tokens: Sequence[int], out: np.ndarray) -> None:
        """forward_batch returning each stream's CDF (vocab + 1 u32) computed on the device."""
        err = validate_batch_args(list(slots), list(tokens), len(slots) * self.vocab, self.vocab, self.pool.cap,
                                  self.pool.seen)
        if err is not None:
            raise BackendError(err, "forward_batch_cdf")
        if len(slots) == 0:
            return
        assert out.dtype == np.uint32 and out.flags.c_contiguous and out.size == len(slots) * (self.vocab + 1)
        s = np.ascontiguousarray(slots, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        res = BackendResult.from_code(self.lib.lib.redukt_backend_forward_batch_cdf(
            len(s), _ptr(s, ctypes.c_uint32), _ptr(t, ctypes.c_uint32), _ptr(out, ctypes.c_uint32), self.vocab + 1))
        if res != BackendResult.OK:
            raise BackendError(res, "forward_batch_cdf")

    def forward_batch_cdf_sym(self, slots: Sequence[int], tokens: Sequence[int], next_syms: Sequence[int],
                              out: np.ndarray) -> BackendResult:
        """forward_batch_cdf returning only cdf[sym], cdf[sym + 1] and the total per stream
        (out: 3 u32 a stream) for each stream's next symbol; returns the result code."""
        assert out.dtype == np.uint32 and out.flags.c_contiguous and out.size == 3 * len(slots)
        s = np.ascontiguousarray(slots, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        y = np.ascontiguousarray(next_syms, dtype=np.uint32)
        return BackendResult.from_code(self.lib.lib.redukt_backend_forward_batch_cdf_sym(
            len(s), _ptr(s, ctypes.c_uint32), _ptr(t, ctypes.c_uint32), _ptr(y, ctypes.c_uint32),
            _ptr(out, ctypes.c_uint32), self.vocab))

    def forward_batch_cdf_find(self, slots: Sequence[int], tokens: Sequence[int], targets: Sequence[int],
                               out: np.ndarray) -> BackendResult:
        """forward_batch_cdf returning, per stream, the symbol the range decoder finds for its
        target cumulative frequency with that symbol's two bounds and the total (out: 4 u32
        a stream); returns the result code."""
        assert out.dtype == np.uint32 and out.flags.c_contiguous and out.size == 4 * len(slots)
        s = np.ascontiguousarray(slots, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        y = np.ascontiguousarray(targets, dtype=np.uint32)
        return BackendResult.from_code(self.lib.lib.redukt_backend_forward_batch_cdf_find(
            len(s), _ptr(s, ctypes.c_uint32), _ptr(t, ctypes.c_uint32), _ptr(y, ctypes.c_uint32),
            _ptr(out, ctypes.c_uint32), self.vocab))

    def forward_batch_cdf_sym_submit(self, slots: Sequence[int], tokens: Sequence[int], next_syms: Sequence[int]):
        """Queues forward_batch_cdf_sym; returns (result code, ticket)."""
        s = np.ascontiguousarray(slots, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        y = np.ascontiguousarray(next_syms, dtype=np.uint32)
        ticket = ctypes.c_uint64(0)
        code = self.lib.lib.redukt_backend_forward_batch_cdf_sym_submit(
            len(s), _ptr(s, ctypes.c_uint32), _ptr(t, ctypes.c_uint32), _ptr(y, ctypes.c_uint32), self.vocab,
            ctypes.byref(ticket))
        return BackendResult.from_code(code), int(ticket.value)

    def forward_batch_cdf_sym_wait(self, ticket: int, out: np.ndarray) -> BackendResult:
        """Waits for a queued call and writes its three values per stream into out."""
        assert out.dtype == np.uint32 and out.flags.c_contiguous and out.size % 3 == 0
        return BackendResult.from_code(self.lib.lib.redukt_backend_forward_batch_cdf_sym_wait(
            ticket, _ptr(out, ctypes.c_uint32), out.size // 3))

    def cdf_from_logits_device(self, d_logits: int, rows: int, n: int, d_cdf: int) -> BackendResult:
        return BackendResult.from_code(self.lib.lib.redukt_backend_cdf_from_logits_device(d_logits, rows, n, d_cdf))

    def device_status(self) -> BackendResult:
        return BackendResult.from_code(self.lib.lib.redukt_backend_device_status())

    def stream(self) -> int:
        return int(self.lib.lib.redukt_backend_stream() or 0)

    def get_rwkv_state(self, slot: int, layer: int, d_model: int, n_head: int, head_size: int = 64):
        xa, xf = np.empty(d_model, np.float32), np.empty(d_model, np.float32)
        wkv = np.empty((n_head, head_size, head_size), np.float32)
        res = BackendResult.from_code(self.lib.lib.redukt_backend_get_rwkv_state(
            slot, layer, _ptr(xa, ctypes.c_float), _ptr(wkv, ctypes.c_float), _ptr(xf, ctypes.c_float)))
        if res != BackendResult.OK:
            raise BackendError(res, "get_rwkv_state")
        return xa, wkv, xf

    def get_state(self, slot: int, layer: int, d_inner: int, d_conv: int, d_state: int = 16):
        conv = np.empty(d_inner * (d_conv - 1), np.float32)
        ssm = np.empty(d_inner * d_state, np.float32)
        res = BackendResult.from_code(self.lib.lib.redukt_backend_get_state(
            slot, layer, _ptr(conv, ctypes.c_float), _ptr(ssm, ctypes.c_float)))
        if res != BackendResult.OK:
            raise BackendError(res, "get_state")
        return conv, ssm

    def probe_kernel(self, kernel_class: int, events) -> None:
        """events: a ctypes array of c_void_p event handles (kept alive by the caller)."""
        res = BackendResult.from_code(self.lib.lib.redukt_backend_probe_kernel(
            kernel_class, ctypes.cast(events, ctypes.c_void_p) if events is not None else None,
            len(events) if events is not None else 0))
        if res != BackendResult.OK:
            raise BackendError(res, "probe_kernel")

    def probe_used(self) -> int:
        return int(self.lib.lib.redukt_backend_probe_used())

    def close(self) -> None:
        if not self._closed:
            self.lib.free()
            self._closed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
