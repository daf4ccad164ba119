"""ctypes wrapper of the CPU oracle (liboracle.so built from this directory).

TEST INFRASTRUCTURE ONLY: parity checker and the timed CPU baseline.  Imported only by
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB names another build of the same sources (the tests use it to load a build
# with a planted mistake in a child process).
LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

# Profile bits of the Mamba oracle beyond the weight quantisation (oracle.h).
ORC_PROFILE_EXACT = 64   # accepted and ignored: the oracle always computes in the reference order
ORC_PROFILE_FMA = 128    # every GEMV in numeric contract 2 (fma-v1)

_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_lib = None


def build(force: bool = False) -> str:
    args = ["make", "-C", HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.isfile(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for name in ("orc_expf", "orc_lnf", "orc_lane_expf", "orc_sigmoidf", "orc_softplus"):
            getattr(L, name).argtypes = [ctypes.c_float]
            getattr(L, name).restype = ctypes.c_float
        L.orc_softmax_into.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.orc_dot_f32.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.orc_dot_f32.restype = ctypes.c_float
        L.orc_quantize.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i8p, _f32p,
                                   ctypes.POINTER(ctypes.c_int)]
        L.orc_gemv_f32.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p]
        L.orc_gemv_q8.argtypes = [_i8p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p]
        L.orc_dot_f32_fma.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.orc_dot_f32_fma.restype = ctypes.c_float
        L.orc_gemv_f32_fma.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p, _f32p]
        L.orc_gemv_q8_fma.argtypes = [_i8p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p]
        L.orc_rms_norm.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.orc_layer_norm.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.orc_ssm_d16.argtypes = [_f32p] * 8 + [ctypes.c_int]
        L.orc_mamba_load.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        L.orc_mamba_load.restype = ctypes.c_void_p
        L.orc_mamba_free.argtypes = [ctypes.c_void_p]
        L.orc_mamba_dims.argtypes = [ctypes.c_void_p, _u32p]
        L.orc_mamba_pool_init.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        L.orc_mamba_reset.argtypes = [ctypes.c_void_p, _u32p, ctypes.c_uint32]
        L.orc_mamba_set_reset_every.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        L.orc_mamba_forward.argtypes = [ctypes.c_void_p, ctypes.c_uint32, _u32p, _u32p, _f32p]
        L.orc_mamba_get_state.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p]
        L.orc_mamba_dequant.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, _f32p]
        L.orc_rwkv_load.argtypes = [ctypes.c_char_p, ctypes.c_int]
        L.orc_rwkv_load.restype = ctypes.c_void_p
        L.orc_rwkv_free.argtypes = [ctypes.c_void_p]
        L.orc_rwkv_dims.argtypes = [ctypes.c_void_p, _u32p]
        L.orc_rwkv_pool_init.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        L.orc_rwkv_reset.argtypes = [ctypes.c_void_p, _u32p, ctypes.c_uint32]
        L.orc_rwkv_set_reset_every.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        L.orc_rwkv_forward.argtypes = [ctypes.c_void_p, ctypes.c_uint32, _u32p, _u32p, _f32p]
        L.orc_rwkv_get_state.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p, _f32p]
        for name in ("orc_tanh_inplace", "orc_sigmoid_inplace"):
            getattr(L, name).argtypes = [_f32p, ctypes.c_int]
        for name in ("orc_sigmoid_add_into", "orc_decay_sigmoid_into"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, ctypes.c_int]
        L.orc_sigmoid_mix_inplace.argtypes = [_f32p, _f32p, _f32p, _f32p, ctypes.c_int]
        L.orc_group_norm_into.argtypes = [_f32p, _f32p, ctypes.c_int, _f32p, _f32p, ctypes.c_int, ctypes.c_float]
        L.orc_l2_normalize_per_head.argtypes = [_f32p, ctypes.c_int, ctypes.c_int]
        L.orc_mat_vec_small.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int]
        L.orc_wkv_head.argtypes = [_f32p, ctypes.c_int] + [_f32p] * 8
        L.orc_quantize_vec_i8.argtypes = [_f32p, ctypes.c_int, _i8p]
        L.orc_quantize_vec_i8.restype = ctypes.c_float
        L.orc_q8_matvec_a8.argtypes = [_i8p, _f32p, ctypes.c_int, ctypes.c_int, _i8p, ctypes.c_float, _f32p]
        L.orc_lane_sigmoidf.argtypes = [ctypes.c_float]
        L.orc_lane_sigmoidf.restype = ctypes.c_float
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_get_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray, ct=ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def f32c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- scalar / vector math ----
def expf(x: float) -> float:
    return lib().orc_expf(x)


def lnf(x: float) -> float:
    return lib().orc_lnf(x)


def lane_expf(x: float) -> float:
    return lib().orc_lane_expf(x)


def softplus(x: float) -> float:
    return lib().orc_softplus(x)


def sigmoidf(x: float) -> float:
    return lib().orc_sigmoidf(x)


def softmax(logits) -> np.ndarray:
    x = f32c(logits)
    out = np.empty_like(x)
    lib().orc_softmax_into(_p(x), _p(out), x.size)
    return out


def dot(w, v, fma: bool = False) -> float:
    """One dot product in the reference GEMV order, numeric contract 1 (or 2 with fma)."""
    w, v = f32c(w), f32c(v)
    return (lib().orc_dot_f32_fma if fma else lib().orc_dot_f32)(_p(w), _p(v), w.size)


def quantize(w, group: int):
    w = f32c(w)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    g_eff = group if (group > 0 and group % 8 == 0 and cols % group == 0) else cols
    sc = np.empty(rows * (cols // g_eff), np.float32)
    g = ctypes.c_int(0)
    lib().orc_quantize(_p(w), rows, cols, group, _p(q, ctypes.c_int8), _p(sc), ctypes.byref(g))
    return q, sc.reshape(rows, -1), g.value


def quantize_vec_i8(v):
    """quantize_vec_i8_into: (int8 vector, scale)."""
    v = f32c(v)
    q = np.empty(v.size, np.int8)
    sc = lib().orc_quantize_vec_i8(_p(v), v.size, _p(q, ctypes.c_int8))
    return q, np.float32(sc)


def q8_matvec_a8(q, scales, vq, v_scale) -> np.ndarray:
    """The W8A8 product of a per-row int8 matrix with an already quantized vector."""
    q = np.ascontiguousarray(q, np.int8)
    scales = f32c(scales).reshape(-1)
    vq = np.ascontiguousarray(vq, np.int8)
    out = np.empty(q.shape[0], np.float32)
    lib().orc_q8_matvec_a8(_p(q, ctypes.c_int8), _p(scales), q.shape[0], q.shape[1], _p(vq, ctypes.c_int8),
                           float(v_scale), _p(out))
    return out


def gemv_f32(w, v, fma: bool = False) -> np.ndarray:
    w, v = f32c(w), f32c(v)
    out = np.empty(w.shape[0], np.float32)
    (lib().orc_gemv_f32_fma if fma else lib().orc_gemv_f32)(_p(w), w.shape[0], w.shape[1], _p(v), _p(out))
    return out


def gemv_q8(q, scales, group: int, v, fma: bool = False) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    sc, v = f32c(scales), f32c(v)
    out = np.empty(q.shape[0], np.float32)
    (lib().orc_gemv_q8_fma if fma else lib().orc_gemv_q8)(_p(q, ctypes.c_int8), _p(sc), q.shape[0], q.shape[1],
                                                           group, _p(v), _p(out))
    return out


def rms_norm(x, w, eps: float = 1e-5) -> np.ndarray:
    x = f32c(x).copy()
    w = f32c(w)
    lib().orc_rms_norm(_p(x), _p(w), x.size, eps)
    return x


def layer_norm(x, w, b, eps: float = 1e-5) -> np.ndarray:
    x, w, b = f32c(x), f32c(w), f32c(b)
    out = np.empty_like(x)
    lib().orc_layer_norm(_p(out), _p(x), _p(w), _p(b), x.size, eps)
    return out


def ssm_d16(ss, dt, conv_out, a_log, b, c, d_vec):
    """One scan step; returns (y, new_state).  ss: [di,16]."""
    ss = f32c(ss).copy()
    dt, conv_out, a_log, b, c, d_vec = map(f32c, (dt, conv_out, a_log, b, c, d_vec))
    y = np.empty(dt.size, np.float32)
    lib().orc_ssm_d16(_p(y), _p(ss), _p(dt), _p(conv_out), _p(a_log), _p(b), _p(c), _p(d_vec), dt.size)
    return y, ss


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def get_threads() -> int:
    return lib().orc_get_threads()


class MambaOracle:
    """A Mamba model on the CPU oracle with a pool of `cap` stream slots."""

    def __init__(self, rbin_path: str, profile: int = 0, cap: int = 1):
        err = ctypes.c_int(0)
        self.h = lib().orc_mamba_load(rbin_path.encode(), profile, ctypes.byref(err))
        if not self.h:
            raise RuntimeError(f"oracle load failed ({err.value}): {rbin_path}")
        d = np.zeros(8, np.uint32)
        lib().orc_mamba_dims(self.h, _p(d, ctypes.c_uint32))
        self.vocab, self.d_model, self.d_inner, self.d_state, self.d_conv, self.dt_rank, self.n_layer, self.flags = \
            (int(x) for x in d)
        self.cap = 0
        self.pool_init(cap)

    def pool_init(self, cap: int) -> None:
        if lib().orc_mamba_pool_init(self.h, cap) != 0:
            raise MemoryError("oracle pool")
        self.cap = cap

    def set_reset_every(self, every: int) -> None:
        lib().orc_mamba_set_reset_every(self.h, every)

    def reset(self, slots: Optional[Sequence[int]] = None) -> None:
        if slots is None:
            lib().orc_mamba_reset(self.h, None, 0)
        else:
            s = np.ascontiguousarray(slots, dtype=np.uint32)
            if lib().orc_mamba_reset(self.h, _p(s, ctypes.c_uint32), s.size) != 0:
                raise ValueError("bad slot")

    def forward(self, slots: Sequence[int], tokens: Sequence[int]) -> np.ndarray:
        s = np.ascontiguousarray(slots, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty((s.size, self.vocab), np.float32)
        rc = lib().orc_mamba_forward(self.h, s.size, _p(s, ctypes.c_uint32), _p(t, ctypes.c_uint32), _p(out))
        if rc != 0:
            raise ValueError(f"oracle forward rc={rc}")
        return out

    def state(self, slot: int, layer: int):
        conv = np.empty(self.d_inner * (self.d_conv - 1), np.float32)
        ssm = np.empty(self.d_inner * self.d_state, np.float32)
        if lib().orc_mamba_get_state(self.h, slot, layer, _p(conv), _p(ssm)) != 0:
            raise ValueError("bad slot/layer")
        return conv, ssm

    def dequant(self, which: int, layer: int = 0) -> np.ndarray:
        shapes = {0: (2 * self.d_inner, self.d_model), 1: (self.d_model, self.d_inner), 2: (self.vocab, self.d_model),
                  3: (self.dt_rank + 2 * self.d_state, self.d_inner), 4: (self.d_inner, self.dt_rank)}
        out = np.empty(shapes[which], np.float32)
        if lib().orc_mamba_dequant(self.h, which, layer, _p(out)) != 0:
            raise ValueError("bad matrix")
        return out

    def close(self) -> None:
        if self.h:
            lib().orc_mamba_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RwkvOracle:
    """An RWKV-7 model on the CPU oracle with a pool of `cap` stream slots."""

    def __init__(self, path: str, profile: int = 0, cap: int = 1):
        self.h = lib().orc_rwkv_load(path.encode(), profile)
        if not self.h:
            raise RuntimeError(f"oracle load failed: {path}")
        d = np.zeros(11, np.uint32)
        lib().orc_rwkv_dims(self.h, _p(d, ctypes.c_uint32))
        (self.vocab, self.d_model, self.n_head, self.head_size, self.n_layer, self.d_ffn, self.lora_w, self.lora_a,
         self.lora_v, self.lora_g, self.g1k) = (int(x) for x in d)
        self.cap = 0
        self.pool_init(cap)

    def pool_init(self, cap: int) -> None:
        if lib().orc_rwkv_pool_init(self.h, cap) != 0:
            raise MemoryError("oracle pool")
        self.cap = cap

    def set_reset_every(self, every: int) -> None:
        lib().orc_rwkv_set_reset_every(self.h, every)

    def reset(self, slots: Optional[Sequence[int]] = None) -> None:
        if slots is None:
            lib().orc_rwkv_reset(self.h, None, 0)
        else:
            s = np.ascontiguousarray(slots, dtype=np.uint32)
            if lib().orc_rwkv_reset(self.h, _p(s, ctypes.c_uint32), s.size) != 0:
                raise ValueError("bad slot")

    def forward(self, slots: Sequence[int], tokens: Sequence[int]) -> np.ndarray:
        s = np.ascontiguousarray(slots, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty((s.size, self.vocab), np.float32)
        rc = lib().orc_rwkv_forward(self.h, s.size, _p(s, ctypes.c_uint32), _p(t, ctypes.c_uint32), _p(out))
        if rc != 0:
            raise ValueError(f"oracle forward rc={rc}")
        return out

    def state(self, slot: int, layer: int):
        d, hs = self.d_model, self.head_size
        xa, xf = np.empty(d, np.float32), np.empty(d, np.float32)
        wkv = np.empty((self.n_head, hs, hs), np.float32)
        if lib().orc_rwkv_get_state(self.h, slot, layer, _p(xa), _p(wkv), _p(xf)) != 0:
            raise ValueError("bad slot/layer")
        return xa, wkv, xf

    def close(self) -> None:
        if self.h:
            lib().orc_rwkv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

