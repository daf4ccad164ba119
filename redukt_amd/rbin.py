"""`.rbin` weight files: the flat F32 container redukt's GPU plugin reads.

Layout (scripts/convert-weights-gpu.py:43-53, 152-197 in the reference): a 44-byte
header of eleven little-endian u32 words — magic "RGPU" (0x55504752), version (1|2),
vocab, d_model, d_inner, d_state, d_conv, dt_rank, n_layer, flags (bit 0 LayerNorm
bias, bit 1 untied head), tokenizer (v2: 0 byte-level, 1 BPE; v1: reserved) — then the
f32 body: embedding [vocab, d_model], per layer (norm_w, [norm_b], in_proj, conv_w,
conv_b, x_proj, dt_proj_w, dt_proj_b, A_log, D, out_proj), norm_f_w, [norm_f_b],
[lm_head].  The host parses the same header (src/infrastructure/plugin_backend/
model.rs:157-168), so files written here are accepted by the unchanged Rust host.
"""
from __future__ import annotations

import dataclasses
import os
import struct
from typing import Iterable, Iterator, Optional, Tuple

import numpy as np

RBIN_MAGIC = 0x55504752
RBIN_HEADER_LEN = 44
HEADER_FMT = "<11I"
TOK_BYTE = 0
TOK_BPE = 1
FLAG_NORM_BIAS = 1 << 0
FLAG_UNTIED_HEAD = 1 << 1


@dataclasses.dataclass(frozen=True)
class MambaDims:
    vocab: int
    d_model: int
    n_layer: int
    d_state: int = 16
    d_conv: int = 4
    d_inner: int = 0
    dt_rank: int = 0

    def __post_init__(self):
        # MambaConfig::from_d_model (src/infrastructure/mamba/model.rs:34-45).
        if self.d_inner == 0:
            object.__setattr__(self, "d_inner", 2 * self.d_model)
        if self.dt_rank == 0:
            object.__setattr__(self, "dt_rank", (self.d_model + 15) // 16)

    @property
    def xr(self) -> int:
        return self.dt_rank + 2 * self.d_state


MAMBA_130M = MambaDims(vocab=50280, d_model=768, n_layer=24)


@dataclasses.dataclass(frozen=True)
class RbinMeta:
    """What `parse_rbin_header` of the host returns (plugin_backend/model.rs:129-136)."""
    version: int
    vocab_size: int
    tokenizer: Optional[int]


def pack_header(dims: MambaDims, version: int = 2, flags: int = 0, tokenizer: Optional[int] = None) -> bytes:
    if tokenizer is None:
        tokenizer = TOK_BYTE if dims.vocab == 256 else TOK_BPE
    word10 = tokenizer if version == 2 else 0
    return struct.pack(HEADER_FMT, RBIN_MAGIC, version, dims.vocab, dims.d_model, dims.d_inner, dims.d_state,
                       dims.d_conv, dims.dt_rank, dims.n_layer, flags, word10)


def parse_rbin_header(data: bytes) -> Optional[RbinMeta]:
    """Mirror of the host's `parse_rbin_header` (plugin_backend/model.rs:157-168):
    None on a short buffer, bad magic or a version other than 1/2."""
    if len(data) < RBIN_HEADER_LEN:
        return None
    w = struct.unpack_from(HEADER_FMT, data)
    if w[0] != RBIN_MAGIC:
        return None
    if w[1] == 1:
        tok = None
    elif w[1] == 2:
        tok = w[10]
    else:
        return None
    return RbinMeta(version=w[1], vocab_size=w[2], tokenizer=tok)


def rbin_path(weights: str) -> str:
    """Same path rule as the plugin and the host (plugin_backend/model.rs:171-177)."""
    return weights if weights.endswith(".rbin") else os.path.join(weights, "model.rbin")


def tensor_order(dims: MambaDims, flags: int = 0) -> Iterator[Tuple[str, Tuple[int, ...]]]:
    """Names and shapes of the body tensors in file order."""
    d, di, ds, dc, dr = dims.d_model, dims.d_inner, dims.d_state, dims.d_conv, dims.dt_rank
    yield "emb", (dims.vocab, d)
    for i in range(dims.n_layer):
        p = f"layers.{i}."
        yield p + "norm_w", (d,)
        if flags & FLAG_NORM_BIAS:
            yield p + "norm_b", (d,)
        yield p + "in_proj", (2 * di, d)
        yield p + "conv_w", (di, dc)
        yield p + "conv_b", (di,)
        yield p + "x_proj", (dr + 2 * ds, di)
        yield p + "dt_proj_w", (di, dr)
        yield p + "dt_proj_b", (di,)
        yield p + "A_log", (di, ds)
        yield p + "D", (di,)
        yield p + "out_proj", (d, di)
    yield "norm_f_w", (d,)
    if flags & FLAG_NORM_BIAS:
        yield "norm_f_b", (d,)
    if flags & FLAG_UNTIED_HEAD:
        yield "lm_head", (dims.vocab, d)


def write_rbin(path: str, dims: MambaDims, tensors: Iterable[Tuple[str, np.ndarray]], version: int = 2,
               flags: int = 0, tokenizer: Optional[int] = None) -> int:
    """Write header + tensors (which must come in `tensor_order`).  Returns bytes written."""
    expected = list(tensor_order(dims, flags))
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    n = 0
    with open(path, "wb") as f:
        f.write(pack_header(dims, version, flags, tokenizer))
        n += RBIN_HEADER_LEN
        for (name, shape), (tname, arr) in zip(expected, tensors, strict=True):
            if tname != name or tuple(arr.shape) != shape:
                raise ValueError(f"tensor {tname}{arr.shape} where {name}{shape} was expected")
            b = np.ascontiguousarray(arr, dtype="<f4").tobytes()
            f.write(b)
            n += len(b)
    return n


def read_rbin(path: str) -> Tuple[MambaDims, int, dict]:
    """Read a whole .rbin into a dict of float32 arrays (memory-mapped)."""
    with open(path, "rb") as f:
        w = struct.unpack(HEADER_FMT, f.read(RBIN_HEADER_LEN))
    if w[0] != RBIN_MAGIC or w[1] not in (1, 2):
        raise ValueError(f"{path}: not a .rbin v1/v2 file")
    dims = MambaDims(vocab=w[2], d_model=w[3], d_inner=w[4], d_state=w[5], d_conv=w[6], dt_rank=w[7], n_layer=w[8])
    flags = w[9]
    mm = np.memmap(path, dtype="<f4", mode="r", offset=RBIN_HEADER_LEN)
    out, off = {}, 0
    for name, shape in tensor_order(dims, flags):
        cnt = int(np.prod(shape))
        out[name] = np.asarray(mm[off:off + cnt]).reshape(shape)
        off += cnt
    if off != mm.size:
        raise ValueError(f"{path}: body has {mm.size} floats, header implies {off}")
    return dims, flags, out
