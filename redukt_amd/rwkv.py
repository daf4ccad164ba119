"""RWKV-7 weights for libredukt_gpu.so: file format, synthetic models, safetensors import.

The Mamba `.rbin` header cannot describe RWKV-7, so RWKV files extend it: the same magic
"RGPU" with version 3 and a model word.  The host's `parse_rbin_header`
(src/infrastructure/plugin_backend/model.rs:157-168) treats version 3 as "no metadata"
and falls back to choosing the tokenizer by vocabulary size, so such a file never changes
what the unchanged host does with Mamba files.

Header: sixteen little-endian u32 words —
  0 magic 0x55504752, 1 version 3, 2 model (2 = RWKV-7), 3 vocab, 4 d_model, 5 n_head,
  6 head_size, 7 n_layer, 8 d_ffn, 9 decay LoRA rank, 10 a LoRA rank, 11 v LoRA rank,
  12 g LoRA rank, 13 flags (bit 0: the bonus term uses the modified key, `g1k`),
  14 tokenizer (0 byte-level, 1 BPE), 15 reserved 0.
Body: f32 tensors in `tensor_order`.  The embedding is stored already passed through the
first block's ln0 LayerNorm and the LoRA matrices are stored as `matrix @ vector`
([out, in]); both are what the reference does at load (src/infrastructure/rwkv7/
model.rs:246-275, 1004-1020), so a converted file holds exactly the tensors the reference
computes with.
"""
from __future__ import annotations

import dataclasses
import os
import struct
from typing import Dict, Iterator, Optional, Tuple

import numpy as np

from .rbin import RBIN_MAGIC

RWKV_VERSION = 3
MODEL_RWKV7 = 2
HEADER_FMT = "<16I"
HEADER_LEN = 64
FLAG_G1K = 1 << 0
LN_EPS = 1e-5


@dataclasses.dataclass(frozen=True)
class RwkvDims:
    vocab: int
    d_model: int
    n_layer: int
    head_size: int = 64
    d_ffn: int = 0
    lora_w: int = 64
    lora_a: int = 64
    lora_v: int = 32
    lora_g: int = 128
    g1k: bool = False

    def __post_init__(self):
        if self.d_ffn == 0:
            object.__setattr__(self, "d_ffn", 4 * self.d_model)
        if self.d_model % self.head_size:
            raise ValueError("d_model must be a multiple of head_size")

    @property
    def n_head(self) -> int:
        return self.d_model // self.head_size


# RWKV-7 0.1B (Rwkv7Config::default_0_1b, rwkv7/model.rs:24-26; BlinkDL 0.1B LoRA ranks).
RWKV7_0_1B = RwkvDims(vocab=65536, d_model=768, n_layer=12)


def pack_header(dims: RwkvDims, tokenizer: int = 0) -> bytes:
    return struct.pack(HEADER_FMT, RBIN_MAGIC, RWKV_VERSION, MODEL_RWKV7, dims.vocab, dims.d_model, dims.n_head,
                       dims.head_size, dims.n_layer, dims.d_ffn, dims.lora_w, dims.lora_a, dims.lora_v, dims.lora_g,
                       FLAG_G1K if dims.g1k else 0, tokenizer, 0)


def parse_header(data: bytes) -> Optional[RwkvDims]:
    if len(data) < HEADER_LEN:
        return None
    w = struct.unpack_from(HEADER_FMT, data)
    if w[0] != RBIN_MAGIC or w[1] != RWKV_VERSION or w[2] != MODEL_RWKV7 or w[4] != w[5] * w[6]:
        return None
    return RwkvDims(vocab=w[3], d_model=w[4], n_layer=w[7], head_size=w[6], d_ffn=w[8], lora_w=w[9], lora_a=w[10],
                    lora_v=w[11], lora_g=w[12], g1k=bool(w[13] & FLAG_G1K))


def tensor_order(dims: RwkvDims) -> Iterator[Tuple[str, Tuple[int, ...]]]:
    d, f = dims.d_model, dims.d_ffn
    yield "emb", (dims.vocab, d)
    for i in range(dims.n_layer):
        p = f"blocks.{i}."
        for name in ("ln1_w", "ln1_b", "ln2_w", "ln2_b", "x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0"):
            yield p + name, (d,)
        yield p + "w1", (dims.lora_w, d)
        yield p + "w2", (d, dims.lora_w)
        yield p + "a0", (d,)
        yield p + "a1", (dims.lora_a, d)
        yield p + "a2", (d, dims.lora_a)
        yield p + "v0", (d,)
        yield p + "v1", (dims.lora_v, d)
        yield p + "v2", (d, dims.lora_v)
        yield p + "g1", (dims.lora_g, d)
        yield p + "g2", (d, dims.lora_g)
        for name in ("k_k", "k_a", "r_k"):
            yield p + name, (d,)
        for name in ("receptance", "key", "value", "output"):
            yield p + name, (d, d)
        yield p + "ln_x_w", (d,)
        yield p + "ln_x_b", (d,)
        yield p + "ffn_x_k", (d,)
        yield p + "ffn_key", (f, d)
        yield p + "ffn_value", (d, f)
    yield "ln_out_w", (d,)
    yield "ln_out_b", (d,)
    yield "head", (dims.vocab, d)


def file_bytes(dims: RwkvDims) -> int:
    return HEADER_LEN + 4 * sum(int(np.prod(s)) for _, s in tensor_order(dims))


def write_rwkv(path: str, dims: RwkvDims, tensors: Dict[str, np.ndarray], tokenizer: int = 0) -> None:
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "wb") as f:
        f.write(pack_header(dims, tokenizer))
        for name, shape in tensor_order(dims):
            a = tensors[name]
            if tuple(a.shape) != shape:
                raise ValueError(f"{name}: shape {a.shape}, expected {shape}")
            f.write(np.ascontiguousarray(a, dtype="<f4").tobytes())


def read_rwkv(path: str) -> Tuple[RwkvDims, Dict[str, np.ndarray]]:
    with open(path, "rb") as f:
        dims = parse_header(f.read(HEADER_LEN))
    if dims is None:
        raise ValueError(f"{path}: not an RWKV-7 weight file")
    mm = np.memmap(path, dtype="<f4", mode="r", offset=HEADER_LEN)
    out, off = {}, 0
    for name, shape in tensor_order(dims):
        cnt = int(np.prod(shape))
        out[name] = np.asarray(mm[off:off + cnt]).reshape(shape)
        off += cnt
    if off != mm.size:
        raise ValueError(f"{path}: body has {mm.size} floats, header implies {off}")
    return dims, out


def layer_norm_rows(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = LN_EPS) -> np.ndarray:
    """`layer_norm` (src/domain/tensor.rs:721-732) row by row in f32: sequential sums,
    mean, variance, (x - mean) * inv_std * w + b."""
    x = np.asarray(x, np.float32)
    out = np.empty_like(x)
    n = np.float32(x.shape[-1])
    for r in range(x.shape[0]):
        row = x[r]
        s = np.float32(0)
        for v in row:
            s = np.float32(s + v)
        mean = np.float32(s / n)
        c = (row - mean).astype(np.float32)
        q = np.float32(0)
        for v in c:
            q = np.float32(q + np.float32(v * v))
        inv = np.float32(np.float32(1.0) / np.sqrt(np.float32(np.float32(q / n) + np.float32(eps))))
        out[r] = ((c * inv).astype(np.float32) * w).astype(np.float32) + b
    return out


def synthetic(dims: RwkvDims, seed: int = 0) -> Dict[str, np.ndarray]:
    """Seeded random-init RWKV-7: projections and LoRAs N(0, 0.02); decay base w0 so that
    exp(-0.606531 * sigmoid(w0)) lies in (0.9, 0.999); token-shift mixes U(0, 1); norms
    weight 1, bias 0; embedding rows passed through a unit ln0."""
    rng = np.random.default_rng(seed)
    d, f = dims.d_model, dims.d_ffn

    def normal(shape, std=0.02):
        return rng.normal(0.0, std, size=shape).astype(np.float32)

    t: Dict[str, np.ndarray] = {}
    emb = normal((dims.vocab, d), 1.0)
    ones, zeros = np.ones(d, np.float32), np.zeros(d, np.float32)
    # ln0 applied at load (rwkv7/model.rs:266-273); unit weight, zero bias.  Vectorised
    # here: the synthetic rows only need to be normalised, not bit-identical to a
    # sequential sum.
    mu = emb.mean(axis=1, keepdims=True, dtype=np.float64)
    var = ((emb - mu) ** 2).mean(axis=1, keepdims=True)
    t["emb"] = ((emb - mu) / np.sqrt(var + LN_EPS)).astype(np.float32)
    # decay in (0.9, 0.999)  <=>  sigmoid(w0) in (0.00165, 0.1737)  <=>  w0 in (-6.41, -1.56)
    for i in range(dims.n_layer):
        p = f"blocks.{i}."
        t[p + "ln1_w"], t[p + "ln1_b"] = ones.copy(), zeros.copy()
        t[p + "ln2_w"], t[p + "ln2_b"] = ones.copy(), zeros.copy()
        for name in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            t[p + name] = rng.uniform(0.0, 1.0, d).astype(np.float32)
        t[p + "w0"] = rng.uniform(-6.0, -2.0, d).astype(np.float32)
        t[p + "w1"], t[p + "w2"] = normal((dims.lora_w, d)), normal((d, dims.lora_w))
        t[p + "a0"] = rng.normal(0.0, 1.0, d).astype(np.float32)
        t[p + "a1"], t[p + "a2"] = normal((dims.lora_a, d)), normal((d, dims.lora_a))
        t[p + "v0"] = rng.normal(0.0, 1.0, d).astype(np.float32)
        t[p + "v1"], t[p + "v2"] = normal((dims.lora_v, d)), normal((d, dims.lora_v))
        t[p + "g1"], t[p + "g2"] = normal((dims.lora_g, d)), normal((d, dims.lora_g))
        t[p + "k_k"] = rng.uniform(0.5, 1.5, d).astype(np.float32)
        t[p + "k_a"] = rng.uniform(0.0, 1.0, d).astype(np.float32)
        t[p + "r_k"] = normal(d, 0.1)
        for name in ("receptance", "key", "value", "output"):
            t[p + name] = normal((d, d))
        t[p + "ln_x_w"], t[p + "ln_x_b"] = ones.copy(), zeros.copy()
        t[p + "ffn_x_k"] = rng.uniform(0.0, 1.0, d).astype(np.float32)
        t[p + "ffn_key"], t[p + "ffn_value"] = normal((f, d)), normal((d, f))
    t["ln_out_w"], t["ln_out_b"] = ones.copy(), zeros.copy()
    t["head"] = normal((dims.vocab, d))
    return t


def write_synthetic(path: str, dims: RwkvDims, seed: int = 0) -> None:
    write_rwkv(path, dims, synthetic(dims, seed), tokenizer=0)


def from_blinkdl(tensors: Dict[str, np.ndarray], n_layer: int, head_size: int = 64, g1k: bool = False
                 ) -> Tuple[RwkvDims, Dict[str, np.ndarray]]:
    """BlinkDL RWKV-7 tensors (safetensors key names, rwkv7/model.rs:997-1059) to this
    format: ln0 applied to the embedding rows in the reference's order, LoRAs transposed
    to [out, in], v0/v1/v2 of blocks without them taken from a0/a1/a2 as the reference
    does, r_k flattened."""
    g = lambda k: np.asarray(tensors[k], np.float32)  # noqa: E731
    emb_raw = g("emb.weight")
    vocab, d = emb_raw.shape
    out: Dict[str, np.ndarray] = {}
    out["emb"] = layer_norm_rows(emb_raw, g("blocks.0.ln0.weight"), g("blocks.0.ln0.bias"))
    a = "blocks.0.att."
    dims = RwkvDims(vocab=vocab, d_model=d, n_layer=n_layer, head_size=head_size,
                    d_ffn=g("blocks.0.ffn.key.weight").shape[0], lora_w=g(a + "w1").shape[1],
                    lora_a=g(a + "a1").shape[1],
                    lora_v=g("blocks.1.att.v1").shape[1] if n_layer > 1 and "blocks.1.att.v1" in tensors
                    else g(a + "a1").shape[1],
                    lora_g=g(a + "g1").shape[1], g1k=g1k)
    for i in range(n_layer):
        att, ffn, blk, p = f"blocks.{i}.att.", f"blocks.{i}.ffn.", f"blocks.{i}.", f"blocks.{i}."
        out[p + "ln1_w"], out[p + "ln1_b"] = g(blk + "ln1.weight"), g(blk + "ln1.bias")
        out[p + "ln2_w"], out[p + "ln2_b"] = g(blk + "ln2.weight"), g(blk + "ln2.bias")
        for name in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "a0", "k_k", "k_a"):
            out[p + name] = g(att + name).reshape(-1)
        for name in ("w1", "w2", "a1", "a2", "g1", "g2"):
            out[p + name] = np.ascontiguousarray(g(att + name).T)
        has_v = (att + "v0") in tensors
        out[p + "v0"] = g(att + ("v0" if has_v else "a0")).reshape(-1)
        v1 = g(att + ("v1" if has_v else "a1")).T
        v2 = g(att + ("v2" if has_v else "a2")).T
        if v1.shape[0] != dims.lora_v:    # a layer without v LoRA stored at the v rank
            v1 = np.zeros((dims.lora_v, d), np.float32)
            v2 = np.zeros((d, dims.lora_v), np.float32)
        out[p + "v1"], out[p + "v2"] = np.ascontiguousarray(v1), np.ascontiguousarray(v2)
        out[p + "r_k"] = g(att + "r_k").reshape(-1)
        for name in ("receptance", "key", "value", "output"):
            out[p + name] = g(att + name + ".weight")
        out[p + "ln_x_w"], out[p + "ln_x_b"] = g(att + "ln_x.weight"), g(att + "ln_x.bias")
        out[p + "ffn_x_k"] = g(ffn + "x_k").reshape(-1)
        out[p + "ffn_key"], out[p + "ffn_value"] = g(ffn + "key.weight"), g(ffn + "value.weight")
    out["ln_out_w"], out["ln_out_b"] = g("ln_out.weight"), g("ln_out.bias")
    out["head"] = g("head.weight")
    return dims, out
