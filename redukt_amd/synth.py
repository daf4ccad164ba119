"""Seeded synthetic Mamba weights and token streams.

No trained weights travel with this repository, so every measurement and parity test
runs on seeded random weights of the real architecture.  Two initialisations:

* ``"baseline"`` — the measurement workload: projections (in_proj, x_proj, dt_proj,
  out_proj, the tied embedding/head) ~ N(0, 0.02); conv1d weight and bias ~
  U(-1/sqrt(d_conv), 1/sqrt(d_conv)) (the PyTorch Conv1d default the reference model was
  trained from; the workload description leaves conv unspecified); norm weights 1;
  A_log[j][n] = ln(n+1); D = 1; dt_bias the inverse softplus of dt with
  ln(dt) ~ U(ln 1e-3, ln 0.1).
* ``"reference-test"`` — the weight-free model of the reference's unit tests
  (src/infrastructure/mamba/model.rs:1036-1082): xorshift32 uniforms with the same seeds,
  amplitudes and offsets, so the lockstep bit-identity test runs on the same model.

Token ids are Zipf(s) over the vocabulary (rank r has weight r^-s, id = r - 1),
independent per stream, or uniform.
"""
from __future__ import annotations

import hashlib
from typing import Iterator, Tuple

import numpy as np

from .rbin import FLAG_NORM_BIAS, FLAG_UNTIED_HEAD, MambaDims, tensor_order, write_rbin


def _baseline_tensors(dims: MambaDims, seed: int, flags: int) -> Iterator[Tuple[str, np.ndarray]]:
    rng = np.random.default_rng(seed)
    f32 = np.float32
    conv_bound = 1.0 / np.sqrt(dims.d_conv)

    def normal(shape):
        return rng.standard_normal(shape, dtype=f32) * f32(0.02)

    def uniform(shape, lo, hi):
        return rng.uniform(lo, hi, size=shape).astype(f32)

    a_log = np.log(np.arange(1, dims.d_state + 1, dtype=np.float64)).astype(f32)
    for name, shape in tensor_order(dims, flags):
        leaf = name.rsplit(".", 1)[-1]
        if leaf in ("emb", "in_proj", "x_proj", "dt_proj_w", "out_proj", "lm_head"):
            t = normal(shape)
        elif leaf in ("norm_w", "norm_f_w", "D"):
            t = np.ones(shape, f32)
        elif leaf in ("norm_b", "norm_f_b"):
            t = np.zeros(shape, f32)
        elif leaf == "conv_w" or leaf == "conv_b":
            t = uniform(shape, -conv_bound, conv_bound)
        elif leaf == "dt_proj_b":
            dt = np.exp(rng.uniform(np.log(1e-3), np.log(0.1), size=shape))
            t = (dt + np.log(-np.expm1(-dt))).astype(f32)
        elif leaf == "A_log":
            t = np.broadcast_to(a_log, shape).copy()
        else:
            raise AssertionError(name)
        yield name, t


def xorshift_vec(n: int, seed: int, amp: float) -> np.ndarray:
    """`rand_vec` of the reference tests (mamba/model.rs:1036-1044): xorshift32 state,
    ((st as f32 / u32::MAX as f32) * 2 - 1) * amp, all in f32."""
    st = max(seed, 1) & 0xFFFFFFFF
    raw = np.empty(n, np.uint32)
    for i in range(n):
        st ^= (st << 13) & 0xFFFFFFFF
        st ^= st >> 17
        st ^= (st << 5) & 0xFFFFFFFF
        raw[i] = st
    f32 = np.float32
    return ((raw.astype(f32) / f32(4294967295.0)) * f32(2.0) - f32(1.0)) * f32(amp)


def _reference_test_tensors(dims: MambaDims, flags: int) -> Iterator[Tuple[str, np.ndarray]]:
    if flags:
        raise ValueError("the reference test model has RMSNorm and a tied head")
    d, di, ds, dc, dr, V = dims.d_model, dims.d_inner, dims.d_state, dims.d_conv, dims.dt_rank, dims.vocab
    seed = [1000]

    def nxt():
        seed[0] += 17
        return seed[0]

    f32 = np.float32
    layers = []
    for _ in range(dims.n_layer):
        L = {}
        L["norm_w"] = f32(1.0) + xorshift_vec(d, nxt(), 0.5)
        L["in_proj"] = xorshift_vec(2 * di * d, nxt(), 0.3).reshape(2 * di, d)
        L["conv_w"] = xorshift_vec(di * dc, nxt(), 0.5).reshape(di, dc)
        L["conv_b"] = xorshift_vec(di, nxt(), 0.1)
        L["x_proj"] = xorshift_vec((dr + 2 * ds) * di, nxt(), 0.2).reshape(dr + 2 * ds, di)
        L["dt_proj_w"] = xorshift_vec(di * dr, nxt(), 0.5).reshape(di, dr)
        L["dt_proj_b"] = xorshift_vec(di, nxt(), 1.0) - f32(2.0)
        L["A_log"] = np.abs(xorshift_vec(di * ds, nxt(), 1.0)).reshape(di, ds)
        L["D"] = xorshift_vec(di, nxt(), 1.0)
        L["out_proj"] = xorshift_vec(d * di, nxt(), 0.2).reshape(d, di)
        layers.append(L)
    emb = xorshift_vec(V * d, nxt(), 1.0).reshape(V, d)
    norm_f = f32(1.0) + xorshift_vec(d, nxt(), 0.5)
    for name, _shape in tensor_order(dims, flags):
        if name == "emb":
            yield name, emb
        elif name == "norm_f_w":
            yield name, norm_f
        else:
            i, leaf = name.split(".")[1], name.split(".")[2]
            yield name, layers[int(i)][leaf]


def mamba_tensors(dims: MambaDims, seed: int = 0, init: str = "baseline", flags: int = 0):
    if init == "baseline":
        return _baseline_tensors(dims, seed, flags)
    if init == "reference-test":
        return _reference_test_tensors(dims, flags)
    raise ValueError(f"unknown init {init!r}")


def write_synthetic_mamba(path: str, dims: MambaDims, seed: int = 0, init: str = "baseline", flags: int = 0,
                          version: int = 2) -> str:
    """Write a seeded synthetic model; returns the SHA-256 of the file."""
    write_rbin(path, dims, mamba_tensors(dims, seed, init, flags), version=version, flags=flags)
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 22), b""):
            h.update(chunk)
    return h.hexdigest()


def zipf_tokens(rng: np.random.Generator, vocab: int, shape, s: float = 1.1) -> np.ndarray:
    """Token ids with P(id = r-1) proportional to r^-s, by inverse-CDF sampling."""
    w = np.arange(1, vocab + 1, dtype=np.float64) ** -s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = rng.random(size=shape)
    ids = np.searchsorted(cdf, u, side="right")
    return np.minimum(ids, vocab - 1).astype(np.uint32)


def uniform_tokens(rng: np.random.Generator, vocab: int, shape) -> np.ndarray:
    return rng.integers(0, vocab, size=shape, dtype=np.uint32)


__all__ = ["mamba_tensors", "write_synthetic_mamba", "zipf_tokens", "uniform_tokens", "xorshift_vec",
           "FLAG_NORM_BIAS", "FLAG_UNTIED_HEAD"]
