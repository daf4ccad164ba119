"""Float64 RWKV-7 step, written from the model equations (not from the oracle's code), used
to pin the oracle: src/infrastructure/rwkv7/model.rs:643-925 in exact arithmetic up to
float64 rounding.  Matrix-vector products, norms and the WKV recurrence are numpy float64;
the transcendental functions are numpy's."""
from __future__ import annotations

import numpy as np


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _ln(x, w, b, eps=1e-5):
    mu = x.mean()
    var = ((x - mu) ** 2).mean()
    return (x - mu) / np.sqrt(var + eps) * w + b


def _round_away(x):
    return np.where(x < 0, -np.floor(-x + 0.5), np.floor(x + 0.5))


class _A8:
    """A per-row int8 matrix applied to an activation quantized with one scale per vector
    (src/domain/tensor.rs:1791-1866), in float64: q(v) = clamp(round(v * 127 / max|v|)),
    W v ~ (Wq q(v)) * s_row * max|v| / 127."""

    def __init__(self, q, scales):
        self.q = np.asarray(q, np.float64)
        self.s = np.asarray(scales, np.float64).reshape(-1)

    def __matmul__(self, v):
        amax = float(np.max(np.abs(v))) if v.size else 0.0
        scale = amax / 127.0 if amax > 0 else 1.0
        qv = np.clip(_round_away(v / scale), -127, 127)
        return (self.q @ qv) * self.s * scale


class F64Rwkv:
    def __init__(self, dims, tensors, mats=None, a8=None):
        """tensors: the file's f32 arrays; mats: optional replacements (float arrays) for the
        quantized matrices, e.g. their dequantized values; a8: optional {name: (int8 matrix,
        per-row scales)} applied with int8 activations instead."""
        self.dims = dims
        t = {k: np.asarray(v, np.float64) for k, v in tensors.items()}
        if mats:
            t.update({k: np.asarray(v, np.float64) for k, v in mats.items()})
        if a8:
            t.update({k: _A8(q, sc) for k, (q, sc) in a8.items()})
        self.t = t
        self.states = {}

    def _state(self, slot):
        d, L, H, N = self.dims.d_model, self.dims.n_layer, self.dims.n_head, self.dims.head_size
        if slot not in self.states:
            self.states[slot] = {"xa": np.zeros((L, d)), "xf": np.zeros((L, d)), "S": np.zeros((L, H, N, N)),
                                 "vf": np.zeros(d)}
        return self.states[slot]

    def reset(self, slot):
        self.states.pop(slot, None)

    def step(self, slot, token):
        D, t = self.dims, self.t
        H, N = D.n_head, D.head_size
        st = self._state(slot)
        x = t["emb"][token].copy()
        for i in range(D.n_layer):
            p = f"blocks.{i}."
            ln = _ln(x, t[p + "ln1_w"], t[p + "ln1_b"])
            xx = st["xa"][i] - ln
            mix = {c: ln + xx * t[p + "x_" + c] for c in "rwkvag"}
            r = t[p + "receptance"] @ mix["r"]
            k = t[p + "key"] @ mix["k"]
            v = t[p + "value"] @ mix["v"]
            w = np.exp(-0.606531 * _sig(t[p + "w0"] + t[p + "w2"] @ np.tanh(t[p + "w1"] @ mix["w"])))
            a = _sig(t[p + "a0"] + t[p + "a2"] @ (t[p + "a1"] @ mix["a"]))
            g = t[p + "g2"] @ _sig(t[p + "g1"] @ mix["g"])
            kk = (k * t[p + "k_k"]).reshape(H, N)
            nrm = np.sqrt((kk ** 2).sum(axis=1, keepdims=True))
            kk = np.where(nrm > 1e-12, kk / np.where(nrm > 1e-12, nrm, 1.0), 0.0).reshape(-1)
            kmod = k * (1.0 + (a - 1.0) * t[p + "k_a"])
            vout = v.copy()
            if i != 0:
                vout = v + (st["vf"] - v) * _sig(t[p + "v0"] + t[p + "v2"] @ (t[p + "v1"] @ mix["v"]))
            out = np.empty(D.d_model)
            for h in range(H):
                sl = slice(h * N, (h + 1) * N)
                S = st["S"][i, h]
                # S·diag(w) + S·(-kk)(kk*a)^T + v kmod^T, then S·r
                S = S * w[sl][None, :] + np.outer(S @ (-kk[sl]), kk[sl] * a[sl]) + np.outer(vout[sl], kmod[sl])
                st["S"][i, h] = S
                out[sl] = S @ r[sl]
            on = np.empty_like(out)
            for h in range(H):
                sl = slice(h * N, (h + 1) * N)
                on[sl] = _ln(out[sl], t[p + "ln_x_w"][sl], t[p + "ln_x_b"][sl], 64e-5)
                ksrc = kmod if D.g1k else k
                on[sl] += (r[sl] * ksrc[sl] * t[p + "r_k"][sl]).sum() * vout[sl]
            tm = t[p + "output"] @ (on * g)
            st["xa"][i] = ln
            if i == 0:
                st["vf"] = v
            x = x + tm
            ln2 = _ln(x, t[p + "ln2_w"], t[p + "ln2_b"])
            xk = ln2 + (st["xf"][i] - ln2) * t[p + "ffn_x_k"]
            h1 = np.maximum(t[p + "ffn_key"] @ xk, 0.0) ** 2
            x = x + t[p + "ffn_value"] @ h1
            st["xf"][i] = ln2
        return t["head"] @ _ln(x, t["ln_out_w"], t["ln_out_b"])
