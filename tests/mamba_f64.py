"""Float64 Mamba-1 step written from the model's equations with numpy matrix algebra.

Test helper: an independent brute-force check of the oracle's structure (operand
orientation, the x/z split of in_proj, the conv shift register, the dt/B/C split of
x_proj, the discretisation, the D skip and the gate).  It shares no code and no
operation order with the oracle; agreement to ~1e-6 relative pins the structure,
while the oracle's f32 operation order is pinned separately by order-sensitive cases.
"""
import numpy as np


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _softplus(v):
    return np.where(v > 20.0, v, np.log1p(np.exp(np.minimum(v, 20.0))))


class F64Mamba:
    def __init__(self, dims, tensors, flags=0, overrides=None):
        """tensors: dict from rbin.read_rbin / synth; overrides: name -> array (e.g.
        dequantized Q8 matrices)."""
        self.dims = dims
        self.flags = flags
        t = dict(tensors)
        if overrides:
            t.update(overrides)
        self.t = {k: np.asarray(v, np.float64) for k, v in t.items()}
        self.head = self.t["lm_head"] if (flags & 2) else self.t["emb"]
        self.reset()

    def reset(self):
        d = self.dims
        self.conv = [np.zeros((d.d_inner, d.d_conv - 1)) for _ in range(d.n_layer)]
        self.ssm = [np.zeros((d.d_inner, d.d_state)) for _ in range(d.n_layer)]

    def _norm(self, x, w, b):
        if b is None:
            return x / np.sqrt(np.mean(x * x) + 1e-5) * w
        m = x.mean()
        return (x - m) / np.sqrt(np.mean((x - m) ** 2) + 1e-5) * w + b

    def step(self, tok):
        d, t = self.dims, self.t
        di, ds, dr = d.d_inner, d.d_state, d.dt_rank
        x = t["emb"][tok].copy()
        for i in range(d.n_layer):
            p = f"layers.{i}."
            h = self._norm(x, t[p + "norm_w"], t.get(p + "norm_b"))
            xz = t[p + "in_proj"] @ h
            xb, z = xz[:di], xz[di:]
            window = np.concatenate([self.conv[i], xb[:, None]], axis=1)   # oldest .. newest
            v = (window * t[p + "conv_w"]).sum(axis=1) + t[p + "conv_b"]
            self.conv[i] = window[:, 1:]
            u = _silu(v)
            zp = t[p + "x_proj"] @ u
            dt = _softplus(t[p + "dt_proj_w"] @ zp[:dr] + t[p + "dt_proj_b"])
            B, C = zp[dr:dr + ds], zp[dr + ds:dr + 2 * ds]
            upd = np.abs(dt) >= 1e-6                                       # dt-sparse skip
            dA = np.exp(-dt[:, None] * np.exp(t[p + "A_log"]))
            new = dA * self.ssm[i] + (dt * u)[:, None] * B[None, :]
            self.ssm[i] = np.where(upd[:, None], new, self.ssm[i])
            y = self.ssm[i] @ C + t[p + "D"] * u
            x = x + t[p + "out_proj"] @ (y * _silu(z))
        hf = self._norm(x, t["norm_f_w"], t.get("norm_f_b"))
        return self.head @ hf
