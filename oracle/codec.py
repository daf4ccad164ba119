"""Oracle of the host coding path (test infrastructure only: the tests, the smoke check and
the benchmark's CPU leg use it as the checker; nothing in the product imports it).

A numpy / pure-Python restatement, written independently of the C++ library it checks:

  exp_f64          src/domain/fmath.rs:340-430   table-driven double exp (7 table bits,
                   degree-5 polynomial); vectorised over numpy uint64 bit patterns
  cdf_from_logits  src/application/codec.rs:785-798   f64 softmax -> f32 probabilities
  cdf_from_probs   src/domain/coder.rs:43-81     2^24 total, min frequency 1, +0.5 rounding,
                   rounding error on the last maximal frequency
  cdf_uniform      src/domain/coder.rs:83-93
  lookup           src/domain/coder.rs:100-115
  RangeEncoder     src/domain/coder.rs:118-204   (pure Python, small inputs)
  RangeDecoder     src/domain/coder.rs:206-296

Sequential sums use np.cumsum, which adds left to right like the reference's loops (np.sum
would sum pairwise and round differently).

Pinning: exp_f64 by the reference's 24 golden bit patterns and special values
(fmath.rs:525-552, 610-622) and a correctly-rounded decimal bound; the table by its
decimal derivation; cdf_from_probs by closed forms (uniform probabilities give the uniform
CDF, a one-hot vector gives 2^24 - n + 1 to its symbol); the coder by the reference's round
trip, determinism and efficiency tests (coder.rs:302-470, codec.rs:2600-2651).
"""
from __future__ import annotations

import decimal
import struct
from typing import List, Sequence

import numpy as np

TOTAL = 1 << 24

# ---- exp ---------------------------------------------------------------------------------


def _bits(x: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def _from_bits(b: int) -> float:
    return struct.unpack("<d", struct.pack("<Q", b & 0xFFFFFFFFFFFFFFFF))[0]


def _derive_constants():
    ctx = decimal.Context(prec=70)
    ln2 = ctx.ln(decimal.Decimal(2))
    tail = np.empty(128, np.float64)
    head = np.empty(128, np.uint64)
    for k in range(128):
        v = ctx.exp(ctx.multiply(ctx.divide(decimal.Decimal(k), 128), ln2))
        h = float(v)
        tail[k] = float(ctx.subtract(ctx.divide(v, decimal.Decimal(h)), 1))
        head[k] = (_bits(h) - (k << 45)) & 0xFFFFFFFFFFFFFFFF
    ln2n = ctx.divide(ln2, 128)
    hi = _from_bits(_bits(float(ln2n)) & ~0xFFFF)
    lo = float(ctx.subtract(ln2n, decimal.Decimal(hi)))
    return float(1 / ln2) * 128.0, -hi, -lo, tail, head


INVLN2N, NEGLN2HIN, NEGLN2LON, TAIL, HEAD = _derive_constants()
# Minimax coefficients of e^r - 1 - r (orders 2..5) of the musl exp the reference restates
# (fmath.rs:113-118); they are not derivable by a short computation, so they are data.
C2, C3, C4, C5 = (_from_bits(b) for b in (0x3FDFFFFFFFFFFDBD, 0x3FC555555555543C, 0x3FA55555CF172B91,
                                          0x3F81111167A4D017))
SHIFT = 6755399441055744.0  # 1.5 * 2^52


def exp_f64(x) -> np.ndarray:
    """Elementwise; float64 in, float64 out, bit-identical to the reference's exp_f64."""
    x = np.atleast_1d(np.asarray(x, np.float64))
    out = np.empty_like(x)
    ix = x.view(np.uint64)
    abstop = ((ix >> np.uint64(52)) & np.uint64(0x7FF)).astype(np.int64)
    tiny = abstop < 0x3C9
    huge = abstop >= 0x409
    edge = (abstop >= 0x408) & ~huge
    with np.errstate(all="ignore"):
        out[tiny] = 1.0 + x[tiny]
        h = x[huge]
        hv = np.where(h > 0, np.inf, 0.0)
        hv = np.where(np.isnan(h) | (h == np.inf), 1.0 + h, hv)
        out[huge] = hv
        m = ~(tiny | huge)
        xm = x[m]
        z = INVLN2N * xm
        kd = z + SHIFT
        ki = kd.view(np.uint64).copy()
        kd = kd - SHIFT
        r = xm + kd * NEGLN2HIN + kd * NEGLN2LON
        idx = (ki & np.uint64(127)).astype(np.int64)
        sbits = HEAD[idx] + (ki << np.uint64(45))
        r2 = r * r
        tmp = TAIL[idx] + r + r2 * (C2 + r * C3) + r2 * r2 * (C4 + r * C5)
        res = sbits.view(np.float64) * 1.0
        res = res + res * tmp
        em = edge[m]
        if em.any():
            res[em] = [_exp_rescale(float(t), int(s), int(k)) for t, s, k in zip(tmp[em], sbits[em], ki[em])]
        out[m] = res
    return out


def _exp_rescale(tmp: float, sbits: int, ki: int) -> float:
    """Results near overflow or in the subnormal range (fmath.rs:352-379)."""
    if ki & 0x80000000 == 0:
        scale = _from_bits(sbits - (1009 << 52))
        return _from_bits((1009 + 1023) << 52) * (scale + scale * tmp)
    scale = _from_bits(sbits + (1022 << 52))
    y = scale + scale * tmp
    if y < 1.0:
        lo = scale - y + scale * tmp
        hi = 1.0 + y
        lo = 1.0 - hi + y + lo
        y = (hi + lo) - 1.0
        if y == 0.0:
            y = 0.0
    return _from_bits(1 << 52) * y


# ---- CDF ---------------------------------------------------------------------------------


def _seq_sum(a: np.ndarray) -> float:
    return float(np.cumsum(a, dtype=np.float64)[-1]) if a.size else 0.0


def cdf_from_probs(probs) -> np.ndarray:
    p = np.asarray(probs, np.float32)
    n = p.size
    assert 0 < n < TOTAL
    remaining = TOTAL - n
    sum_p = _seq_sum(p.astype(np.float64))
    inv = 1.0 / sum_p if sum_p > 0.0 else 0.0
    with np.errstate(invalid="ignore"):
        v = p.astype(np.float64) * inv * float(remaining) + 0.5
        extra = np.where(v > 0, np.trunc(np.nan_to_num(v, nan=0.0)), 0.0).astype(np.uint64)
    freqs = (extra + np.uint64(1)).astype(np.int64) & 0xFFFFFFFF
    diff = remaining - int(extra.sum(dtype=np.uint64))
    if diff != 0:
        at = n - 1 - int(np.argmax(freqs[::-1]))
        freqs[at] = (int(freqs[at]) + diff) & 0xFFFFFFFF
    cdf = np.zeros(n + 1, np.uint64)
    cdf[1:] = np.cumsum(freqs.astype(np.uint64)) & np.uint64(0xFFFFFFFF)
    return cdf.astype(np.uint32)


def cdf_uniform(n: int) -> np.ndarray:
    each = TOTAL // n
    return (np.arange(n + 1, dtype=np.uint64) * np.uint64(each)).astype(np.uint32)


def softmax_probs(logits) -> np.ndarray:
    """The f32 probability vector cdf_from_logits builds its CDF from."""
    l64 = np.asarray(logits, np.float32).astype(np.float64)
    finite = l64[~np.isnan(l64)]
    mx = float(finite.max()) if finite.size else -np.inf
    with np.errstate(all="ignore"):
        e = exp_f64(l64 - mx)
        s = _seq_sum(e)
        return (e * (1.0 / s)).astype(np.float32)


def cdf_from_logits(logits) -> np.ndarray:
    return cdf_from_probs(softmax_probs(logits))


def lookup(cdf: np.ndarray, cum: int) -> int:
    n = cdf.size - 1
    lo, hi = 0, n
    while lo < hi:
        mid = (lo + hi) // 2
        if int(cdf[mid + 1]) <= cum:
            lo = mid + 1
        else:
            hi = mid
    return lo


# ---- range coder -------------------------------------------------------------------------

M32 = 0xFFFFFFFF


class RangeEncoder:
    def __init__(self):
        self.low, self.range, self.cache, self.ff, self.first = 0, M32, 0, 0, True
        self.out = bytearray()

    def _shift_low(self):
        if (self.low & M32) < 0xFF000000 or (self.low >> 32) != 0:
            carry = (self.low >> 32) & 0xFF
            if not self.first:
                self.out.append((self.cache + carry) & 0xFF)
            self.first = False
            self.out.extend([(0xFF + carry) & 0xFF] * self.ff)
            self.ff = 0
            self.cache = (self.low >> 24) & 0xFF
        else:
            self.ff += 1
        self.low = (self.low & 0x00FFFFFF) << 8

    def encode(self, lo: int, hi: int, total: int):
        r = self.range // total
        self.low += lo * r
        self.range = (r * (hi - lo)) & M32 if hi < total else (self.range - ((r * lo) & M32)) & M32
        while self.range < TOTAL:
            self._shift_low()
            self.range = (self.range << 8) & M32

    def encode_symbol(self, s: int, cdf: np.ndarray):
        self.encode(int(cdf[s]), int(cdf[s + 1]), int(cdf[-1]))

    def finish(self) -> bytes:
        for _ in range(5):
            self._shift_low()
        if not self.first:
            self.out.append(self.cache)
            self.out.extend([0xFF] * self.ff)
        return bytes(self.out)


class RangeDecoder:
    def __init__(self, data: bytes):
        self.data, self.pos = bytes(data), 0
        self.low, self.range, self.code = 0, M32, 0
        for _ in range(4):
            self.code = ((self.code << 8) | self._next()) & M32

    def _next(self) -> int:
        if self.pos < len(self.data):
            self.pos += 1
            return self.data[self.pos - 1]
        return 0

    def decode_symbol(self, cdf: np.ndarray) -> int:
        total = int(cdf[-1])
        r = self.range // total
        if r == 0:
            raise ValueError("range underflow")
        cum = min(((self.code - self.low) & M32) // r, total - 1)
        s = lookup(cdf, cum)
        lo, hi = int(cdf[s]), int(cdf[s + 1])
        self.low = (self.low + r * lo) & M32
        self.range = (r * (hi - lo)) & M32 if hi < total else (self.range - r * lo) & M32
        while self.range < TOTAL:
            self.code = ((self.code << 8) | self._next()) & M32
            self.low = (self.low << 8) & M32
            self.range = (self.range << 8) & M32
        return s


def encode_tokens(cdfs: Sequence[np.ndarray], symbols: Sequence[int]) -> bytes:
    enc = RangeEncoder()
    for c, s in zip(cdfs, symbols):
        enc.encode_symbol(int(s), c)
    return enc.finish()


def decode_tokens(data: bytes, cdfs: Sequence[np.ndarray]) -> List[int]:
    dec = RangeDecoder(data)
    return [dec.decode_symbol(c) for c in cdfs]


def ideal_bits(cdfs: Sequence[np.ndarray], symbols: Sequence[int]) -> float:
    """Information content of the coded symbols under their CDFs, in bits: the length an
    ideal arithmetic coder reaches, which a range coder may exceed only by its flush."""
    return float(sum(-np.log2((int(c[s + 1]) - int(c[s])) / int(c[-1])) for c, s in zip(cdfs, symbols)))
