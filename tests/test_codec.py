"""Host coding path: the oracle pinned against the reference's known answers and closed
forms, then libredukt_host.so held bit-exact to the oracle.

Known answers used as fixtures: the 24 exp golden bit patterns and special values
(src/domain/fmath.rs:525-552, 610-622), the ≤ 1 ulp sweep against the platform exp
(fmath.rs:624-645, here against math.exp over the same two input bands), and the coder's
round-trip / efficiency / corruption tests (src/domain/coder.rs:302-470) and determinism
tests (src/application/codec.rs:2600-2651)."""
import decimal
import io
import math
import os
import struct
import sys

import numpy as np
import pytest

from oracle import codec as O
from redukt_amd import codec as C

HERE = os.path.dirname(os.path.abspath(__file__))
HOST_DIR = os.path.join(HERE, "..", "redukt_amd", "csrc", "host")

# (input bits, exp output bits), fmath.rs:529-554
EXP_GOLDEN = [
    (0x0000000000000000, 0x3ff0000000000000), (0x8000000000000000, 0x3ff0000000000000),
    (0x3ff0000000000000, 0x4005bf0a8b145769), (0xbff0000000000000, 0x3fd78b56362cef38),
    (0x3fe0000000000000, 0x3ffa61298e1e069c), (0xbfe0000000000000, 0x3fe368b2fc6f960a),
    (0x3ddb7cdfd9d7bdbb, 0x3ff000000006df38), (0x3c670ef54646d497, 0x3ff0000000000000),
    (0x3fe62e42fefa39ef, 0x4000000000000000), (0x4008000000000000, 0x403415e5bf6fb106),
    (0xc0026bb1bbb55516, 0x3fb9999999999998), (0xc01d000000000000, 0x3f47455fe323fafd),
    (0xc034000000000000, 0x3e21b48655f37267), (0xc042c00000000000, 0x3c8dd5c566301ec8),
    (0xc04e000000000000, 0x3a85ae191a99585a), (0xc059000000000000, 0x36ea8c1f14e2af5d),
    (0xc085e00000000000, 0x00d14f2b0fb9307f), (0xc086240000000000, 0x000e6cf6d08897ac),
    (0xc087480000000000, 0x0000000000000001), (0xc087500000000000, 0x0000000000000000),
    (0x4086280000000000, 0x7fdd422d2be5dc9b), (0x4086300000000000, 0x7ff0000000000000),
    (0xbf60000000000000, 0x3feff003ff556aa9), (0xc028b0fcb4f1e4b4, 0x3ed23d2c7da10725),
]


def f64(b):
    return struct.unpack("<d", struct.pack("<Q", b))[0]


def bits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def xorshift_units(seed, n):
    """The reference tests' XorShift64 (fmath.rs:587-598): (next >> 11) / 2^53."""
    out = np.empty(n, np.float64)
    s = seed
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        out[i] = (s >> 11) / float(1 << 53)
    return out


def sweep_inputs(n=1 << 16):
    u = xorshift_units(0x9E3779B97F4A7C15, n)
    x = np.where(np.arange(n) % 2 == 0, -60.0 * u, -745.0 + 1455.0 * u)
    return x


def ulp_diff(a, b):
    ka = np.asarray(a, np.float64).view(np.int64)
    kb = np.asarray(b, np.float64).view(np.int64)
    ka = np.where(ka < 0, np.int64(-(2 ** 63)) - ka, ka)
    kb = np.where(kb < 0, np.int64(-(2 ** 63)) - kb, kb)
    return np.abs(ka - kb)


# ---- the oracle's exp against the reference's known answers and the mathematics -------------

def test_oracle_exp_golden_bits():
    x = np.array([g for g, _ in EXP_GOLDEN], np.uint64).view(np.float64)
    got = O.exp_f64(x).view(np.uint64)
    want = np.array([w for _, w in EXP_GOLDEN], np.uint64)
    bad = [(hex(g), hex(int(a)), hex(w)) for (g, w), a in zip(EXP_GOLDEN, got) if int(a) != w]
    assert not bad, bad


def test_oracle_exp_special_values():
    v = O.exp_f64([-np.inf, np.inf, np.nan, 1000.0, -1000.0])
    assert v[0] == 0.0 and v[1] == np.inf and np.isnan(v[2]) and v[3] == np.inf
    assert bits(float(v[4])) == 0


def test_oracle_exp_within_one_ulp_of_platform_exp():
    x = sweep_inputs()
    ref = np.array([math.exp(t) if t < 709.78 else math.inf for t in x])
    assert int(ulp_diff(O.exp_f64(x), ref).max()) <= 1


def test_oracle_exp_correctly_rounded_bound():
    """|exp_f64(x) - e^x| < 0.52 ulp against 60-digit decimal e^x; a wrong table entry,
    polynomial coefficient or reduction constant breaks this by whole ulps."""
    ctx = decimal.Context(prec=60)
    rng = np.random.default_rng(5)
    x = np.concatenate([-60.0 * rng.random(1500), rng.uniform(-700, 700, 500), rng.uniform(-0.01, 0.01, 200)])
    got = O.exp_f64(x)
    worst = 0.0
    for xi, gi in zip(x, got):
        true = ctx.exp(decimal.Decimal(float(xi)))
        ulp = math.ulp(float(gi))
        err = abs(decimal.Decimal(float(gi)) - true) / decimal.Decimal(ulp)
        worst = max(worst, float(err))
    assert worst < 0.52, worst


def test_exp_table_header_is_its_generator_output():
    sys.path.insert(0, HOST_DIR)
    try:
        import gen_exp_table
    finally:
        sys.path.pop(0)
    buf = io.StringIO()
    gen_exp_table.main(buf)
    with open(os.path.join(HOST_DIR, "exp_table.h")) as f:
        assert f.read() == buf.getvalue()


# ---- the oracle's CDF against closed forms --------------------------------------------------

def test_oracle_cdf_uniform_probs_equal_uniform_cdf():
    for n in (2, 256, 4096):
        assert np.array_equal(O.cdf_from_probs(np.full(n, 1.0 / n, np.float32)), O.cdf_uniform(n))


def test_oracle_cdf_one_hot():
    n, k = 1000, 417
    p = np.zeros(n, np.float32)
    p[k] = 1.0
    f = np.diff(O.cdf_from_probs(p).astype(np.int64))
    assert f[k] == O.TOTAL - n + 1 and np.all(np.delete(f, k) == 1)


def test_oracle_cdf_fix_up_goes_to_last_maximum():
    # three equal maxima; the deficit of the rounding lands on the last of them
    p = np.array([1, 1, 1], np.float32) / 3
    f = np.diff(O.cdf_from_probs(p).astype(np.int64))
    base = int(((O.TOTAL - 3) / 3) + 0.5)
    assert f[0] == f[1] == 1 + base and f[2] == 1 + base + (O.TOTAL - 3 - 3 * base)
    assert f.sum() == O.TOTAL


# ---- the library against the oracle (bit-exact) -------------------------------------------

def test_lib_exp_golden_and_special():
    for g, w in EXP_GOLDEN:
        assert bits(C.exp_f64(f64(g))) == w, hex(g)
    assert C.exp_f64(-math.inf) == 0.0 and C.exp_f64(math.inf) == math.inf
    assert math.isnan(C.exp_f64(math.nan)) and C.exp_f64(1000.0) == math.inf
    assert bits(C.exp_f64(-1000.0)) == 0


def test_lib_exp_equals_oracle_on_sweep():
    x = sweep_inputs()
    lib = np.array([C.exp_f64(float(t)) for t in x])
    assert np.array_equal(lib.view(np.uint64), O.exp_f64(x).view(np.uint64))
    # the edge bands: near overflow, the subnormal range and tiny |x|
    rng = np.random.default_rng(1)
    e = np.concatenate([rng.uniform(700, 709.9, 300), rng.uniform(-745.2, -700, 300), rng.uniform(-1e-17, 1e-17, 50)])
    lib = np.array([C.exp_f64(float(t)) for t in e])
    assert np.array_equal(lib.view(np.uint64), O.exp_f64(e).view(np.uint64))


def _ref_probs(kind, n, seed=0):
    """The distributions of coder.rs:302-470 and random ones."""
    rng = np.random.default_rng(seed)
    if kind == "skewed":
        p = np.full(n, 0.001, np.float32)
        p[0] = 0.90
    elif kind == "large":
        p = np.full(n, 1e-8, np.float32)
        p[0], p[1], p[2] = 0.3, 0.2, 0.1
        p[3:100] = 0.004
    elif kind == "efficiency":
        p = np.full(n, 0.0001, np.float32)
        p[0], p[1], p[2] = 0.5, 0.3, 0.1
    else:
        p = rng.dirichlet(np.full(n, 0.05)).astype(np.float32)
    # the reference normalises with an f32 sequential sum (`probs.iter().sum()` on f32)
    s = np.float32(0)
    for v in p:
        s = np.float32(s + v)
    return (p / s).astype(np.float32)


@pytest.mark.parametrize("kind,n", [("skewed", 100), ("large", 65536), ("efficiency", 256), ("random", 50280),
                                    ("random", 3)])
def test_lib_cdf_from_probs_equals_oracle(kind, n):
    p = _ref_probs(kind, n)
    lib, orc = C.cdf_from_probs(p), O.cdf_from_probs(p)
    assert np.array_equal(lib, orc)
    f = np.diff(lib.astype(np.int64))
    assert lib[-1] == C.CDF_TOTAL and f.min() >= 1


def _logit_rows(vocab, rows, seed):
    rng = np.random.default_rng(seed)
    out = rng.normal(0, 3.0, (rows, vocab)).astype(np.float32)
    out[0, :] = 0.0                                      # all equal
    if rows > 1:
        out[1, ::7] = out[1].max()                           # tied maxima
    if rows > 2:
        out[2] = (rng.standard_cauchy(vocab) * 20).astype(np.float32)  # exp underflow tails
    if rows > 3:
        out[3] = (np.arange(vocab) - vocab / 2).astype(np.float32) * 0.1  # codec.rs:2641 shape
    return out


@pytest.mark.parametrize("vocab", [256, 50280, 65536])
def test_lib_cdf_from_logits_equals_oracle(vocab):
    for i, row in enumerate(_logit_rows(vocab, 5, vocab)):
        lib, orc = C.cdf_from_logits(row), O.cdf_from_logits(row)
        assert np.array_equal(lib, orc)
        assert lib[-1] == C.CDF_TOTAL
        if i != 0:  # row 0 is flat: see the next test
            assert np.diff(lib.astype(np.int64)).min() >= 1


def test_flat_distribution_over_large_vocab_wraps_like_the_reference():
    """Cdf::from_probs rounds every flat share up when (2^24 - n)/n has a fraction
    >= .5 (50280 symbols: 332.68 -> 333), and its fix-up then takes the whole surplus
    (16304) from the last symbol, whose u32 frequency wraps (coder.rs:63-71 in a release
    build).  The library reproduces those bits; the total still reads 2^24."""
    row = np.zeros(50280, np.float32)
    lib = C.cdf_from_logits(row)
    assert np.array_equal(lib, O.cdf_from_logits(row))
    f = np.diff(lib.astype(np.int64))
    assert np.all(f[:-1] == 334) and int(lib[-2]) == 50279 * 334 and lib[-1] == C.CDF_TOTAL
    # 256 symbols divide the total evenly: no surplus, the uniform CDF
    assert np.array_equal(C.cdf_from_logits(np.zeros(256, np.float32)), C.cdf_uniform(256))


def test_lib_cdf_from_logits_nan_row_matches_oracle():
    row = np.linspace(-3, 3, 300).astype(np.float32)
    row[10] = np.nan
    assert np.array_equal(C.cdf_from_logits(row), O.cdf_from_logits(row))


def test_lib_cdf_batch_equals_rows_for_any_thread_count():
    lg = _logit_rows(50280, 12, 7)
    rows = np.stack([C.cdf_from_logits(r) for r in lg])
    for threads in (0, 1, 3, 8):
        assert np.array_equal(C.cdf_from_logits_batch(lg, threads), rows)


def test_lib_cdf_invalid_sizes():
    with pytest.raises(C.CodecError):
        C.cdf_from_probs(np.zeros(0, np.float32))
    with pytest.raises(C.CodecError):
        C.cdf_uniform(0)


def test_lib_uniform_and_lookup():
    for n in (1, 256, 50280, 65536):
        c = C.cdf_uniform(n)
        assert np.array_equal(c, O.cdf_uniform(n))
    c = C.cdf_from_probs(_ref_probs("random", 1000, 3))
    rng = np.random.default_rng(0)
    for cum in list(rng.integers(0, C.CDF_TOTAL, 300)) + [0, C.CDF_TOTAL - 1]:
        s = C.lookup(c, int(cum))
        assert s == O.lookup(c, int(cum)) and c[s] <= cum < c[s + 1]


# ---- range coder (coder.rs:302-470) ----------------------------------------------------------

def _roundtrip(cdfs, symbols):
    enc = C.RangeEncoder()
    for c, s in zip(cdfs, symbols):
        enc.encode_symbol(s, c)
    data = enc.finish()
    assert data == O.encode_tokens(cdfs, symbols)  # same bytes as the oracle coder
    dec = C.RangeDecoder(data)
    assert [dec.decode_symbol(c) for c in cdfs] == list(symbols)
    assert O.decode_tokens(data, cdfs) == list(symbols)
    # an ideal coder needs ideal_bits.  This one adds its 5-byte flush and, per symbol, the
    # truncation of r = range / total (range >= 2^24 = total, so at most log2((r+1)/r) <= 1 bit)
    ideal = O.ideal_bits(cdfs, symbols)
    assert ideal - 8 <= 8 * len(data) <= ideal + 40 + len(symbols)
    return data


def test_roundtrip_uniform():
    cdf = C.cdf_uniform(256)
    _roundtrip([cdf] * 1000, [i % 256 for i in range(1000)])


def test_roundtrip_skewed():
    cdf = C.cdf_from_probs(_ref_probs("skewed", 100))
    _roundtrip([cdf] * 14, [0, 0, 0, 1, 0, 0, 50, 0, 99, 0, 0, 0, 42, 0])


def test_roundtrip_large_alphabet():
    cdf = C.cdf_from_probs(_ref_probs("large", 65536))
    _roundtrip([cdf] * 10, [0, 1, 2, 50, 1000, 65535, 0, 0, 32768, 2])


def test_roundtrip_varying_distributions():
    syms = [10, 200, 50, 100, 0, 255, 128]
    cdfs = []
    for s in syms:
        p = np.full(256, 0.001, np.float32)
        p[s], p[(s + 1) % 256] = 0.5, 0.2
        cdfs.append(C.cdf_from_probs(p / p.sum(dtype=np.float32)))
    _roundtrip(cdfs, syms)


def test_roundtrip_random_logits_and_carries():
    """Long streams of CDFs from logits, with runs of near-certain symbols, which is where
    0xFF runs and carries into them happen."""
    rng = np.random.default_rng(11)
    lg = _logit_rows(512, 64, 3)
    cdfs = [C.cdf_from_logits(r) for r in lg] * 8
    syms = [int(rng.integers(0, 512)) if i % 5 else int(np.argmax(np.diff(c.astype(np.int64))))
            for i, c in enumerate(cdfs)]
    _roundtrip(cdfs, syms)


def test_compression_efficiency():
    cdf = C.cdf_from_probs(_ref_probs("efficiency", 256))
    enc = C.RangeEncoder()
    for _ in range(10000):
        enc.encode_symbol(0, cdf)
    data = enc.finish()
    ratio = len(data) * 8.0 / (10000 * -math.log2(0.5))
    assert 0.95 < ratio < 1.05


def test_decode_symbol_checked_rejects_out_of_range():
    cdf = C.cdf_uniform(256)
    enc = C.RangeEncoder()
    enc.encode_symbol(200, cdf)
    dec = C.RangeDecoder(enc.finish())
    with pytest.raises(C.CodecError) as e:
        dec.decode_symbol(cdf, vocab=100)
    assert e.value.status == C.CodecStatus.SYMBOL_OUT_OF_RANGE


def test_decode_empty_stream():
    dec = C.RangeDecoder(b"")
    dec.decode_symbol(C.cdf_uniform(256))


def test_decode_corrupted_stream_detected():
    cdf = C.cdf_uniform(256)
    syms = [10, 20, 30, 40, 50]
    enc = C.RangeEncoder()
    for s in syms:
        enc.encode_symbol(s, cdf)
    data = bytearray(enc.finish())
    data[1] ^= 0xFF
    dec = C.RangeDecoder(bytes(data))
    got = []
    try:
        got = [dec.decode_symbol(cdf) for _ in syms]
    except C.CodecError:
        pass
    assert got != syms


def test_coder_and_cdf_deterministic():
    p = np.full(256, 0.001, np.float32)
    p[0], p[1], p[10] = 0.4, 0.3, 0.1
    cdf = C.cdf_from_probs(p / p.sum(dtype=np.float32))
    syms = [0, 1, 0, 10, 255, 0, 0, 1, 128, 50]

    def once():
        e = C.RangeEncoder()
        for s in syms:
            e.encode_symbol(s, cdf)
        return e.finish()

    assert once() == once()
    lg = ((np.arange(256) - 128.0) * 0.1).astype(np.float32)
    a, b = C.RangeEncoder(), C.RangeEncoder()
    a.encode_symbol(42, C.cdf_from_logits(lg))
    b.encode_symbol(42, C.cdf_from_logits(lg))
    assert a.finish() == b.finish()


def test_encoder_size_and_finish_idempotent():
    cdf = C.cdf_uniform(300)
    e = C.RangeEncoder()
    for i in range(100):
        e.encode_symbol((i * 37) % 300, cdf)
    est = e.size()
    d1 = e.finish()
    assert e.finish() == d1 and abs(est - len(d1)) <= 5
    with pytest.raises(C.CodecError):
        e.encode_symbol(0, cdf)
