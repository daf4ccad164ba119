"""The oracle's W8A8 path: the reference's own RWKV-7 Q8 arithmetic
(src/domain/tensor.rs:105-143 Q8Tensor, :1791-1800 quantize_vec_i8_into, :1819-1866
q8_mat_vec_mul_into), selected by profile bit 5 with per-row int8 weights.

Pinned three ways:
- the vector quantizer against a numpy statement of its definition (IEEE f32 divide and
  multiply, round half away from zero written with floor in float64, where it is exact for
  f32 inputs), on random vectors and on crafted ties, zeros, NaN, infinities and a
  subnormal maximum; a half-to-even quantizer (numpy's round) fails the tie case;
- the product against numpy's int64 matrix product and float32 rescale, including sums
  beyond 2^24 where the int -> f32 conversion rounds;
- the whole step against the float64 model of tests/rwkv_f64.py with the same int8
  weights and int8 activations quantized in float64.
"""
import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import rwkv
from tests.rwkv_f64 import F64Rwkv

W8A8 = 32
SMALL = rwkv.RwkvDims(vocab=300, d_model=128, n_layer=2, head_size=64, d_ffn=256, lora_w=16, lora_a=16,
                      lora_v=8, lora_g=32)


def np_quantize(v):
    """quantize_vec_i8_into from its definition."""
    v = np.asarray(v, np.float32)
    a = np.abs(v)
    a = a[~np.isnan(a)]
    amax = np.float32(a.max()) if a.size else np.float32(0)
    with np.errstate(all="ignore"):
        scale = amax / np.float32(127) if amax > 0 else np.float32(1)
        inv = np.float32(1) / scale
        t = (v * inv).astype(np.float64)            # the f32 product, exactly
        r = np.where(t < 0, -np.floor(-t + 0.5), np.floor(t + 0.5))
        r = np.clip(r, -127, 127)
        q = np.where(np.isnan(r), 0, r).astype(np.int8)
    return q, np.float32(scale)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("seed", range(8))
def test_quantize_vec_matches_definition(seed):
    rng = np.random.default_rng(seed)
    n = [1, 7, 64, 128, 768, 1000, 3072, 4096][seed]
    v = (rng.standard_normal(n) * [1e-30, 1e-3, 0.02, 1, 3, 50, 1e5, 1e30][seed]).astype(np.float32)
    q, sc = O.quantize_vec_i8(v)
    want_q, want_sc = np_quantize(v)
    assert same_bits(sc, want_sc)
    assert np.array_equal(q, want_q)
    # the largest magnitude maps to +-127 and every element is within half a step
    i = int(np.argmax(np.abs(v)))
    assert abs(int(q[i])) == 127
    assert np.all(np.abs(q.astype(np.float64) * np.float64(sc) - v) <= np.float64(sc) * (0.5 + 1e-5))


def test_ties_round_half_away_from_zero():
    v = np.array([127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5, 3.25, -0.25], np.float32)
    q, sc = O.quantize_vec_i8(v)
    assert sc == 1.0
    assert q.tolist() == [127, 1, 2, 3, -1, -2, -3, 127, -127, 3, 0]
    # a quantizer rounding ties to even gives other values on the same input
    assert np.round(v).astype(np.int8).tolist() != q.tolist()
    assert np.array_equal(q, np_quantize(v)[0])


def test_special_vectors():
    cases = {
        "zeros": np.zeros(16, np.float32),
        "neg-zero": np.full(9, -0.0, np.float32),
        "nan": np.array([1.0, np.nan, -3.0, 0.5], np.float32),
        "all-nan": np.full(5, np.nan, np.float32),
        "inf": np.array([1.0, np.inf, -2.0, 0.0], np.float32),
        "subnormal-max": np.array([1e-45, -1e-45, 0.0, 3e-45], np.float32),
        "empty-ish": np.array([0.0], np.float32),
    }
    for name, v in cases.items():
        q, sc = O.quantize_vec_i8(v)
        want_q, want_sc = np_quantize(v)
        assert same_bits(sc, want_sc), name
        assert np.array_equal(q, want_q), (name, q, want_q)
    assert O.quantize_vec_i8(cases["zeros"])[1] == 1.0
    assert O.quantize_vec_i8(cases["nan"])[0].tolist() == [42, 0, -127, 21]
    assert O.quantize_vec_i8(cases["inf"])[0].tolist() == [0, 0, 0, 0]            # scale inf, inv 0
    assert O.quantize_vec_i8(cases["subnormal-max"])[0].tolist() == [127, -127, 0, 127]  # scale 0, inv inf


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (64, 768), (33, 3072)])
def test_matvec_a8_is_the_integer_product(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    q = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    vq = rng.integers(-127, 128, cols, dtype=np.int8)
    sc = (rng.random(rows) * 1e-3).astype(np.float32)
    vs = np.float32(0.0173)
    got = O.q8_matvec_a8(q, sc, vq, vs)
    s = q.astype(np.int64) @ vq.astype(np.int64)
    want = s.astype(np.float32) * (sc * vs)
    assert same_bits(got, want)


def test_matvec_a8_sums_beyond_f32_precision():
    # 3072 products of 127 * 127: 49,548,288 needs 26 bits; the conversion rounds to even
    q = np.full((2, 3072), 127, np.int8)
    q[1, 0] = 126
    vq = np.full(3072, 127, np.int8)
    got = O.q8_matvec_a8(q, np.ones(2, np.float32), vq, 1.0)
    s = q.astype(np.int64) @ vq.astype(np.int64)
    assert s.tolist() == [49548288, 49548161]
    assert got.tolist() == [49548288.0, 49548160.0]
    assert int(got[1]) != int(s[1])                     # not representable: rounded


def test_w8a8_needs_per_row_weights(tmp_path):
    p = str(tmp_path / "m.rbin")
    rwkv.write_synthetic(p, SMALL, seed=3)
    for prof in (W8A8, W8A8 | 1):
        with pytest.raises(RuntimeError):
            O.RwkvOracle(p, prof)
    O.RwkvOracle(p, W8A8 | 2).close()


# ---- the whole step against float64 ----

QNAMES = ["receptance", "key", "value", "output", "ffn_key", "ffn_value"]


def a8_mats(t, dims):
    out = {}
    for name in ["head"] + [f"blocks.{i}.{m}" for i in range(dims.n_layer) for m in QNAMES]:
        w = np.asarray(t[name], np.float32)
        q, sc, _ = O.quantize(w, w.shape[1])
        out[name] = (q, sc.reshape(-1))
    return out


def worst_against_f64(path, dims, tokens, profile=W8A8 | 2):
    _, t = rwkv.read_rwkv(path)
    orc = O.RwkvOracle(path, profile, cap=2)
    ref = F64Rwkv(dims, t, a8=a8_mats(t, dims))
    worst = 0.0
    for step in tokens:
        lo = orc.forward([0, 1], list(step))
        for b in range(2):
            worst = max(worst, float(np.max(np.abs(lo[b] - ref.step(b, step[b])))))
    orc.close()
    return worst


TOKENS = [[5, 17], [250, 3], [17, 17], [0, 299], [42, 7], [8, 9]]
A8_TOL = 1e-5


def test_w8a8_step_matches_float64(tmp_path):
    p = str(tmp_path / "m.rbin")
    rwkv.write_synthetic(p, SMALL, seed=1)
    # float64 and the f32 step round activations at the same points unless an element sits
    # within float32 rounding of a half step; for this model and these tokens none does,
    # so the two agree to float32 accuracy
    assert worst_against_f64(p, SMALL, TOKENS) < A8_TOL


def test_w8a8_differs_from_weight_only(tmp_path):
    """The activation quantization is taken: the W8A8 logits are not the weight-only ones,
    and the weight-only logits miss the float64 W8A8 model by far more than the tolerance."""
    p = str(tmp_path / "m.rbin")
    rwkv.write_synthetic(p, SMALL, seed=1)
    a = O.RwkvOracle(p, W8A8 | 2, cap=1)
    b = O.RwkvOracle(p, 2, cap=1)
    la, lb = a.forward([0], [5]), b.forward([0], [5])
    a.close()
    b.close()
    assert np.max(np.abs(la - lb)) > 100 * A8_TOL
    assert worst_against_f64(p, SMALL, TOKENS[:2], profile=2) > 100 * A8_TOL
