"""Pins the oracle's scalar math and kernel orders (CPU only).

Each check is chosen so that a plausible restatement mistake fails it: known answers
from the reference's own tests, f64 brute force with error bounds, closed forms, and
inputs whose result depends on the exact accumulation order.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_known_answers.json")))
F32 = np.float32


def test_expf_known_values():
    g = GOLD["portable_expf_known_values"]
    for x, expected in g["cases"]:
        got = O.expf(x)
        assert abs((got - expected) / expected) < g["rel_err_max"], (x, got, expected)


def test_lnf_known_values():
    for x, expected in GOLD["portable_lnf_known_values"]["cases"]:
        got = O.lnf(F32(x))
        tol = abs(expected) * 1e-6 if abs(expected) > 1.0 else 1e-6
        assert abs(got - expected) < tol, (x, got, expected)


def test_expf_sweep_accuracy_and_clamps():
    # Degree-5 Cephes: relative error within a few ulp over the whole unclamped range;
    # a wrong coefficient or reduction constant shows up as >1e-5 somewhere.
    xs = np.linspace(-87.0, 88.0, 20001, dtype=np.float32)
    worst = max(abs(O.expf(float(x)) / math.exp(float(x)) - 1.0) for x in xs)
    assert worst < 4e-7, worst
    assert O.expf(-1000.0) == O.expf(-87.3365447505531)   # lower clamp
    assert O.expf(1000.0) == O.expf(88.3762626647949)     # upper clamp
    assert O.expf(0.0) == 1.0
    assert math.isnan(O.expf(float("nan")))
    assert O.lane_expf(float("nan")) == O.expf(-87.3365447505531)  # NaN lane -> lower clamp


def test_lnf_sweep_and_special_cases():
    xs = np.exp(np.linspace(-80, 80, 20001)).astype(np.float32)
    worst = max(abs(O.lnf(float(x)) - math.log(float(x))) / max(1.0, abs(math.log(float(x)))) for x in xs)
    assert worst < 3e-7, worst
    assert O.lnf(1.0) == 0.0
    assert O.lnf(0.0) == -math.inf
    assert math.isnan(O.lnf(-1.0))
    assert O.lnf(math.inf) == math.inf
    sub = float(np.float32(1e-40))   # subnormal: the 2^25 rescale branch
    assert abs(O.lnf(sub) - math.log(sub)) < 1e-4


def test_softplus_threshold_and_accuracy():
    assert O.softplus(20.5) == F32(20.5)      # identity above the threshold of 20
    assert O.softplus(25.0) == 25.0
    for x in np.linspace(-30, 20, 501, dtype=np.float32):
        ref = math.log1p(math.exp(float(x)))
        # ln(1 + e^x) is evaluated in f32: 1 + e^x carries an absolute rounding error of
        # up to half an ulp of 1, so small results are accurate to ~6e-8 absolute ...
        assert abs(O.softplus(float(x)) - ref) <= 2e-6 * ref + 1.2e-7, x
    # ... and e^x below 2^-24 is absorbed entirely.
    assert O.softplus(-17.0) == 0.0


def test_sigmoid():
    for x in np.linspace(-20, 20, 401, dtype=np.float32):
        assert abs(O.sigmoidf(float(x)) - 1.0 / (1.0 + math.exp(-float(x)))) < 2e-7


def test_softmax_properties():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(50280).astype(np.float32) * 3
    p = O.softmax(x)
    ref = np.exp(x.astype(np.float64) - x.max())
    ref /= ref.sum()
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-4
    # The reference sums 50,280 f32 exponentials sequentially, so the denominator carries
    # a relative error of order 1e-5..1e-4 at this size; the L1 distance to the exact
    # softmax is that error.
    assert np.abs(p - ref).sum() < 1e-4
    assert np.all(np.diff(p[np.argsort(x, kind="stable")]) >= 0)   # monotone in the logit
    u = O.softmax(np.full(7, -np.inf, np.float32))     # all -inf -> uniform
    assert np.all(u == np.float32(1.0) / np.float32(7.0))


# ---- accumulation orders ----

def test_dot_lane_grouping_is_by_column_residue():
    # Columns 0 and 8 share lane 0: 2^24 + 1 rounds to 2^24, then lane 4 cancels it.
    # A sequential sum would give 1; the reference's 8-lane order gives 0.
    w = np.zeros(16, np.float32)
    w[0], w[8], w[4] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    assert O.dot(w, np.ones(16, np.float32)) == 0.0


def test_dot_hsum_tree():
    # Lanes l0=2^24, l1=1, l2=-2^24: ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) = 0 + 1 = 1,
    # while the scan's tree ((l0+l4)+(l1+l5)) + ... would absorb the 1 and give 0.
    w = np.zeros(8, np.float32)
    w[0], w[1], w[2] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    assert O.dot(w, np.ones(8, np.float32)) == 1.0


def test_dot_tail_is_added_after_the_tree():
    # n = 9: the tail element joins after the 8-lane tree: (2^24 + 1) rounds, then -2^24.
    w = np.array([2.0 ** 24, 0, 0, 0, 0, 0, 0, 0, 1.0], np.float32)
    assert O.dot(w, np.ones(9, np.float32)) == 2.0 ** 24
    w2 = np.array([2.0 ** 24, 0, 0, 0, -(2.0 ** 24), 0, 0, 0, 1.0], np.float32)
    assert O.dot(w2, np.ones(9, np.float32)) == 1.0


def test_dot_close_to_f64_and_exact_on_integers():
    rng = np.random.default_rng(1)
    for n in (1, 7, 8, 9, 48, 768, 1536):
        w = rng.standard_normal(n).astype(np.float32)
        v = rng.standard_normal(n).astype(np.float32)
        ref = float(np.dot(w.astype(np.float64), v.astype(np.float64)))
        bound = n * 1.2e-7 * float(np.abs(w.astype(np.float64) * v).sum()) + 1e-30
        assert abs(O.dot(w, v) - ref) <= bound
        wi = rng.integers(-50, 50, n).astype(np.float32)
        vi = rng.integers(-50, 50, n).astype(np.float32)
        assert O.dot(wi, vi) == float(np.dot(wi.astype(np.int64), vi.astype(np.int64)))


def test_ssm_hsum_tree_differs_from_gemv_tree():
    # State lanes s[0]=2^24, s[1]=1, s[2]=-2^24 with C = 1 for n<8, 0 above: the scan sums
    # ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) = 2^24 + -2^24 = 0 (the 1 is absorbed).
    ss = np.zeros((1, 16), np.float32)
    ss[0, 0], ss[0, 1], ss[0, 2] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    c = np.zeros(16, np.float32)
    c[:8] = 1.0
    y, new = O.ssm_d16(ss, [0.0], [0.0], np.zeros(16), np.zeros(16), c, [0.0])   # dt = 0 -> skip
    assert y[0] == 0.0
    assert np.array_equal(new, ss)


# ---- selective scan ----

def test_ssm_closed_form_constant_inputs():
    # Constant dt, x, B: s_t = dA^t s_0 + dt x B (1 - dA^t)/(1 - dA) per state n.
    dt, x = 0.05, 0.7
    a_log = np.log(np.arange(1, 17, dtype=np.float64)).astype(np.float32)
    b = np.linspace(-1, 1, 16).astype(np.float32)
    c = np.linspace(0.5, -0.5, 16).astype(np.float32)
    ss = np.zeros((1, 16), np.float32)
    T = 200
    for _ in range(T):
        y, ss = O.ssm_d16(ss, [dt], [x], a_log, b, c, [1.0])
    A = np.exp(a_log.astype(np.float64))
    dA = np.exp(-dt * A)
    s_ref = dt * x * b * (1 - dA ** T) / (1 - dA)
    np.testing.assert_allclose(ss[0], s_ref, rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose(y[0], float(s_ref @ c) + 1.0 * x, rtol=2e-5)


def test_ssm_dt_skip():
    ss0 = np.arange(16, dtype=np.float32).reshape(1, 16) * 0.1
    c = np.ones(16, np.float32)
    y, ss = O.ssm_d16(ss0, [9e-7], [3.0], np.zeros(16), np.ones(16), c, [2.0])
    assert np.array_equal(ss, ss0)                       # |dt| < 1e-6: state untouched
    y2, ss2 = O.ssm_d16(ss0, [1.1e-6], [3.0], np.zeros(16), np.ones(16), c, [2.0])
    assert not np.array_equal(ss2, ss0)                  # just above: updated


def test_ssm_single_channel_brute_force():
    rng = np.random.default_rng(5)
    di = 5
    ss = rng.standard_normal((di, 16)).astype(np.float32)
    a_log = np.abs(rng.standard_normal((di, 16))).astype(np.float32)
    b, c = rng.standard_normal(16).astype(np.float32), rng.standard_normal(16).astype(np.float32)
    dt = np.array([0.01, 0.2, 1.5, 3e-7, 0.05], np.float32)
    x = rng.standard_normal(di).astype(np.float32)
    dvec = rng.standard_normal(di).astype(np.float32)
    y, new = O.ssm_d16(ss, dt, x, a_log, b, c, dvec)
    for j in range(di):
        s64 = ss[j].astype(np.float64)
        if abs(dt[j]) >= 1e-6:
            s64 = np.exp(-float(dt[j]) * np.exp(a_log[j].astype(np.float64))) * s64 + float(dt[j]) * float(x[j]) * b
        np.testing.assert_allclose(new[j], s64, rtol=1e-5, atol=1e-6)
        assert abs(y[j] - (s64 @ c + dvec[j] * x[j])) < 1e-4


# ---- norms ----

def test_rms_norm_closed_form():
    for cval in (0.0, 1e-3, 0.5, 3.0):
        w = np.linspace(0.5, 1.5, 768).astype(np.float32)
        out = O.rms_norm(np.full(768, cval, np.float32), w)
        expect = cval / math.sqrt(cval * cval + 1e-5) * w.astype(np.float64)
        np.testing.assert_allclose(out, expect, rtol=1e-6, atol=1e-30)


def test_layer_norm_matches_f64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(768).astype(np.float32) * 2 + 1
    w, b = rng.standard_normal(768).astype(np.float32), rng.standard_normal(768).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = (x64 - x64.mean()) / np.sqrt(x64.var() + 1e-5) * w + b
    np.testing.assert_allclose(O.layer_norm(x, w, b), ref, rtol=1e-5, atol=1e-5)


# ---- Q8 weight-only (gemv.rs:256-273, tests gemv.rs:678-760) ----

def test_q8_error_bounded_by_half_step():
    rng = np.random.default_rng(3)
    t = rng.uniform(-1, 1, (64, 256)).astype(np.float32)
    for group in (256, 64, 32):
        q, sc, g = O.quantize(t, group)
        assert g == group
        deq = q.astype(np.float32) * np.repeat(sc, group, axis=1)
        step = np.abs(t).reshape(64, -1, group).max(axis=2) / 127.0
        assert np.all(np.abs(t - deq) <= np.repeat(step, group, axis=1) * 0.5 + 1e-7)


def test_q8_invalid_group_falls_back_to_per_row():
    t = np.random.default_rng(9).uniform(-1, 1, (4, 100)).astype(np.float32)
    for g in (64, 12, 0):
        assert O.quantize(t, g)[2] == 100


def test_q8_zero_group_and_rounding_half_away():
    t = np.random.default_rng(11).uniform(-1, 1, (8, 64)).astype(np.float32)
    t[1] = 0.0
    t[2, :8] = 0.0
    q, sc, _ = O.quantize(t, 8)
    assert np.all(q[1] == 0) and np.all(sc[1] == 1.0) and sc[2, 0] == 1.0
    out = O.gemv_q8(q, sc, 8, np.random.default_rng(2).uniform(-1, 1, 64))
    assert out[1] == 0.0 and np.all(np.isfinite(out))
    # amax = 127 -> scale 1: w = +-2.5 must round away from zero to +-3, 1.5 -> 2, -0.5 -> -1.
    row = np.zeros((1, 8), np.float32)
    row[0, :5] = [127.0, 2.5, -2.5, 1.5, -0.5]
    q1, s1, _ = O.quantize(row, 8)
    assert s1[0, 0] == 1.0 and list(q1[0, :5]) == [127, 3, -3, 2, -1]


def test_q8_gemv_close_to_f32():
    rng = np.random.default_rng(41)
    rows, cols = 512, 768
    t = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    v = rng.uniform(-1, 1, cols).astype(np.float32)
    f = O.gemv_f32(t, v)
    sum_abs_v = float(np.abs(v).sum())
    for group in (cols, 64):
        q, sc, g = O.quantize(t, group)
        o = O.gemv_q8(q, sc, g, v)
        bound = sum_abs_v * np.abs(t).max(axis=1) / 127.0 * 0.5 + 1e-3
        assert np.all(np.abs(f - o) <= bound)
        deq = q.astype(np.float64) * np.repeat(sc.astype(np.float64), g, axis=1)
        np.testing.assert_allclose(o, deq @ v.astype(np.float64), rtol=1e-4, atol=2e-5)


def test_q8_group_scales_apply_per_group():
    # Two groups with different scales: the row sum is dot_0*s_0 + dot_1*s_1.
    w = np.zeros((1, 16), np.float32)
    w[0, :8] = 127.0
    w[0, 8:] = 0.5
    q, sc, g = O.quantize(w, 8)
    assert g == 8 and list(sc[0]) == [1.0, np.float32(0.5) / np.float32(127.0)]
    v = np.ones(16, np.float32)
    assert abs(O.gemv_q8(q, sc, 8, v)[0] - (8 * 127 + 8 * 0.5)) < 1e-3
