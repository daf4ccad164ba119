"""The round-based exact sequential sum of the device CDF (cdf_step.hip, exact_seq_sum),
restated in Python and checked against the plain sequential f64 sum it must reproduce.

The device sums a row's non-negative terms in rounds: while the running sum s stays in one
binade, s = T u on the grid u = 2^(E-52) and fl(s + x) = (T + round(x / u)) u, so a round is
an integer prefix sum; a term whose x / u is a tie, a NaN, or that takes T to the top of the
binade is an event and takes one real f64 add.  This restatement follows the same steps
(window, grid, events, commit), so a flaw in the method (a missed tie, a wrong crossing
test, the subnormal grid, the -0.0 start) fails here on the CPU, on inputs built to hit
each case; the GPU tests then check the kernel against the host CDF bit for bit.
"""
import math

import numpy as np
import pytest

ROUND = 64   # terms per round (the device takes 8192; the rule does not depend on it)


def sequential(x, s0):
    s = np.float64(s0)
    for v in x:
        s = np.float64(s + np.float64(v))
    return s


def ldexp_inf(v, k):
    """ldexp that overflows to +inf, as the device's does."""
    try:
        return math.ldexp(v, k)
    except OverflowError:
        return math.inf


def rounds_sum(x, s0, window=ROUND, head=0):
    """The device's steps: the first `head` terms added one by one (when the row has that
    many), then rounds over windows of `window` terms, the first window starting after the
    head."""
    x = [float(v) for v in x]
    n = len(x)
    s = float(s0)
    if n >= head > 0:
        assert head <= window
        for v in x[:head]:
            s = float(np.float64(s) + np.float64(v))
    k0 = 0
    while k0 < n:
        frm = head if (k0 == 0 and n >= head) else 0
        while frm < window and k0 + frm < n:
            if math.isnan(s):
                return s
            if s < 2.0 ** -1022:
                ks, top = 1074, 1 << 52
            else:
                ks, top = 52 - (math.frexp(s)[1] - 1), 1 << 53
            T0 = int(math.ldexp(s, ks))
            T = T0
            first, t_ev = None, None
            for r in range(frm, min(window, n - k0)):
                v = x[k0 + r]
                if math.isnan(v):
                    first, t_ev = r, T
                    break
                q = ldexp_inf(v, ks)
                if not (q < 2.0 ** 53):
                    first, t_ev = r, T
                    break
                m = math.floor(q)
                fr = q - m
                if fr == 0.5:
                    first, t_ev = r, T
                    break
                a = int(m) + (1 if fr > 0.5 else 0)
                if T + a >= top:
                    first, t_ev = r, T
                    break
                T += a
            if first is None:
                s = math.ldexp(float(T), -ks)
                frm = window
            else:
                s = float(np.float64(math.ldexp(float(t_ev), -ks)) + np.float64(x[k0 + first]))
                frm = first + 1
        k0 += window
    return s


def same(a, b):
    return (math.isnan(a) and math.isnan(b)) or np.float64(a).view(np.uint64) == np.float64(b).view(np.uint64)


@pytest.mark.parametrize("seed", range(6))
def test_exp_rows(seed):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal(3000) * [0.1, 1, 3, 8, 30, 300][seed]
    e = np.exp(logits - logits.max())
    assert same(rounds_sum(e, 0.0), sequential(e, 0.0))
    p = (e * (1.0 / sequential(e, 0.0))).astype(np.float32).astype(np.float64)
    assert same(rounds_sum(p, -0.0), sequential(p, -0.0))


def test_ties_round_to_even():
    # s = 1 (grid 2^-52): a term of exactly half a grid step ties; the result depends on the
    # parity of s's last bit, which alternates as odd steps are added
    half = 2.0 ** -53
    x = [1.0, half, half, 2.0 ** -52, half, 3 * half, half, 2.0 ** -52 + half, half] * 20
    assert same(rounds_sum(x, 0.0), sequential(x, 0.0))
    # ties on a coarser grid and just below a binade top
    x = [2.0 ** 10] + [2.0 ** -43, 2.0 ** -42 * 3] * 100 + [2.0 ** 11 - 2.0 ** 10 - 2.0 ** -42] + [2.0 ** -43] * 50
    assert same(rounds_sum(x, 0.0), sequential(x, 0.0))


def test_crossings_every_few_terms():
    x = [2.0 ** k for k in range(-30, 20)] + [1.0] * 500 + [2.0 ** -60] * 100
    assert same(rounds_sum(x, 0.0), sequential(x, 0.0))


def test_subnormal_grid_and_zero_starts():
    tiny = 2.0 ** -1074
    x = [0.0, 0.0, tiny, 3 * tiny, 2.0 ** -1030, 2.0 ** -1022, tiny, 1e-300, 0.0, 1.0]
    assert same(rounds_sum(x, 0.0), sequential(x, 0.0))
    assert same(rounds_sum([0.0, 0.0], -0.0), sequential([0.0, 0.0], -0.0))   # -0.0 + 0.0 = +0.0
    assert same(rounds_sum([0.0], -0.0), 0.0)
    assert same(rounds_sum([tiny] * 300, -0.0), sequential([tiny] * 300, -0.0))


def test_nan_propagates():
    x = [0.5, 0.25, float("nan"), 0.125]
    assert math.isnan(rounds_sum(x, 0.0))


@pytest.mark.parametrize("window", [1, 3, 64, 1000])
def test_window_size_does_not_matter(window):
    rng = np.random.default_rng(11)
    x = np.exp(rng.standard_normal(2500) * 4)
    assert same(rounds_sum(x, 0.0, window), sequential(x, 0.0))


@pytest.mark.parametrize("head,window", [(1, 1), (16, 64), (64, 64), (256, 1000), (256, 8192)])
def test_a_sequential_head_then_rounds(head, window):
    # the head ends inside or at the end of the first window; rows shorter than the head go
    # to the rounds alone; ties and crossings sit on both sides of the head's end
    rng = np.random.default_rng(head + window)
    half = 2.0 ** -53
    x = np.concatenate([np.exp(rng.standard_normal(300) * 3), [1.0] + [half, 2.0 ** -52] * 20,
                        np.exp(rng.standard_normal(2000))])
    for row in (x, x[:head - 1] if head > 1 else x[:0], x[:head], x[:head + 3]):
        for s0 in (0.0, -0.0):
            assert same(rounds_sum(row, s0, window, head), sequential(row, s0))
    p = (x * (1.0 / sequential(x, 0.0))).astype(np.float32).astype(np.float64)
    assert same(rounds_sum(p, -0.0, window, head), sequential(p, -0.0))


def test_a_missed_tie_is_caught():
    # planted mistake: rounding ties up instead of to even changes these sums, so the
    # tie rule is what makes the method exact
    half = 2.0 ** -53
    x = [1.0] + [half, 2.0 ** -52] * 10

    def ties_up(x, s0):
        s = float(s0)
        for v in x:
            t = np.float64(s) + np.float64(v)
            # round-half-up on the grid of s
            u = 2.0 ** (math.frexp(s)[1] - 53) if s >= 2.0 ** -1022 else 2.0 ** -1074
            q = (v / u) if s else None
            if q is not None and q - math.floor(q) == 0.5:
                t = s + (math.floor(q) + 1) * u
            s = float(t)
        return s

    assert not same(ties_up(x, 0.0), sequential(x, 0.0))
    assert same(rounds_sum(x, 0.0), sequential(x, 0.0))
