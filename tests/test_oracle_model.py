"""Pins the oracle's Mamba model (CPU only): structure against an independent float64
brute force, and the reference's own invariants — lockstep == single stream bit for
bit (src/infrastructure/mamba/model.rs:1091-1134), thread-count independence, reset ==
fresh and the periodic reset schedule (model.rs:315-320)."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import rbin, synth
from tests.mamba_f64 import F64Mamba

SMALL = rbin.MambaDims(vocab=1200, d_model=64, n_layer=2)
PROFILES = [0, 1, 2, 2 | 4]


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    d = tmp_path_factory.mktemp("oracle_models")
    out = {}
    out["reftest"] = str(d / "reftest.rbin")
    synth.write_synthetic_mamba(out["reftest"], SMALL, init="reference-test")
    out["baseline"] = str(d / "baseline.rbin")
    synth.write_synthetic_mamba(out["baseline"], rbin.MambaDims(vocab=1000, d_model=96, n_layer=3), seed=7)
    out["bias_untied"] = str(d / "bias_untied.rbin")
    synth.write_synthetic_mamba(out["bias_untied"], rbin.MambaDims(vocab=500, d_model=64, n_layer=2), seed=3,
                                flags=rbin.FLAG_NORM_BIAS | rbin.FLAG_UNTIED_HEAD)
    return out


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("profile", PROFILES)
def test_lockstep_bit_identical_to_single_stream(models, profile):
    m = O.MambaOracle(models["reftest"], profile, cap=9)
    v = m.vocab
    for n in (2, 3, 5, 9):
        steps = 6
        toks = [[(s * 131 + t * 977 + 7) % v for t in range(steps)] for s in range(n)]
        ref_logits = []
        for s in range(n):
            m.reset()
            for t in range(steps):
                lo = m.forward([0], [toks[s][t]])
            ref_logits.append(lo[0])
            ref_state = [m.state(0, l) for l in range(m.n_layer)]
            ref_logits[-1] = (lo[0], ref_state)
        m.reset()
        for t in range(steps):
            lo = m.forward(list(range(n)), [toks[s][t] for s in range(n)])
        for s in range(n):
            assert np.array_equal(bits(lo[s]), bits(ref_logits[s][0])), (profile, n, s)
            for l in range(m.n_layer):
                c, ss = m.state(s, l)
                assert np.array_equal(bits(c), bits(ref_logits[s][1][l][0]))
                assert np.array_equal(bits(ss), bits(ref_logits[s][1][l][1]))
    m.close()


def test_thread_count_independence(models):
    outs = []
    for threads in (1, 3, 8):
        O.set_threads(threads)
        m = O.MambaOracle(models["baseline"], 1, cap=4)
        for t in range(3):
            lo = m.forward([3, 1, 0, 2], [5 + t, 17, 999, 0])
        outs.append(lo)
        m.close()
    O.set_threads(os.cpu_count() or 1)
    assert all(np.array_equal(bits(outs[0]), bits(o)) for o in outs[1:])


@pytest.mark.parametrize("name,profile", [("reftest", 0), ("baseline", 0), ("bias_untied", 0),
                                          ("reftest", 1), ("baseline", 2), ("baseline", 6), ("bias_untied", 6)])
def test_matches_float64_brute_force(models, name, profile):
    path = models[name]
    dims, flags, tensors = rbin.read_rbin(path)
    m = O.MambaOracle(path, profile, cap=1)
    overrides = None
    if profile & 3:
        overrides = {"emb": m.dequant(2)}
        for l in range(dims.n_layer):
            overrides[f"layers.{l}.in_proj"] = m.dequant(0, l)
            overrides[f"layers.{l}.out_proj"] = m.dequant(1, l)
            if profile & 4:
                overrides[f"layers.{l}.x_proj"] = m.dequant(3, l)
                overrides[f"layers.{l}.dt_proj_w"] = m.dequant(4, l)
        if flags & rbin.FLAG_UNTIED_HEAD:
            pytest.skip("the oracle exposes no dequantized view of an untied head")
    ref = F64Mamba(dims, tensors, flags, overrides)
    rng = np.random.default_rng(11)
    toks = rng.integers(0, dims.vocab, 12)
    worst = 0.0
    for t in toks:
        got = m.forward([0], [int(t)])[0].astype(np.float64)
        want = ref.step(int(t))
        worst = max(worst, float(np.max(np.abs(got - want)) / (np.max(np.abs(want)) + 1e-12)))
    # f32 vs f64 through a few layers: ~2e-7 relative; every structural slip tried
    # (conv shift or tap, B/C swap, dropped dt bias, D skip or 1/n, wrong z, decay) is >4e-5.
    assert worst < 2e-6, worst
    for l in range(dims.n_layer):
        conv, ssm = m.state(0, l)
        np.testing.assert_allclose(ssm.reshape(dims.d_inner, 16), ref.ssm[l], rtol=1e-3, atol=1e-5)
        np.testing.assert_allclose(conv.reshape(dims.d_inner, dims.d_conv - 1), ref.conv[l], rtol=1e-4, atol=1e-6)
    m.close()


def test_reset_equals_fresh_and_periodic_reset(models):
    m = O.MambaOracle(models["baseline"], 0, cap=2)
    first = m.forward([1], [42])[0]
    m.forward([1], [7])
    m.reset([1])
    assert np.array_equal(bits(m.forward([1], [42])[0]), bits(first))
    # Period 3: the 4th forward since the last reset starts from zero state again.
    m2 = O.MambaOracle(models["baseline"], 0, cap=1)
    m2.set_reset_every(3)
    seq = [42, 5, 9, 42, 5, 9, 42]
    outs = [m2.forward([0], [t])[0] for t in seq]
    assert np.array_equal(bits(outs[3]), bits(outs[0]))
    assert np.array_equal(bits(outs[4]), bits(outs[1]))
    assert np.array_equal(bits(outs[6]), bits(outs[0]))
    assert not np.array_equal(bits(outs[1]), bits(outs[0]))
    m.close()
    m2.close()


def test_invalid_arguments_leave_state_untouched(models):
    m = O.MambaOracle(models["baseline"], 0, cap=3)
    m.forward([0, 1], [1, 2])
    before = [m.state(s, 0) for s in range(3)]
    for slots, toks in (([0, 0], [1, 2]), ([3], [1]), ([1], [1000]), ([0, 1, 2, 0], [1, 1, 1, 1])):
        with pytest.raises(ValueError):
            m.forward(slots, toks)
    after = [m.state(s, 0) for s in range(3)]
    for (c0, s0), (c1, s1) in zip(before, after):
        assert np.array_equal(c0, c1) and np.array_equal(s0, s1)
    m.close()


def test_q8_profiles_stay_close_to_f32(models):
    # Weight-only int8 moves logits by a bounded amount; the groups-of-64 profile is the
    # more accurate one (the reason the reference chose it, model.rs:50-56).
    f = O.MambaOracle(models["baseline"], 0, cap=1)
    g = O.MambaOracle(models["baseline"], 1, cap=1)
    r = O.MambaOracle(models["baseline"], 2, cap=1)
    eg = er = 0.0
    for t in (3, 99, 512, 7, 0):
        lf, lg, lr = f.forward([0], [t])[0], g.forward([0], [t])[0], r.forward([0], [t])[0]
        eg = max(eg, float(np.abs(lf - lg).max()))
        er = max(er, float(np.abs(lf - lr).max()))
    assert 0 < eg < 0.05 and 0 < er < 0.05
    for x in (f, g, r):
        x.close()
