"""The wavefront-GEMV tier (weight profile bit 4) on the GPU, through the C ABI.

The tier computes the Mamba projections as f32 dot products on the vector ALUs (the
small-batch family); it is chosen at init, never by n (the batch-invariance rule of
PLUGIN-FFI-V2.md:97-101: a stream's logits may not depend on the batch it runs in), so:

* logits within max |err| <= 1e-3 and probability L1 <= 1e-4 of the CPU oracle (the oracle
  knows one arithmetic for the model; the tier bit only changes how the GPU computes it),
  on small models and full Mamba-130M, F32 and int8 per-row weights;
* inside the tier a stream's bits do not depend on n, its batch position or its slot, v1
  equals batch, and runs repeat bit for bit;
* the device-side argument check contains bad entries as in the matrix-core family.
"""
import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, hip, rbin, synth

pytestmark = pytest.mark.gpu

TOL_ABS = 1e-3
TOL_L1 = 1e-4
GEMV = ffi.PROFILE_GEMV
SMALL = {"reftest": rbin.MambaDims(vocab=1200, d_model=64, n_layer=2),
         "base": rbin.MambaDims(vocab=1000, d_model=96, n_layer=3)}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def probs64(logits):
    x = np.asarray(logits, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def assert_parity(gpu, cpu, what=""):
    err = float(np.max(np.abs(gpu.astype(np.float64) - cpu)))
    l1 = float(np.max(np.abs(probs64(gpu) - probs64(cpu)).sum(axis=-1)))
    assert err <= TOL_ABS and l1 <= TOL_L1, f"{what}: max|dlogit|={err:.3e} L1={l1:.3e}"
    return err, l1


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    assert hip.device_count() > 0, "no GPU visible"
    d = tmp_path_factory.mktemp("gemv_models")
    out = {"reftest": str(d / "reftest.rbin"), "base": str(d / "base.rbin")}
    synth.write_synthetic_mamba(out["reftest"], SMALL["reftest"], init="reference-test")
    synth.write_synthetic_mamba(out["base"], SMALL["base"], seed=7)
    return out


@pytest.mark.parametrize("name,profile", [("reftest", 0), ("reftest", 2), ("base", 0), ("base", 2), ("base", 6)])
def test_gemv_small_model_parity(small, name, profile):
    with ffi.PluginBackend(small[name], profile=profile | GEMV) as be:
        orc = O.MambaOracle(small[name], profile, cap=9)
        v = be.vocab
        be.batch_init(9)
        for t in range(6):
            toks = [(s * 131 + t * 977 + 7) % v for s in range(9)]
            g = np.empty((9, v), np.float32)
            be.forward_batch(list(range(9)), toks, g)
            assert_parity(g, orc.forward(list(range(9)), toks), f"{name} p{profile} step {t}")
        dims = SMALL[name]
        for layer in range(dims.n_layer):
            gc, gs = be.get_state(4, layer, dims.d_inner, 4)
            cc, cs = orc.state(4, layer)
            np.testing.assert_allclose(gc, cc, rtol=1e-4, atol=1e-5)
            np.testing.assert_allclose(gs, cs, rtol=1e-3, atol=1e-5)
        orc.close()


@pytest.mark.parametrize("profile", [0, 6])
def test_gemv_mamba130m_parity(full_model, profile):
    n = 4
    rng = np.random.default_rng(31)
    toks = synth.zipf_tokens(rng, 50280, (6, n))
    with ffi.PluginBackend(full_model, profile=profile | GEMV) as be:
        orc = O.MambaOracle(full_model, profile, cap=n)
        be.batch_init(n)
        worst = (0.0, 0.0)
        for t in range(6):
            tl = [int(x) for x in toks[t]]
            g = np.empty((n, be.vocab), np.float32)
            be.forward_batch(list(range(n)), tl, g)
            worst = max(worst, assert_parity(g, orc.forward(list(range(n)), tl), f"130M gemv p{profile} step {t}"))
        orc.close()
    print(f"Mamba-130M GEMV tier profile {profile}: worst max|dlogit|={worst[0]:.3e} L1={worst[1]:.3e}")


@pytest.mark.parametrize("profile", [0, 2])
def test_gemv_batch_invariance_and_v1(small, profile):
    with ffi.PluginBackend(small["base"], profile=profile | GEMV) as be:
        v = be.vocab
        seq = [(13 * i + 5) % v for i in range(5)]
        out = np.empty(v, np.float32)
        be.lib.lib.redukt_backend_reset_state()
        v1 = []
        for t in seq:
            assert be.lib.lib.redukt_backend_forward(t, out.ctypes.data_as(ffi._f32p), v) == ffi.BackendResult.OK
            v1.append(out.copy())
        be.batch_init(40)
        rng = np.random.default_rng(5)
        for n, pos in ((1, 0), (2, 1), (7, 3), (33, 32), (39, 17)):
            be.batch_reset(None)
            slots = [int(s) for s in rng.permutation(40)[:n]]
            for i, t in enumerate(seq):
                toks = [int(x) for x in rng.integers(0, v, n)]
                toks[pos] = t
                g = np.empty((n, v), np.float32)
                be.forward_batch(slots, toks, g)
                assert np.array_equal(bits(g[pos]), bits(v1[i])), (n, pos, i)


def test_gemv_run_to_run_and_probabilities(small):
    runs = []
    for _ in range(2):
        with ffi.PluginBackend(small["reftest"], profile=2 | GEMV) as be:
            be.batch_init(5)
            outs = []
            for t in range(4):
                p = np.empty((5, be.vocab), np.float32)
                be.forward_batch(list(range(5)), [(s * 31 + t * 7) % be.vocab for s in range(5)], p, probs=True)
                outs.append(p)
            runs.append(np.stack(outs))
    assert np.array_equal(bits(runs[0]), bits(runs[1]))
    assert np.allclose(runs[0].sum(axis=-1), 1.0, atol=1e-5)


def test_gemv_device_check_contains_bad_entries(small):
    dims = SMALL["base"]
    with ffi.PluginBackend(small["base"], profile=GEMV) as be:
        v = be.vocab
        be.batch_init(8)
        d_s = hip.DeviceBuffer.from_array(np.array([7, 6, 7, 4, 2], np.uint32))
        d_t = hip.DeviceBuffer.from_array(np.array([9, 8, 7, 6, v + 3], np.uint32))
        d_o = hip.DeviceBuffer(5 * v * 4)
        try:
            before = {s: be.get_state(s, 0, dims.d_inner, 4) for s in (0, 2, 5)}
            be.forward_batch_device(5, d_s.ptr, d_t.ptr, d_o.ptr)
            assert be.device_status() == ffi.BackendResult.INVALID_ARGUMENT
            for s, (c0, x0) in before.items():
                c1, x1 = be.get_state(s, 0, dims.d_inner, 4)
                assert np.array_equal(c0, c1) and np.array_equal(x0, x1), s
        finally:
            for b in (d_s, d_t, d_o):
                b.close()


def test_gemv_tier_refuses_what_it_does_not_serve(small, tmp_path):
    # group-64 int8 weights and LayerNorm models are served by the matrix-core family only
    path = str(tmp_path / "flags.rbin")
    synth.write_synthetic_mamba(path, rbin.MambaDims(vocab=500, d_model=64, n_layer=2), seed=3,
                                flags=rbin.FLAG_NORM_BIAS)
    lib = ffi.PluginLibrary()
    info = ffi.BackendInfo()
    for p, prof in ((small["base"], 1 | GEMV), (path, GEMV)):
        rc = lib.lib.redukt_backend_init_ex(p.encode(), 0, prof, ffi.ctypes.byref(info))
        assert rc == ffi.BackendResult.INIT_FAILED, (p, prof, rc)
    lib.lib.redukt_backend_free()
