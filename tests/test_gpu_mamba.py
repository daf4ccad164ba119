"""GPU parity and contract tests of libredukt_gpu.so through its C ABI.

Mirrors the checks of the reference's GPU validation harness
(notebooks/redukt-gpu-cuda-test.py:254-289) and the FFI v2 contract
(docs/api/PLUGIN-FFI-V2.md:55-108), against the CPU oracle on the same seeded weights:

* logits within |err| <= 1e-3 and probability-vector L1 <= 1e-4 of the oracle;
* v1 == batch bit-exact, batch invariance (any n, position, slot), run-to-run bitwise;
* reset == fresh, the periodic reset schedule, INVALID_ARGUMENT leaves state untouched;
* the v3 probability and device-resident entry points.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, hip, rbin, synth

pytestmark = pytest.mark.gpu

TOL_ABS = 1e-3      # max |logit_gpu - logit_cpu|
TOL_L1 = 1e-4       # sum |p_gpu - p_cpu|
SMALL_REFTEST = rbin.MambaDims(vocab=1200, d_model=64, n_layer=2)
SMALL_BASE = rbin.MambaDims(vocab=1000, d_model=96, n_layer=3)


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


@pytest.fixture(scope="session")
def models(tmp_path_factory):
    assert hip.device_count() > 0, "no GPU visible"
    d = tmp_path_factory.mktemp("gpu_models")
    out = {"reftest": str(d / "reftest.rbin"), "base": str(d / "base.rbin"), "flags": str(d / "flags.rbin")}
    synth.write_synthetic_mamba(out["reftest"], SMALL_REFTEST, init="reference-test")
    synth.write_synthetic_mamba(out["base"], SMALL_BASE, seed=7)
    synth.write_synthetic_mamba(out["flags"], rbin.MambaDims(vocab=500, d_model=64, n_layer=2), seed=3,
                                flags=rbin.FLAG_NORM_BIAS | rbin.FLAG_UNTIED_HEAD)
    return out


def run_lockstep(backend, oracle, n, steps, tok_fn, cap=None):
    backend.batch_init(cap or n)
    outs = []
    for t in range(steps):
        toks = [tok_fn(s, t) for s in range(n)]
        g = np.empty((n, backend.vocab), np.float32)
        backend.forward_batch(list(range(n)), toks, g)
        c = oracle.forward(list(range(n)), toks) if oracle is not None else None
        outs.append((g, c))
    return outs


# profile 8 / 14: the scan's decay factors by the portable exp (exact element-wise scan)
@pytest.mark.parametrize("name,profile", [("reftest", 0), ("reftest", 1), ("reftest", 2), ("reftest", 6),
                                          ("reftest", 8), ("base", 0), ("base", 1), ("base", 6), ("base", 14),
                                          ("flags", 0), ("flags", 6)])
def test_small_model_parity(models, name, profile):
    with ffi.PluginBackend(models[name], profile=profile) as be:
        orc = O.MambaOracle(models[name], profile, cap=9)
        v = be.vocab
        outs = run_lockstep(be, orc, 9, 6, lambda s, t: (s * 131 + t * 977 + 7) % v)
        for t, (g, c) in enumerate(outs):
            assert_parity(g, c, f"{name} p{profile} step {t}")
        for l in range(orc.n_layer):
            for s in (0, 8):
                gc, gs = be.get_state(s, l, orc.d_inner, orc.d_conv)
                cc, cs = orc.state(s, l)
                np.testing.assert_allclose(gc, cc, rtol=1e-4, atol=1e-5)
                np.testing.assert_allclose(gs, cs, rtol=1e-3, atol=1e-5)
        orc.close()


def test_v1_equals_batch8_bit_exact(models):
    with ffi.PluginBackend(models["base"], profile=0) as be:
        v = be.vocab
        seq = [(37 * i + 11) % v for i in range(16)]
        out = np.empty(v, np.float32)
        be.lib.lib.redukt_backend_reset_state()
        v1 = []
        for t in seq:
            rc = be.lib.lib.redukt_backend_forward(t, out.ctypes.data_as(ffi._f32p), v)
            assert rc == ffi.BackendResult.OK
            v1.append(out.copy())
        be.batch_init(8)
        slots = [5, 0, 7, 2, 1, 3, 6, 4]
        other = np.random.default_rng(0).integers(0, v, size=(len(seq), 7))
        for i, t in enumerate(seq):
            g = np.empty((8, v), np.float32)
            be.forward_batch(slots, [t] + [int(x) for x in other[i]], g)
            assert np.array_equal(bits(g[0]), bits(v1[i])), f"step {i}"
        # batch_reset(slot 5) then step 0 == fresh
        be.batch_reset([5])
        g = np.empty((1, v), np.float32)
        be.forward_batch([5], [seq[0]], g)
        assert np.array_equal(bits(g[0]), bits(v1[0]))


@pytest.mark.parametrize("profile", [0, 6])
def test_batch_invariance_any_n_position_slot(models, profile):
    with ffi.PluginBackend(models["reftest"], profile=profile) as be:
        v = be.vocab
        seq = [(13 * i + 5) % v for i in range(5)]
        be.batch_init(72)
        alone = []
        for t in seq:
            g = np.empty((1, v), np.float32)
            be.forward_batch([71], [t], g)
            alone.append(g[0].copy())
        rng = np.random.default_rng(1)
        # with int8 per-row weights (profile 6) n >= 64 takes the four-tile in_proj blocks,
        # n < 64 the two-tile ones; F32 weights take the two-tile blocks at every n
        for n, pos in ((2, 1), (7, 3), (33, 32), (63, 0), (64, 40), (71, 70)):
            be.batch_reset(None)
            slots = [int(s) for s in rng.permutation(71)[:n]]
            for i, t in enumerate(seq):
                toks = [int(x) for x in rng.integers(0, v, n)]
                toks[pos] = t
                g = np.empty((n, v), np.float32)
                be.forward_batch(slots, toks, g)
                assert np.array_equal(bits(g[pos]), bits(alone[i])), (n, pos, i)


@pytest.mark.parametrize("profile", [0, 6])
def test_batch_invariance_streams_per_scan_thread(models, profile):
    # From 256 streams a scan thread runs two streams of its channel, and with an odd
    # count the last pair is half empty.  A stream's bits depend on neither.
    with ffi.PluginBackend(models["reftest"], profile=profile) as be:
        v = be.vocab
        seq = [(29 * i + 3) % v for i in range(4)]
        be.batch_init(520)
        alone = []
        for t in seq:
            g = np.empty((1, v), np.float32)
            be.forward_batch([519], [t], g)
            alone.append(g[0].copy())
        rng = np.random.default_rng(2)
        for n, pos in ((255, 254), (256, 1), (257, 256), (259, 257), (513, 512), (519, 3)):
            be.batch_reset(None)
            slots = [int(s) for s in rng.permutation(519)[:n]]
            for i, t in enumerate(seq):
                toks = [int(x) for x in rng.integers(0, v, n)]
                toks[pos] = t
                g = np.empty((n, v), np.float32)
                be.forward_batch(slots, toks, g)
                assert np.array_equal(bits(g[pos]), bits(alone[i])), (n, pos, i)


def test_run_to_run_bitwise(models):
    results = []
    for _ in range(2):
        with ffi.PluginBackend(models["base"], profile=1) as be:
            v = be.vocab
            outs = run_lockstep(be, None, 5, 8, lambda s, t: (s * 31 + t * 7) % v)
            results.append(np.stack([g for g, _ in outs]))
    assert np.array_equal(bits(results[0]), bits(results[1]))


def test_invalid_arguments_launch_nothing(models):
    with ffi.PluginBackend(models["base"], profile=0) as be:
        v = be.vocab
        be.batch_init(4)
        g = np.empty((2, v), np.float32)
        be.forward_batch([0, 1], [3, 4], g)
        before = [be.get_state(s, l, SMALL_BASE.d_inner, 4) for s in range(4) for l in range(3)]
        L = be.lib.lib
        p = lambda a, t: a.ctypes.data_as(ffi.ctypes.POINTER(t))
        u32, f32 = ffi.ctypes.c_uint32, ffi.ctypes.c_float
        out = np.empty((5, v), np.float32)
        cases = [([1, 1], [0, 0], v), ([4], [0], v), ([0], [v], v), ([0], [0], v + 1), ([0, 1, 2, 3, 0], [0] * 5, v)]
        for slots, toks, vv in cases:
            s = np.array(slots, np.uint32)
            t = np.array(toks, np.uint32)
            rc = L.redukt_backend_forward_batch(len(s), p(s, u32), p(t, u32), p(out, f32), vv)
            assert rc == ffi.BackendResult.INVALID_ARGUMENT, (slots, toks, vv)
        assert L.redukt_backend_forward_batch(1, None, None, None, v) == ffi.BackendResult.INVALID_ARGUMENT
        bad = np.array([4], np.uint32)
        assert L.redukt_backend_batch_reset(p(bad, u32), 1) == ffi.BackendResult.INVALID_ARGUMENT
        assert L.redukt_backend_batch_init(4097) == ffi.BackendResult.INVALID_ARGUMENT
        after = [be.get_state(s, l, SMALL_BASE.d_inner, 4) for s in range(4) for l in range(3)]
        for (c0, s0), (c1, s1) in zip(before, after):
            assert np.array_equal(c0, c1) and np.array_equal(s0, s1)
        assert L.redukt_backend_forward_batch(0, None, None, None, v) == ffi.BackendResult.OK  # n = 0: no-op


def test_periodic_reset_through_the_host_tick(models):
    with ffi.PluginBackend(models["base"], profile=0) as be:
        orc = O.MambaOracle(models["base"], 0, cap=3)
        orc.set_reset_every(4)
        be.prepare_streams(3)
        states = [be.create_state() for _ in range(3)]
        for st in states:
            st.set_reset_every(4)
        v = be.vocab
        seq = [[(s * 17 + t * 5 + 1) % 5 for t in range(10)] for s in range(3)]
        gpu = []
        for t in range(10):
            toks = [seq[s][t] for s in range(3)]
            g = np.empty((3, v), np.float32)
            be.forward_multi(toks, states, g)
            c = orc.forward([0, 1, 2], toks)
            assert_parity(g, c, f"step {t}")
            gpu.append(g)
        for s in range(3):   # forwards 5 and 9 restart from zero state
            if seq[s][4] == seq[s][0]:
                assert np.array_equal(bits(gpu[4][s]), bits(gpu[0][s]))
        orc.close()


def test_probability_vector(models):
    with ffi.PluginBackend(models["reftest"], profile=0) as be:
        orc = O.MambaOracle(models["reftest"], 0, cap=4)
        v = be.vocab
        be.batch_init(4)
        for t in range(3):
            toks = [(s * 7 + t * 3) % v for s in range(4)]
            pg = np.empty((4, v), np.float32)
            be.forward_batch(list(range(4)), toks, pg, probs=True)
            lc = orc.forward(list(range(4)), toks)
            pc = np.stack([O.softmax(r) for r in lc])
            l1 = np.abs(pg.astype(np.float64) - pc).sum(axis=1)
            assert np.all(l1 <= TOL_L1), l1
            assert np.all(np.abs(pg.astype(np.float64).sum(axis=1) - 1.0) < 1e-5)
        orc.close()


@pytest.mark.parametrize("vocab", [51200, 51201])
def test_probability_vector_both_softmax_forms(tmp_path, vocab):
    # Up to 51,200 symbols a row of the softmax is held in registers, above it the kernel
    # walks the row in memory for each phase; both must give the oracle's probabilities.
    path = str(tmp_path / f"v{vocab}.rbin")
    synth.write_synthetic_mamba(path, rbin.MambaDims(vocab=vocab, d_model=64, n_layer=1), seed=11)
    with ffi.PluginBackend(path, profile=0) as be:
        orc = O.MambaOracle(path, 0, cap=3)
        be.batch_init(3)
        for t in range(2):
            toks = [(s * 4099 + t * 977 + 5) % vocab for s in range(3)]
            pg = np.empty((3, vocab), np.float32)
            be.forward_batch(list(range(3)), toks, pg, probs=True)
            lc = orc.forward(list(range(3)), toks)
            pc = np.stack([O.softmax(r) for r in lc])
            l1 = np.abs(pg.astype(np.float64) - pc).sum(axis=1)
            assert np.all(l1 <= TOL_L1), (vocab, t, l1)
            assert np.all(np.abs(pg.astype(np.float64).sum(axis=1) - 1.0) < 1e-5)
        orc.close()


def test_device_resident_entry_point(models):
    with ffi.PluginBackend(models["base"], profile=2) as be:
        v = be.vocab
        be.batch_init(8)
        toks = [[(s * 11 + t * 3) % v for s in range(4)] for t in range(4)]
        host = []
        for t in range(4):
            g = np.empty((4, v), np.float32)
            be.forward_batch([0, 1, 2, 3], toks[t], g)
            host.append(g)
        d_slots = hip.DeviceBuffer.from_array(np.array([7, 6, 5, 4], np.uint32))
        d_toks = hip.DeviceBuffer(16)
        d_out = hip.DeviceBuffer(4 * v * 4)
        try:
            for t in range(4):
                d_toks.upload(np.array(toks[t], np.uint32))
                be.forward_batch_device(4, d_slots.ptr, d_toks.ptr, d_out.ptr)
                assert be.device_status() == ffi.BackendResult.OK
                dev = d_out.download(np.float32, 4 * v).reshape(4, v)
                assert np.array_equal(bits(dev), bits(host[t])), t
            d_toks.upload(np.array([0, 1, v, 2], np.uint32))          # token out of range
            be.forward_batch_device(4, d_slots.ptr, d_toks.ptr, d_out.ptr)
            assert be.device_status() == ffi.BackendResult.INVALID_ARGUMENT
            assert be.device_status() == ffi.BackendResult.OK          # the flag clears
            d_slots.upload(np.array([7, 6, 7, 4], np.uint32))         # duplicate slot
            d_toks.upload(np.array([0, 1, 2, 3], np.uint32))
            be.forward_batch_device(4, d_slots.ptr, d_toks.ptr, d_out.ptr)
            assert be.device_status() == ffi.BackendResult.INVALID_ARGUMENT
        finally:
            for b in (d_slots, d_toks, d_out):
                b.close()


def _device_step(be, slots, toks, v):
    d_s = hip.DeviceBuffer.from_array(np.array(slots, np.uint32))
    d_t = hip.DeviceBuffer.from_array(np.array(toks, np.uint32))
    d_o = hip.DeviceBuffer(len(slots) * v * 4)
    try:
        be.forward_batch_device(len(slots), d_s.ptr, d_t.ptr, d_o.ptr)
        status = be.device_status()
        return status, d_o.download(np.float32, len(slots) * v).reshape(len(slots), v)
    finally:
        for b in (d_s, d_t, d_o):
            b.close()


@pytest.mark.parametrize("profile", [6, ffi.PROFILE_Q8_G64 | ffi.PROFILE_EXACT | ffi.PROFILE_FMA])
def test_device_check_contains_bad_entries(models, profile):
    # A device-checked step with a repeated slot or a bad token routes the offending entries
    # to the pool's scratch slot: slots the call does not name keep their state bit for bit,
    # and the valid entries (a repeated slot's first occurrence included) advance exactly as
    # they would in a valid call (on the matrix-core tier and the reference-order tier).
    dims = SMALL_BASE
    with ffi.PluginBackend(models["base"], profile=profile) as be:
        v = be.vocab
        be.batch_init(8)
        state = lambda s: [be.get_state(s, l, dims.d_inner, 4) for l in range(dims.n_layer)]
        def start():
            be.batch_reset(None)
            st, _ = _device_step(be, [7, 6, 5, 4, 0, 1, 2, 3], [(11 * i + 5) % v for i in range(8)], v)
            assert st == ffi.BackendResult.OK
        start()
        snap = {s: state(s) for s in range(8)}
        st, dup = _device_step(be, [7, 6, 7, 4, 2], [9, 8, 7, 6, v + 3], v)
        assert st == ffi.BackendResult.INVALID_ARGUMENT
        for s in (0, 1, 2, 3, 5):
            for (c0, s0), (c1, s1) in zip(snap[s], state(s)):
                assert np.array_equal(c0, c1) and np.array_equal(s0, s1), s
        after = {s: state(s) for s in (7, 6, 4)}
        start()
        st, ok = _device_step(be, [7, 6, 4], [9, 8, 6], v)
        assert st == ffi.BackendResult.OK
        for pos_dup, pos_ok in ((0, 0), (1, 1), (3, 2)):
            assert np.array_equal(bits(dup[pos_dup]), bits(ok[pos_ok])), pos_dup
        for s in (7, 6, 4):
            for (c0, s0), (c1, s1) in zip(after[s], state(s)):
                assert np.array_equal(c0, c1) and np.array_equal(s0, s1), s


@pytest.mark.parametrize("profile", [0, 1, 6, 14])
def test_mamba130m_parity(full_model, profile):
    with ffi.PluginBackend(full_model, profile=profile) as be:
        orc = O.MambaOracle(full_model, profile, cap=4)
        rng = np.random.default_rng(2)
        toks = synth.zipf_tokens(rng, be.vocab, (6, 4))
        outs = run_lockstep(be, orc, 4, 6, lambda s, t: int(toks[t, s]))
        worst = max(assert_parity(g, c, f"130M p{profile} step {t}") for t, (g, c) in enumerate(outs))
        print(f"Mamba-130M profile {profile}: worst max|dlogit|={worst[0]:.3e} L1={worst[1]:.3e}")
        orc.close()


def test_mamba130m_parity_64_streams(full_model):
    # 64 streams take the four-tile in_proj blocks; the oracle checks every stream.
    with ffi.PluginBackend(full_model, profile=6) as be:
        orc = O.MambaOracle(full_model, 6, cap=64)
        rng = np.random.default_rng(4)
        toks = synth.zipf_tokens(rng, be.vocab, (2, 64))
        outs = run_lockstep(be, orc, 64, 2, lambda s, t: int(toks[t, s]))
        worst = max(assert_parity(g, c, f"130M n64 step {t}") for t, (g, c) in enumerate(outs))
        print(f"Mamba-130M 64 streams: worst max|dlogit|={worst[0]:.3e} L1={worst[1]:.3e}")
        orc.close()


def test_mamba130m_reset_boundary_and_large_batch_invariance(full_model):
    # At the real period (4096 forwards) the 4097th forward restarts from zero state:
    # its logits equal the first forward's, bit for bit.  Checked on the GPU alone.
    with ffi.PluginBackend(full_model, profile=6) as be:
        v = be.vocab
        be.prepare_streams(128)
        states = [be.create_state() for _ in range(2)]
        for st in states:
            st.set_reset_every(4096)
        rng = np.random.default_rng(3)
        seq = synth.zipf_tokens(rng, v, (4097, 2))
        seq[4096] = seq[0]
        out = np.empty((2, v), np.float32)
        first = None
        for t in range(4097):
            be.forward_multi([int(x) for x in seq[t]], states, out)
            if t == 0:
                first = out.copy()
        assert np.array_equal(bits(out), bits(first))
        # The restarted forward is a fresh stream's first forward: the oracle's from zero
        # state, within the parity tolerance.
        orc = O.MambaOracle(full_model, 6, cap=2)
        assert_parity(out, orc.forward([0, 1], [int(x) for x in seq[4096]]), "forward 4097 vs oracle")
        orc.close()
        # A stream inside a 128-stream batch gets the bits it gets alone, at full size.
        tok = int(seq[1, 0])
        be.batch_reset(None)
        alone = np.empty((1, v), np.float32)
        be.forward_batch([127], [tok], alone)
        be.batch_reset(None)
        slots = [int(s) for s in rng.permutation(127)]
        slots.insert(77, 127)
        toks = [int(x) for x in synth.zipf_tokens(rng, v, 128)]
        toks[77] = tok
        g = np.empty((128, v), np.float32)
        be.forward_batch(slots, toks, g)
        assert np.array_equal(bits(g[77]), bits(alone[0]))
        # And inside a 513-stream batch (two streams per scan thread, the last pair half
        # empty), in a full pair and in the half-empty one.
        be.batch_init(520)
        be.forward_batch([519], [tok], alone)
        for pos in (511, 512):
            be.batch_reset(None)
            slots = [int(s) for s in rng.permutation(519)[:512]]
            slots.insert(pos, 519)
            toks = [int(x) for x in synth.zipf_tokens(rng, v, 513)]
            toks[pos] = tok
            g = np.empty((513, v), np.float32)
            be.forward_batch(slots, toks, g)
            assert np.array_equal(bits(g[pos]), bits(alone[0])), pos


def _steps(path, profile, n, steps, seed, probs=False, cap=None):
    rng = np.random.default_rng(seed)
    with ffi.PluginBackend(path, profile=profile) as be:
        v = be.vocab
        be.batch_init(cap or n)
        slots = [int(s) for s in rng.permutation(cap or n)[:n]]
        outs = []
        for _ in range(steps):
            toks = [int(x) for x in rng.integers(0, v, n)]
            g = np.empty((n, v), np.float32)
            be.forward_batch(slots, toks, g, probs=probs)
            outs.append(g)
        return np.stack(outs)


@pytest.mark.parametrize("split", [2, 4])
@pytest.mark.parametrize("n,profile,probs", [(100, 6, False), (33, 0, True), (64, 2, False)])
def test_split_steps_are_bitwise_identical(models, monkeypatch, split, n, profile, probs):
    # A step split into parts of whole 16-stream groups, each part on its own stream,
    # gives every stream the bits of the unsplit step (ragged last parts included).
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "1")
    ref = _steps(models["reftest"], profile, n, 3, 5, probs, cap=n + 7)
    monkeypatch.setenv("REDUKT_GPU_PART_MIN", "16")
    monkeypatch.setenv("REDUKT_GPU_SPLIT", str(split))
    got = _steps(models["reftest"], profile, n, 3, 5, probs, cap=n + 7)
    assert np.array_equal(bits(ref), bits(got))


def test_split_mamba130m_128_streams_bitwise(full_model, monkeypatch):
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "1")
    ref = _steps(full_model, 6, 128, 2, 9)
    monkeypatch.setenv("REDUKT_GPU_PART_MIN", "16")
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "4")
    got = _steps(full_model, 6, 128, 2, 9)
    assert np.array_equal(bits(ref), bits(got))


def test_default_split_mamba130m_112_streams_bitwise(full_model, monkeypatch):
    # The default split of 112 streams (parts of 64 and 48 streams, out_proj at two row
    # tiles per workgroup) gives every stream the bits of the unsplit step.
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "1")
    ref = _steps(full_model, 6, 112, 2, 13)
    monkeypatch.delenv("REDUKT_GPU_SPLIT")
    monkeypatch.delenv("REDUKT_GPU_PART_MIN", raising=False)
    got = _steps(full_model, 6, 112, 2, 13)
    assert np.array_equal(bits(ref), bits(got))


@pytest.mark.parametrize("tiles", [2, 3, 4])
def test_out_proj_tiles_per_workgroup_are_bitwise_identical(full_model, monkeypatch, tiles):
    # out_proj workgroups covering several row tiles (read each stream group's gated tiles
    # once for all of them) give every stream the bits of one tile per workgroup.
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "1")
    monkeypatch.setenv("REDUKT_GPU_OUT_TILES", "1")
    ref = _steps(full_model, 6, 48, 2, 11)
    monkeypatch.setenv("REDUKT_GPU_OUT_TILES", str(tiles))
    got = _steps(full_model, 6, 48, 2, 11)
    assert np.array_equal(bits(ref), bits(got))


def test_split_device_check_covers_every_part(models, monkeypatch):
    # A slot repeated in two different parts is caught by the device check of the whole
    # step: the later entry never touches the real slot, the first advances it exactly as a
    # valid call does, and the slot the later position would otherwise name is untouched.
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "4")
    monkeypatch.setenv("REDUKT_GPU_PART_MIN", "16")
    dims = SMALL_BASE
    with ffi.PluginBackend(models["base"], profile=0) as be:
        v = be.vocab
        be.batch_init(64)
        state = lambda s: [be.get_state(s, l, dims.d_inner, 4) for l in range(dims.n_layer)]
        first = [(7 * i + 1) % v for i in range(64)]
        toks = [(5 * i + 2) % v for i in range(64)]

        def start():
            be.batch_reset(None)
            st, _ = _device_step(be, list(range(64)), first, v)
            assert st == ffi.BackendResult.OK

        start()
        s60 = state(60)
        slots = list(range(64))
        slots[60] = 3       # part 3 repeats part 0's slot 3
        st, bad = _device_step(be, slots, toks, v)
        assert st == ffi.BackendResult.INVALID_ARGUMENT
        s3_bad = state(3)
        for (c0, x0), (c1, x1) in zip(s60, state(60)):
            assert np.array_equal(c0, c1) and np.array_equal(x0, x1)
        start()
        keep = [i for i in range(64) if i != 60]
        st, good = _device_step(be, [slots[i] for i in keep], [toks[i] for i in keep], v)
        assert st == ffi.BackendResult.OK
        for (c0, x0), (c1, x1) in zip(s3_bad, state(3)):
            assert np.array_equal(c0, c1) and np.array_equal(x0, x1)
        assert np.array_equal(bits(bad[keep]), bits(good))
