"""GPU parity of the RWKV-7 step (libredukt_gpu.so through the C ABI) against the CPU
oracle: logits within max |Δ| <= 1e-3 and probability L1 <= 1e-4 (the tolerances of the
Mamba tests), states within float tolerance, and the bitwise properties of the plugin
contract (docs/api/PLUGIN-FFI-V2.md:85-108): v1 == batch at any position and slot,
batch invariance over n, run-to-run identity, reset == fresh stream."""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, hip, rwkv

pytestmark = pytest.mark.gpu

TOL_ABS = 1e-3
TOL_L1 = 1e-4
SMALL = rwkv.RwkvDims(vocab=300, d_model=128, n_layer=2, head_size=64, d_ffn=256, lora_w=16, lora_a=16,
                      lora_v=8, lora_g=32)
# RWKV-7 0.1B layers at full width and depth; vocabulary cut to 4096 to keep the CPU side
# of the test short (the head is the same kernel at any vocabulary).
WIDE = dataclasses.replace(rwkv.RWKV7_0_1B, vocab=4096)


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
def rwkv_models(tmp_path_factory):
    assert hip.device_count() > 0, "no GPU visible"
    d = tmp_path_factory.mktemp("rwkv_models")
    out = {"small": str(d / "small.rbin"), "g1k": str(d / "g1k.rbin")}
    rwkv.write_synthetic(out["small"], SMALL, seed=1)
    rwkv.write_synthetic(out["g1k"], dataclasses.replace(SMALL, g1k=True, n_layer=3), seed=2)
    return out


@pytest.fixture(scope="session")
def wide_model(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("rwkv_wide") / "wide.rbin")
    rwkv.write_synthetic(p, WIDE, seed=0)
    return p


def lockstep(be, orc, n, steps, tok_fn, slots=None):
    slots = slots or list(range(n))
    outs = []
    for t in range(steps):
        toks = [tok_fn(s, t) for s in range(n)]
        g = np.empty((n, be.vocab), np.float32)
        be.forward_batch(slots, toks, g)
        outs.append((g, orc.forward(list(range(n)), toks) if orc is not None else None))
    return outs


@pytest.mark.parametrize("name,profile", [("small", 0), ("small", 1), ("small", 2), ("g1k", 0), ("g1k", 2)])
def test_small_rwkv_parity(rwkv_models, name, profile):
    path = rwkv_models[name]
    with ffi.PluginBackend(path, profile=profile) as be:
        assert bytes(be.info.name).rstrip(b"\0").startswith(b"hip-gfx950-rwkv7")
        orc = O.RwkvOracle(path, profile, cap=19)
        be.batch_init(19)
        v = be.vocab
        outs = lockstep(be, orc, 19, 6, lambda s, t: (s * 37 + t * 101 + 3) % v)
        for t, (g, c) in enumerate(outs):
            assert_parity(g, c, f"{name} p{profile} step {t}")
        for layer in range(orc.n_layer):
            for s in (0, 18):
                ga, gw, gf = be.get_rwkv_state(s, layer, orc.d_model, orc.n_head)
                ca, cw, cf = orc.state(s, layer)
                np.testing.assert_allclose(ga, ca, rtol=1e-4, atol=2e-5)
                np.testing.assert_allclose(gf, cf, rtol=1e-4, atol=2e-5)
                np.testing.assert_allclose(gw, cw, rtol=1e-3, atol=2e-5)
        orc.close()


def test_rwkv_v1_equals_batch_bit_exact(rwkv_models):
    with ffi.PluginBackend(rwkv_models["small"], profile=0) as be:
        v = be.vocab
        seq = [(37 * i + 11) % v for i in range(8)]
        out = np.empty(v, np.float32)
        be.lib.lib.redukt_backend_reset_state()
        v1 = []
        for t in seq:
            assert be.lib.lib.redukt_backend_forward(t, out.ctypes.data_as(ffi._f32p), v) == ffi.BackendResult.OK
            v1.append(out.copy())
        be.batch_init(24)
        rng = np.random.default_rng(0)
        for n, pos in ((1, 0), (5, 3), (17, 16), (24, 9)):
            be.batch_reset(None)
            slots = [int(s) for s in rng.permutation(24)[:n]]
            for i, t in enumerate(seq):
                toks = [int(x) for x in rng.integers(0, v, n)]
                toks[pos] = t
                g = np.empty((n, v), np.float32)
                be.forward_batch(slots, toks, g)
                assert np.array_equal(bits(g[pos]), bits(v1[i])), (n, pos, i)


def test_rwkv_run_to_run_and_reset(rwkv_models):
    runs = []
    for _ in range(2):
        with ffi.PluginBackend(rwkv_models["small"], profile=2) as be:
            be.batch_init(8)
            outs = lockstep(be, None, 8, 5, lambda s, t: (s * 7 + t * 13) % be.vocab)
            runs.append(np.stack([g for g, _ in outs]))
            # reset slot 3, then its next step equals a fresh stream's first step
            be.batch_reset([3])
            g = np.empty((1, be.vocab), np.float32)
            be.forward_batch([3], [42], g)
            be.batch_init(1)
            f = np.empty((1, be.vocab), np.float32)
            be.forward_batch([0], [42], f)
            assert np.array_equal(bits(g), bits(f))
    assert np.array_equal(bits(runs[0]), bits(runs[1]))


def test_rwkv_periodic_reset_and_probabilities(rwkv_models):
    """The host's tick schedule (plugin_backend/model.rs:44-49) through forward_multi,
    against the oracle's periodic reset; odd steps return the probability vector."""
    with ffi.PluginBackend(rwkv_models["small"], profile=0) as be:
        orc = O.RwkvOracle(rwkv_models["small"], 0, cap=4)
        orc.set_reset_every(3)
        be.prepare_streams(4)
        states = [be.create_state() for _ in range(4)]
        for st in states:
            st.set_reset_every(3)
        for t in range(7):
            toks = [(t * 5 + s) % be.vocab for s in range(4)]
            g = np.empty((4, be.vocab), np.float32)
            be.forward_multi(toks, states, g)
            c = orc.forward(list(range(4)), toks)
            assert_parity(g, c, f"periodic step {t}")
        slots = [st.slot for st in states]
        p = np.empty((4, be.vocab), np.float32)
        toks = [3, 1, 4, 1]
        be.forward_batch(slots, toks, p, probs=True)
        c = orc.forward(list(range(4)), toks)
        ref = np.stack([O.softmax(r) for r in c])
        assert float(np.max(np.abs(p - ref).sum(axis=-1))) <= TOL_L1
        assert np.allclose(p.sum(axis=-1), 1.0, atol=1e-5)
        orc.close()


@pytest.mark.parametrize("profile", [0, 2])
def test_rwkv7_0_1b_layers_parity(wide_model, profile):
    with ffi.PluginBackend(wide_model, profile=profile) as be:
        orc = O.RwkvOracle(wide_model, profile, cap=4)
        be.batch_init(64)
        slots = [60, 2, 33, 7]
        outs = lockstep(be, orc, 4, 3, lambda s, t: (s * 911 + t * 37 + 1) % be.vocab, slots=slots)
        for t, (g, c) in enumerate(outs):
            assert_parity(g, c, f"0.1B p{profile} step {t}")
        orc.close()


def _rwkv_steps(path, profile, n, steps, seed, probs=False):
    rng = np.random.default_rng(seed)
    with ffi.PluginBackend(path, profile=profile) as be:
        be.batch_init(n + 5)
        slots = [int(s) for s in rng.permutation(n + 5)[:n]]
        outs = []
        for _ in range(steps):
            toks = [int(x) for x in rng.integers(0, be.vocab, n)]
            g = np.empty((n, be.vocab), np.float32)
            be.forward_batch(slots, toks, g, probs=probs)
            outs.append(g)
        return np.stack(outs)


@pytest.mark.parametrize("split", [2, 4])
@pytest.mark.parametrize("profile,probs", [(0, False), (2, True), (2 | ffi.PROFILE_W8A8, False)])
def test_rwkv_split_steps_are_bitwise_identical(rwkv_models, monkeypatch, split, profile, probs):
    # A step split into parts of whole 16-stream groups (a ragged last part included), each
    # part on its own stream, gives every stream the bits of the unsplit step; the W8A8 tier
    # runs its steps in one part whatever the split asks.
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "1")
    ref = _rwkv_steps(rwkv_models["g1k"], profile, 50, 3, 17, probs)
    monkeypatch.setenv("REDUKT_GPU_PART_MIN", "16")
    monkeypatch.setenv("REDUKT_GPU_SPLIT", str(split))
    got = _rwkv_steps(rwkv_models["g1k"], profile, 50, 3, 17, probs)
    assert np.array_equal(bits(ref), bits(got))


@pytest.mark.parametrize("tiles", [2, 4])
@pytest.mark.parametrize("profile", [0, 1, 2])
def test_rwkv_projection_tiles_per_workgroup_are_bitwise_identical(rwkv_models, monkeypatch, tiles, profile):
    # Projection workgroups covering several row tiles (one load of the activation
    # fragments for all of them; segments of one tile, LoRA ranks below 16 rows, included)
    # give every stream the bits of one tile per workgroup.
    monkeypatch.setenv("REDUKT_GPU_SPLIT", "1")
    monkeypatch.setenv("REDUKT_GPU_PROJ_TILES", "1")
    ref = _rwkv_steps(rwkv_models["g1k"], profile, 50, 3, 19, True)
    monkeypatch.setenv("REDUKT_GPU_PROJ_TILES", str(tiles))
    got = _rwkv_steps(rwkv_models["g1k"], profile, 50, 3, 19, True)
    assert np.array_equal(bits(ref), bits(got))


@pytest.mark.parametrize("tiles", [2, 4])
def test_rwkv7_0_1b_projection_tiles_bitwise(wide_model, monkeypatch, tiles):
    monkeypatch.setenv("REDUKT_GPU_PROJ_TILES", "1")
    ref = _rwkv_steps(wide_model, 2, 20, 2, 23)
    monkeypatch.setenv("REDUKT_GPU_PROJ_TILES", str(tiles))
    got = _rwkv_steps(wide_model, 2, 20, 2, 23)
    assert np.array_equal(bits(ref), bits(got))


@pytest.mark.parametrize("profile", [0, 2])
def test_rwkv_batch_invariance_across_split_sizes(rwkv_models, profile):
    # Default settings: below 96 streams one part with one projection tile per workgroup,
    # from 96 two parts with four; a stream's bits depend on neither its batch, its
    # position nor its slot.
    with ffi.PluginBackend(rwkv_models["small"], profile=profile) as be:
        v = be.vocab
        seq = [(53 * i + 7) % v for i in range(4)]
        be.batch_init(140)
        alone = []
        for t in seq:
            g = np.empty((1, v), np.float32)
            be.forward_batch([139], [t], g)
            alone.append(g[0].copy())
        rng = np.random.default_rng(4)
        for n, pos in ((95, 94), (96, 0), (113, 64), (139, 100)):
            be.batch_reset(None)
            slots = [int(s) for s in rng.permutation(139)[:n]]
            for i, t in enumerate(seq):
                toks = [int(x) for x in rng.integers(0, v, n)]
                toks[pos] = t
                g = np.empty((n, v), np.float32)
                be.forward_batch(slots, toks, g)
                assert np.array_equal(bits(g[pos]), bits(alone[i])), (n, pos, i)


@pytest.mark.parametrize("profile", [0, 2])
def test_rwkv7_0_1b_64_streams_2048_tokens(wide_model, profile):
    # The RWKV-7 workload (F32 and int8 per-row) at its full horizon: 64 lockstep streams of uniform
    # byte ids for 2,048 tokens (RWKV-7 0.1B layers, vocabulary cut to 4,096), every 4th
    # stream (16 of them) compared with the oracle at every token within the logit and
    # probability tolerances; drift in the 64x64 WKV state or the token-shift state would
    # show as a growing error.  About a minute of oracle steps on 16 host threads.
    n, steps = 64, 2048
    watch = list(range(0, n, 4))
    rng = np.random.default_rng(2048)
    toks = rng.integers(0, 256, size=(steps, n))
    with ffi.PluginBackend(wide_model, profile=profile) as be:
        orc = O.RwkvOracle(wide_model, profile, cap=len(watch))
        be.batch_init(n)
        g = np.empty((n, be.vocab), np.float32)
        worst = 0.0
        for t in range(steps):
            row = [int(x) for x in toks[t]]
            be.forward_batch(list(range(n)), row, g)
            c = orc.forward(list(range(len(watch))), [row[s] for s in watch])
            err, _ = assert_parity(g[watch], c, f"step {t}")
            worst = max(worst, err)
            if t % 256 == 255:
                print(f"step {t + 1}: max |dlogit| so far {worst:.2e}", flush=True)
        orc.close()
