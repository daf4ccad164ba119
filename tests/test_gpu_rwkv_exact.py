"""RWKV-7 in the reference's own arithmetic on the GPU, through the C ABI, against the
oracle: the W8A8 tier (profile bit 5 with per-row int8 weights) against the oracle's W8A8
path (the reference's RWKV-7 Q8 arithmetic, src/domain/tensor.rs:105-143, 1791-1866), and
the F32 reference-order tier (profile bit 6) against the oracle's F32 path (every
projection in mat_vec_mul_into's dot_avx2_order, tensor.rs:1602-1693).

In both tiers every matrix product is either an exact integer sum or the reference's own
f32 dot order, and every other operation follows the reference's order, sums included, so
the bar is bit-exact equality with the oracle: logits at every step and every stream, the
recurrent state of every layer, on a small model, a g1k model and the full-width RWKV-7
0.1B (vocabulary 65,536), with periodic resets, slots in any order and batches of any size.
The probability vector is held to the tolerance of the other tiers (the softmax is shared
with them).  Since the bits are the CPU path's, an archive coded on the CPU (the oracle
behind the plugin ABI) decodes on the GPU, the GPU codes the same bytes, and an RDKT v5
archive of the RWKV-7 backbone written on the GPU decodes on the CPU from its header alone.
"""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import archive, ffi, hip, rwkv
from redukt_amd.lockstep import Lockstep

pytestmark = pytest.mark.gpu

A8 = ffi.PROFILE_Q8_ROW | ffi.PROFILE_W8A8
REF = ffi.PROFILE_EXACT
# tier: (library profile, oracle profile, backend name)
TIERS = {"w8a8": (A8, A8, "hip-gfx950-rwkv7-w8a8"), "f32-ref": (REF, 0, "hip-gfx950-rwkv7-f32-ref")}
# the RDKT header's weight-profile code of each tier (the reference's RWKV-7 Q8 is W8A8)
SMALL = rwkv.RwkvDims(vocab=300, d_model=128, n_layer=2, head_size=64, d_ffn=256, lora_w=16, lora_a=16,
                      lora_v=8, lora_g=32)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def models(tmp_path_factory):
    assert hip.device_count() > 0, "no GPU visible"
    d = tmp_path_factory.mktemp("rwkv_a8")
    out = {"small": str(d / "small.rbin"), "g1k": str(d / "g1k.rbin"), "b01": str(d / "b01.rbin"),
           "odd": str(d / "odd.rbin")}
    rwkv.write_synthetic(out["small"], SMALL, seed=1)
    rwkv.write_synthetic(out["g1k"], dataclasses.replace(SMALL, g1k=True, n_layer=3), seed=2)
    rwkv.write_synthetic(out["b01"], rwkv.RWKV7_0_1B, seed=0)
    rwkv.write_synthetic(out["odd"], dataclasses.replace(SMALL, lora_v=12), seed=3)
    return out


def first_diff(g, c):
    bad = np.flatnonzero(bits(g).ravel() != bits(c).ravel())
    if not bad.size:
        return None
    i = int(bad[0])
    return i, float(g.ravel()[i]), float(c.ravel()[i]), int(bad.size)


def run_equal(be, orc, n, steps, tok_fn, slots=None, states=()):
    slots = slots or list(range(n))
    for t in range(steps):
        toks = [tok_fn(s, t) for s in range(n)]
        g = np.empty((n, be.vocab), np.float32)
        be.forward_batch(slots, toks, g)
        c = orc.forward(slots, toks)
        assert first_diff(g, c) is None, (t, first_diff(g, c))
    for s in states:
        for layer in range(orc.n_layer):
            for got, want, what in zip(be.get_rwkv_state(s, layer, orc.d_model, orc.n_head), orc.state(s, layer),
                                       ("x_att", "wkv", "x_ffn")):
                assert np.array_equal(bits(got), bits(want)), (s, layer, what)


@pytest.fixture(params=sorted(TIERS))
def tier(request):
    return TIERS[request.param]


@pytest.mark.parametrize("name", ["small", "g1k"])
def test_bit_exact_small(models, name, tier):
    path = models[name]
    prof, oprof, label = tier
    with ffi.PluginBackend(path, profile=prof) as be:
        assert be.info.name_str() == label
        orc = O.RwkvOracle(path, oprof, cap=19)
        be.batch_init(19)
        run_equal(be, orc, 19, 8, lambda s, t: (s * 37 + t * 101 + 3) % be.vocab, states=(0, 7, 18))
        orc.close()


def test_long_horizon(models, tier):
    """8 streams for 400 steps on the g1k model: every logit and the final state, bit for bit."""
    path = models["g1k"]
    prof, oprof, _ = tier
    with ffi.PluginBackend(path, profile=prof) as be:
        orc = O.RwkvOracle(path, oprof, cap=8)
        be.batch_init(8)
        run_equal(be, orc, 8, 400, lambda s, t: (s * 97 + t * 31 + 11) % be.vocab, states=(0, 5))
        orc.close()


def test_bit_exact_rwkv7_0_1b(models, tier):
    path = models["b01"]
    prof, oprof, _ = tier
    with ffi.PluginBackend(path, profile=prof) as be:
        assert be.vocab == 65536
        orc = O.RwkvOracle(path, oprof, cap=40)
        be.batch_init(40)
        rng = np.random.default_rng(5)
        # 40 streams: two full groups of 16 and a partial one; slots in scrambled order
        slots = [int(s) for s in rng.permutation(40)]
        orc_slots = slots
        for t in range(4):
            toks = [int(x) for x in rng.integers(0, 65536, 40)]
            g = np.empty((40, 65536), np.float32)
            be.forward_batch(slots, toks, g)
            c = orc.forward(orc_slots, toks)
            assert first_diff(g, c) is None, (t, first_diff(g, c))
        for s in (slots[0], slots[39]):
            for layer in (0, 11):
                for got, want in zip(be.get_rwkv_state(s, layer, 768, 12), orc.state(s, layer)):
                    assert np.array_equal(bits(got), bits(want)), (s, layer)
        orc.close()


def test_batch_sizes_and_v1(models, tier):
    """One stream's bits do not depend on the batch it runs in, its position or its slot,
    and the v1 single-stream entry point gives the same bits."""
    path = models["small"]
    with ffi.PluginBackend(path, profile=tier[0]) as be:
        v = be.vocab
        seq = [(53 * i + 7) % v for i in range(6)]
        out = np.empty(v, np.float32)
        be.lib.lib.redukt_backend_reset_state()
        v1 = []
        for t in seq:
            assert be.lib.lib.redukt_backend_forward(t, out.ctypes.data_as(ffi._f32p), v) == ffi.BackendResult.OK
            v1.append(out.copy())
        be.batch_init(40)
        rng = np.random.default_rng(1)
        for n, pos in ((1, 0), (16, 15), (17, 16), (40, 23)):
            be.batch_reset(None)
            slots = [int(s) for s in rng.permutation(40)[:n]]
            for i, t in enumerate(seq):
                toks = [int(x) for x in rng.integers(0, v, n)]
                toks[pos] = t
                g = np.empty((n, v), np.float32)
                be.forward_batch(slots, toks, g)
                assert np.array_equal(bits(g[pos]), bits(v1[i])), (n, pos, i)


def test_periodic_reset_and_probabilities(models, tier):
    """The host's tick schedule (plugin_backend/model.rs:44-49) against the oracle's
    periodic reset, bit for bit; odd steps hand back the probability vector."""
    path = models["small"]
    prof, oprof, _ = tier
    with ffi.PluginBackend(path, profile=prof) as be:
        orc = O.RwkvOracle(path, oprof, cap=6)
        orc.set_reset_every(3)
        be.prepare_streams(6)
        states = [be.create_state() for _ in range(6)]
        assert [st.slot for st in states] == list(range(6))
        for st in states:
            st.set_reset_every(3)
        for t in range(8):
            toks = [(s * 31 + t * 17 + 1) % be.vocab for s in range(6)]
            c = orc.forward(list(range(6)), toks)
            g = np.empty((6, be.vocab), np.float32)
            if t % 2 == 0:
                be.forward_multi(toks, states, g)
                assert first_diff(g, c) is None, (t, first_diff(g, c))
            else:
                for st in states:
                    st.tick()
                be.forward_batch([st.slot for st in states], toks, g, probs=True)
                ref = np.stack([O.softmax(r) for r in c])
                assert float(np.max(np.abs(g - ref).sum(axis=-1))) <= 1e-4
                assert np.allclose(g.sum(axis=-1), 1.0, atol=1e-5)
        orc.close()


def test_run_to_run(models, tier):
    runs = []
    for _ in range(2):
        with ffi.PluginBackend(models["small"], profile=tier[0]) as be:
            be.batch_init(8)
            g = np.empty((8, be.vocab), np.float32)
            outs = []
            for t in range(4):
                be.forward_batch(list(range(8)), [(s * 7 + t * 13) % be.vocab for s in range(8)], g)
                outs.append(g.copy())
            runs.append(np.stack(outs))
    assert np.array_equal(bits(runs[0]), bits(runs[1]))


def test_w8a8_init_rules(models, tmp_path):
    lib = ffi.PluginLibrary()
    try:
        # Mamba models, group-64 weights and F32 have no W8A8 tier
        mamba = str(tmp_path / "m.rbin")
        from redukt_amd import rbin, synth
        synth.write_synthetic_mamba(mamba, rbin.MambaDims(vocab=300, d_model=64, n_layer=1), seed=1)
        for path, prof in ((mamba, A8), (models["small"], ffi.PROFILE_W8A8 | 1), (models["small"], ffi.PROFILE_W8A8),
                           (models["odd"], A8)):
            with pytest.raises(ffi.BackendError):
                lib.init(path, profile=prof)
            lib.free()
        info = lib.init(models["odd"], profile=ffi.PROFILE_Q8_ROW)   # rank 12 is fine without W8A8
        assert info.name_str() == "hip-gfx950-rwkv7-q8row"
    finally:
        lib.free()


@pytest.mark.parametrize("name", sorted(TIERS))
def test_named_profiles_from_the_environment(models, monkeypatch, name):
    monkeypatch.setenv("REDUKT_GPU_PROFILE", {"w8a8": "q8row-w8a8", "f32-ref": "f32-ref"}[name])
    lib = ffi.PluginLibrary()
    try:
        assert lib.init(models["small"]).name_str() == TIERS[name][2]
    finally:
        lib.free()


def test_reference_order_init_rules(models):
    """RWKV-7's reference-order tier is F32 in numeric contract 1 only: its int8 arithmetic
    is the W8A8 tier's, and the reference's RWKV-7 GEMVs have no fma-v1 twin."""
    lib = ffi.PluginLibrary()
    try:
        for path, prof in ((models["small"], REF | ffi.PROFILE_Q8_G64), (models["small"], REF | ffi.PROFILE_Q8_ROW),
                           (models["small"], REF | ffi.PROFILE_FMA), (models["small"], ffi.PROFILE_FMA),
                           (models["small"], REF | A8), (models["odd"], REF)):
            with pytest.raises(ffi.BackendError):
                lib.init(path, profile=prof)
            lib.free()
    finally:
        lib.free()


def test_archives_cross_devices(models, oracle_plugin, tier):
    """Lockstep coding of several files (crossing reset boundaries) on the CPU oracle and on
    the GPU gives the same bytes, each side decodes the other's, and GPU streams packed
    into RDKT v5 archives of the RWKV-7 backbone decode on the CPU with the restored data's
    CRC-32 (src/application/codec.rs:540-580, 648-741).  Those archives are what the
    reference writes for RWKV (FORMAT-SPEC.md:224-240): BACKBONE 0, PROFILE 0x10 (RWKV's
    quantisation is not part of the format: both ends run the same configuration) and no
    reset period (RWKV never resets, model_loader.rs:121-128), so their streams are coded
    without resets."""
    prof, oprof, _ = tier
    path = models["g1k"]
    rng = np.random.default_rng(9 + prof)
    files = [rng.integers(0, SMALL.vocab, k).astype(np.uint32) for k in (300, 1, 90, 520)]
    print(f"rwkv cross-device round trip profile {prof}", flush=True)
    with Lockstep(path, plugin_path=oracle_plugin, profile=oprof, slots=3) as cpu:
        cpu_bytes, _ = cpu.compress(files, reset_every=256)
    with Lockstep(path, profile=prof, slots=3) as gpu:
        gpu_bytes, _ = gpu.compress(files, reset_every=256)
        assert gpu_bytes == cpu_bytes, "the GPU codes other bytes than the CPU"
        back, _ = gpu.decompress(cpu_bytes, [len(f) for f in files], reset_every=256)
    for f, b in zip(files, back):
        assert np.array_equal(f, b)
    with Lockstep(path, profile=prof, slots=3) as gpu:
        arc_streams, _ = gpu.compress(files, reset_every=0)
    for f, stm in zip(files, arc_streams):
        payload = f.astype("<u4").tobytes()
        h = archive.default_header(len(payload), backbone=archive.BACKBONE_RWKV, quant=0, reset_log2=0)
        arc = archive.pack(h, stm, payload)
        assert arc[12:14] == bytes([0x00, 0x10])
        hd, body, crc = archive.unpack(arc)
        assert (hd.backbone, hd.quant, hd.contract, hd.reset_every) == (archive.BACKBONE_RWKV, 0, 1, 0)
        with Lockstep(path, plugin_path=oracle_plugin, profile=oprof, slots=1) as cpu:
            back, _ = cpu.decompress([body], [hd.total_bytes // 4], reset_every=hd.reset_every)
        assert archive.crc32(back[0].astype("<u4").tobytes()) == crc
        assert np.array_equal(back[0], f)


def _device_step(be, slots, toks):
    v = be.vocab
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


@pytest.mark.parametrize("profile", [ffi.PROFILE_Q8_ROW, A8, REF])
def test_device_check_contains_bad_entries(models, profile):
    """RWKV-7 through forward_batch_device (matrix-core int8, W8A8 and F32 reference-order
    tiers): a valid call equals forward_batch bit for bit; a call with a repeated slot and a
    bad token reports INVALID_ARGUMENT, leaves the slots it does not name untouched, and
    advances its valid entries exactly as a valid call would."""
    d, h = SMALL.d_model, SMALL.d_model // 64
    with ffi.PluginBackend(models["small"], profile=profile) as be:
        v = be.vocab
        be.batch_init(8)
        state = lambda s: [be.get_rwkv_state(s, l, d, h) for l in range(SMALL.n_layer)]
        first = [(13 * i + 5) % v for i in range(8)]

        def start():
            be.batch_reset(None)
            st, out = _device_step(be, [7, 6, 5, 4, 0, 1, 2, 3], first)
            assert st == ffi.BackendResult.OK
            return out

        dev = start()
        be.batch_reset(None)
        host = np.empty((8, v), np.float32)
        be.forward_batch([7, 6, 5, 4, 0, 1, 2, 3], first, host)
        assert np.array_equal(bits(dev), bits(host))
        start()
        snap = {s: state(s) for s in range(8)}
        st, dup = _device_step(be, [7, 6, 7, 4, 2], [9, 8, 7, 6, v + 3])
        assert st == ffi.BackendResult.INVALID_ARGUMENT
        for s in (0, 1, 2, 3, 5):
            for a, b in zip(snap[s], state(s)):
                for x, y in zip(a, b):
                    assert np.array_equal(bits(x), bits(y)), s
        after = {s: state(s) for s in (7, 6, 4)}
        start()
        st, ok = _device_step(be, [7, 6, 4], [9, 8, 6])
        assert st == ffi.BackendResult.OK
        for pos_dup, pos_ok in ((0, 0), (1, 1), (3, 2)):
            assert np.array_equal(bits(dup[pos_dup]), bits(ok[pos_ok])), pos_dup
        for s in (7, 6, 4):
            for a, b in zip(after[s], state(s)):
                for x, y in zip(a, b):
                    assert np.array_equal(bits(x), bits(y)), s
