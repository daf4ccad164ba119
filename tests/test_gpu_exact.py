"""The reference-order tier (weight profile bits 6 and 7) on the GPU, through the C ABI.

The tier computes every projection in the reference CPU path's own GEMV order and both of
its numeric contracts (contract 1, and with bit 7 contract 2 / fma-v1, gemv_fma.rs), with
sequential norms and the portable exp in the scan, so:

* the logits equal the CPU oracle's bit for bit, step after step, for F32, group-64 and
  per-row int8 weights (x_proj / dt_proj quantized too), RMSNorm and LayerNorm models,
  tied and untied heads, and full Mamba-130M; so does every layer's recurrent state;
* therefore a stream's bits do not depend on n, position or slot, and v1 equals batch;
* an archive coded on the CPU (the oracle behind the plugin ABI) decodes on the GPU and
  the GPU codes the same bytes: the reference's numeric contracts carry across devices.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import archive, ffi, hip, rbin, synth
from redukt_amd.lockstep import Lockstep

pytestmark = pytest.mark.gpu

EXACT = ffi.PROFILE_EXACT
FMA = ffi.PROFILE_FMA
SMALL = {"reftest": rbin.MambaDims(vocab=1200, d_model=64, n_layer=2),
         "base": rbin.MambaDims(vocab=1000, d_model=96, n_layer=3),
         "bias_untied": rbin.MambaDims(vocab=500, d_model=64, n_layer=2)}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    assert hip.device_count() > 0, "no GPU visible"
    d = tmp_path_factory.mktemp("exact_models")
    out = {k: str(d / f"{k}.rbin") for k in SMALL}
    synth.write_synthetic_mamba(out["reftest"], SMALL["reftest"], init="reference-test")
    synth.write_synthetic_mamba(out["base"], SMALL["base"], seed=7)
    synth.write_synthetic_mamba(out["bias_untied"], SMALL["bias_untied"], seed=3,
                                flags=rbin.FLAG_NORM_BIAS | rbin.FLAG_UNTIED_HEAD)
    return out


def check_bitwise(path, dims, profile, contract, n, steps, slots=None, seed=1):
    """n streams (in `slots`) for `steps` steps on the GPU and on the oracle: every logit and,
    at the end, every layer's conv and SSM state equal bit for bit."""
    slots = list(range(n)) if slots is None else slots
    cap = max(slots) + 1
    rng = np.random.default_rng(seed)
    print(f"exact tier {os.path.basename(path)} profile {profile} contract {contract} n {n}", flush=True)
    with ffi.PluginBackend(path, profile=profile | EXACT | (FMA if contract == 2 else 0)) as be:
        orc = O.MambaOracle(path, profile | (O.ORC_PROFILE_FMA if contract == 2 else 0), cap=cap)
        be.batch_init(cap)
        for t in range(steps):
            toks = [int(x) for x in synth.zipf_tokens(rng, dims.vocab, (n,))]
            g = np.empty((n, dims.vocab), np.float32)
            be.forward_batch(slots, toks, g)
            c = orc.forward(slots, toks)
            if not np.array_equal(bits(g), bits(c)):
                bad = np.argwhere(bits(g) != bits(c))
                err = float(np.max(np.abs(g.astype(np.float64) - c)))
                raise AssertionError(f"step {t}: {len(bad)} logits differ (first {bad[0].tolist()}), max|d|={err:.3e}")
        for s in slots:
            for layer in range(dims.n_layer):
                gc, gs = be.get_state(s, layer, dims.d_inner, dims.d_conv)
                cc, cs = orc.state(s, layer)
                assert np.array_equal(bits(gc), bits(cc)), ("conv", s, layer)
                assert np.array_equal(bits(gs), bits(cs)), ("ssm", s, layer)
        orc.close()


@pytest.mark.parametrize("contract", [1, 2])
@pytest.mark.parametrize("name,profile", [("reftest", 0), ("reftest", 1), ("base", 0), ("base", 1), ("base", 2),
                                          ("base", 6), ("base", 5), ("bias_untied", 0), ("bias_untied", 1)])
def test_exact_tier_equals_oracle_bit_for_bit(small, name, profile, contract):
    check_bitwise(small[name], SMALL[name], profile, contract, n=5, steps=6, slots=[3, 0, 6, 1, 4])


@pytest.mark.parametrize("contract", [1, 2])
@pytest.mark.parametrize("profile", [0, 1])
def test_exact_tier_wide_batch(small, profile, contract):
    # 37 streams: the projections' workgroups of four streams and the head's of eight, each
    # with a partial last group; slots scrambled over a pool of 40
    slots = [int(s) for s in np.random.default_rng(3).permutation(40)[:37]]
    check_bitwise(small["base"], SMALL["base"], profile, contract, n=37, steps=3, slots=slots, seed=11)


def test_exact_tier_probability_vector(small):
    # forward_batch_probs on the reference-order tier: the shared softmax of bit-identical
    # logits, within the probability tolerance of the oracle's softmax
    path, dims = small["base"], SMALL["base"]
    with ffi.PluginBackend(path, profile=1 | EXACT | FMA) as be:
        orc = O.MambaOracle(path, 1 | O.ORC_PROFILE_FMA, cap=6)
        be.batch_init(6)
        for t in range(3):
            toks = [(s * 41 + t * 17 + 2) % dims.vocab for s in range(6)]
            g = np.empty((6, dims.vocab), np.float32)
            be.forward_batch(list(range(6)), toks, g, probs=True)
            ref = np.stack([O.softmax(r) for r in orc.forward(list(range(6)), toks)])
            assert float(np.max(np.abs(g - ref).sum(axis=-1))) <= 1e-4
        orc.close()


def test_exact_tier_long_horizon(small):
    # 8 streams for 600 steps, int8 groups of 64 in contract 2: every logit of every step
    # and the final state bit for bit (no drift however long the recurrence runs)
    check_bitwise(small["base"], SMALL["base"], 1, 2, n=8, steps=600, seed=21)


@pytest.mark.parametrize("contract", [1, 2])
@pytest.mark.parametrize("profile", [0, 1])
def test_exact_tier_mamba130m_equals_oracle(full_model, profile, contract):
    check_bitwise(full_model, rbin.MAMBA_130M, profile, contract, n=3, steps=3, seed=profile + 5 * contract)


def test_exact_tier_v1_and_batch_and_reset(small):
    # v1 through redukt_backend_forward, the batch at another position and slot, and the
    # periodic reset, all against the oracle's single stream bit for bit.
    path, dims = small["base"], SMALL["base"]
    seq = [(13 * i + 5) % dims.vocab for i in range(7)]
    orc = O.MambaOracle(path, 1 | O.ORC_PROFILE_FMA, cap=1)
    orc.set_reset_every(4)
    want = [orc.forward([0], [t])[0] for t in seq]
    orc.close()
    with ffi.PluginBackend(path, profile=1 | EXACT | FMA) as be:
        out = np.empty(dims.vocab, np.float32)
        L = be.lib.lib
        L.redukt_backend_reset_state()
        for i, t in enumerate(seq):
            if i == 4:
                L.redukt_backend_reset_state()
            assert L.redukt_backend_forward(t, out.ctypes.data_as(ffi._f32p), dims.vocab) == ffi.BackendResult.OK
            assert np.array_equal(bits(out), bits(want[i])), ("v1", i)
        be.batch_init(16)
        be.batch_reset(None)
        for i, t in enumerate(seq):
            if i == 4:
                be.batch_reset([11])
            toks = [(t + 1) % dims.vocab, t, 3]
            g = np.empty((3, dims.vocab), np.float32)
            be.forward_batch([2, 11, 7], toks, g)
            assert np.array_equal(bits(g[1]), bits(want[i])), ("batch", i)


@pytest.mark.parametrize("profile,contract,device_cdf", [(0, 1, False), (1, 2, False), (1, 2, True), (6, 1, False)])
def test_archive_coded_on_cpu_decodes_on_gpu(small, oracle_plugin, profile, contract, device_cdf):
    # device_cdf: the GPU side also builds each step's CDF on the device (the same bits as
    # the host's CDF of the same logits)
    path, dims = small["base"], SMALL["base"]
    rng = np.random.default_rng(17 + profile)
    files = [synth.zipf_tokens(rng, dims.vocab, (k,)).astype(np.uint32) for k in (90, 1, 33, 140)]
    prof = profile | (FMA if contract == 2 else 0)
    print(f"cross-device round trip profile {profile} contract {contract}", flush=True)
    with Lockstep(path, plugin_path=oracle_plugin, profile=prof, slots=3) as cpu:
        cpu_bytes, _ = cpu.compress(files, reset_every=64)
    with Lockstep(path, profile=prof | EXACT, slots=3, device_cdf=device_cdf) as gpu:
        gpu_bytes, _ = gpu.compress(files, reset_every=64)
        assert gpu_bytes == cpu_bytes, "the GPU codes other bytes than the CPU"
        back, _ = gpu.decompress(cpu_bytes, [len(f) for f in files], reset_every=64)
    for f, b in zip(files, back):
        assert np.array_equal(f, b)
    with Lockstep(path, plugin_path=oracle_plugin, profile=prof, slots=2) as cpu:
        back, _ = cpu.decompress(gpu_bytes, [len(f) for f in files], reset_every=64)
    for f, b in zip(files, back):
        assert np.array_equal(f, b)


@pytest.mark.parametrize("quant,contract", [(1, 2), (0, 1)])
def test_rdkt_archive_written_on_gpu_decodes_on_cpu(small, oracle_plugin, quant, contract):
    """GPU-coded streams in RDKT v5 archives with the header of the CPU Mamba backbone
    (BACKBONE 1, PROFILE = weight profile code + numeric contract, RESET_LOG2 8): the CPU side
    takes its weight profile, contract and reset period from the header alone, decodes the
    stream and checks the CRC-32 of the restored data (src/application/codec.rs:540-580,
    648-720).  The files cross reset boundaries."""
    path, dims = small["base"], SMALL["base"]
    rng = np.random.default_rng(40 + quant)
    files = [synth.zipf_tokens(rng, dims.vocab, (k,)).astype(np.uint32) for k in (300, 1, 90, 520)]
    with Lockstep(path, profile=quant | EXACT | (FMA if contract == 2 else 0), slots=3, device_cdf=False) as gpu:
        streams, _ = gpu.compress(files, reset_every=256)
    for f, stm in zip(files, streams):
        payload = f.astype("<u4").tobytes()
        h = archive.default_header(len(payload), backbone=archive.BACKBONE_MAMBA, quant=quant, reset_log2=8)
        h.contract = contract
        arc = archive.pack(h, stm, payload)
        hd, body, crc = archive.unpack(arc)
        assert (hd.backbone, hd.quant, hd.contract, hd.reset_every) == (archive.BACKBONE_MAMBA, quant, contract, 256)
        cpu_profile = hd.quant | (O.ORC_PROFILE_FMA if hd.contract == 2 else 0)
        with Lockstep(path, plugin_path=oracle_plugin, profile=cpu_profile, slots=1) as cpu:
            back, _ = cpu.decompress([body], [hd.total_bytes // 4], reset_every=hd.reset_every)
        assert archive.crc32(back[0].astype("<u4").tobytes()) == crc
        assert np.array_equal(back[0], f)


@pytest.mark.parametrize("name,label", [("f32-ref", "hip-gfx950-mamba-f32-ref"), ("q8-ref", "hip-gfx950-mamba-q8-ref"),
                                        ("f32-ref-fma", "hip-gfx950-mamba-f32-ref-fma"),
                                        ("q8-ref-fma", "hip-gfx950-mamba-q8-ref-fma")])
def test_named_profiles_from_the_environment(small, monkeypatch, name, label):
    # the v1 init takes its weight profile from REDUKT_GPU_PROFILE, by name
    monkeypatch.setenv("REDUKT_GPU_PROFILE", name)
    lib = ffi.PluginLibrary()
    try:
        assert lib.init(small["base"]).name_str() == label
    finally:
        lib.free()


def test_exact_tier_refuses_what_it_does_not_serve(small):
    lib = ffi.PluginLibrary()
    info = ffi.BackendInfo()
    for prof in (EXACT | ffi.PROFILE_GEMV, FMA | ffi.PROFILE_GEMV, EXACT | ffi.PROFILE_W8A8 | 2):
        rc = lib.lib.redukt_backend_init_ex(small["base"].encode(), 0, prof, ffi.ctypes.byref(info))
        assert rc == ffi.BackendResult.INIT_FAILED, (prof, rc)
    assert lib.lib.redukt_backend_init_ex(small["base"].encode(), 0, 256, ffi.ctypes.byref(info)) == \
        ffi.BackendResult.INVALID_ARGUMENT
    lib.lib.redukt_backend_free()
