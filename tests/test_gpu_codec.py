"""compress -> decompress with the GPU on both ends (libredukt_gpu.so under the C++
lockstep driver of libredukt_host.so).

* The restored tokens equal the input, byte for byte (src/application/codec.rs:3255-3290
  shape: uniform first token, then the CDF of the backbone's logits).
* Lockstep coding equals the single-stream v1 path for every file, at any slot count,
  and a batched stream decodes single-file (tests/roundtrip.rs:681-736).
* The CDFs coded from the GPU's logits are the oracle's CDFs of those same logits, bit
  for bit (src/application/codec.rs:785-798).
"""
import numpy as np
import pytest

from oracle import codec as OC
from redukt_amd import archive, codec, ffi, hip, rbin, rwkv, synth
from redukt_amd.lockstep import Lockstep, LockstepError

pytestmark = pytest.mark.gpu

Q8ROW_ALL = ffi.PROFILE_Q8_ROW | ffi.PROFILE_Q8_SMALL  # int8 per-row everywhere (the benchmark profile)

SMALL = rbin.MambaDims(vocab=1000, d_model=96, n_layer=3)
SMALL_RWKV = rwkv.RwkvDims(vocab=300, d_model=128, n_layer=2, head_size=64, d_ffn=256, lora_w=16, lora_a=16,
                           lora_v=8, lora_g=32)


@pytest.fixture(scope="module")
def small_models(tmp_path_factory):
    assert hip.device_count() > 0, "no GPU visible"
    d = tmp_path_factory.mktemp("codec_models")
    out = {"mamba": str(d / "mamba.rbin"), "rwkv": str(d / "rwkv.rbin")}
    synth.write_synthetic_mamba(out["mamba"], SMALL, seed=7)
    rwkv.write_synthetic(out["rwkv"], SMALL_RWKV, seed=1)
    return out


def token_files(vocab, lengths, seed):
    rng = np.random.default_rng(seed)
    return [synth.zipf_tokens(rng, vocab, (n,)).astype(np.uint32) for n in lengths]


def roundtrip_case(path, profile, files, reset_every, slot_counts):
    print(f"codec round trip {path} profile {profile} files {[len(f) for f in files]}", flush=True)
    with Lockstep(path, profile=profile, slots=0) as single:
        ref, _ = single.compress(files, reset_every=reset_every)
        one, _ = single.decompress([ref[-1]], [len(files[-1])], reset_every=reset_every)
        assert np.array_equal(one[0], files[-1])
    for slots in slot_counts:
        with Lockstep(path, profile=profile, slots=slots) as ls:
            out, st = ls.compress(files, reset_every=reset_every)
            assert out == ref, f"slots={slots}: lockstep bytes != single-stream bytes"
            back, _ = ls.decompress(out, [len(f) for f in files], reset_every=reset_every)
            for f, b in zip(files, back):
                assert np.array_equal(f, b), f"slots={slots}: restored tokens differ"
    return ref


@pytest.mark.parametrize("profile", [0, 2])
def test_mamba_roundtrip_lockstep_equals_single(small_models, profile):
    files = token_files(SMALL.vocab, (57, 1, 200, 129, 8), 3)
    ref = roundtrip_case(small_models["mamba"], profile, files, 64, (1, 3, 5))
    assert all(len(r) > 0 for r in ref)


def test_rwkv_roundtrip_lockstep_equals_single(small_models):
    files = token_files(SMALL_RWKV.vocab, (40, 1, 90, 17), 4)
    roundtrip_case(small_models["rwkv"], 0, files, 0, (2, 4))


def test_cdf_of_gpu_logits_is_oracle_cdf(small_models):
    """The host CDF builder consumes the GPU's logits exactly as the oracle would."""
    with ffi.PluginBackend(small_models["mamba"], profile=0) as be:
        be.batch_init(6)
        for t in range(3):
            toks = [(s * 131 + t * 7 + 5) % be.vocab for s in range(6)]
            g = np.empty((6, be.vocab), np.float32)
            be.forward_batch(list(range(6)), toks, g)
            lib = codec.cdf_from_logits_batch(g)
            for r in range(6):
                assert np.array_equal(lib[r], OC.cdf_from_logits(g[r])), (t, r)


def test_mamba130m_lockstep_roundtrip(full_model):
    """Mamba-130M (vocab 50280), int8 per-row, 32 files of 48-80 tokens in 8 slots with
    continuous batching; the period 16 makes every file cross several resets."""
    files = token_files(50280, [48 + (i * 7) % 33 for i in range(32)], 9)
    with Lockstep(full_model, profile=Q8ROW_ALL, slots=8) as ls:
        out, st = ls.compress(files, reset_every=16)
        back, sd = ls.decompress(out, [len(f) for f in files], reset_every=16)
    for f, b in zip(files, back):
        assert np.array_equal(f, b)
    n_tok = sum(len(f) for f in files)
    bits_per_tok = 8.0 * sum(len(o) for o in out) / n_tok
    print(f"Mamba-130M q8row lockstep 8 slots: {n_tok} tokens, {bits_per_tok:.2f} bits/token, "
          f"compress {st.tok_per_s:.0f} tok/s (code {st.code_secs:.3f}s fwd {st.forward_secs:.3f}s), "
          f"decompress {sd.tok_per_s:.0f} tok/s")
    # first 4 files again alone through the v1 path: identical streams
    with Lockstep(full_model, profile=Q8ROW_ALL, slots=0) as single:
        ref, _ = single.compress(files[:4], reset_every=16)
    assert ref == out[:4]


@pytest.mark.parametrize("reset_log2,lengths", [(12, (70, 33, 1, 90)), (8, (600, 260, 300, 513, 257))])
def test_mamba130m_rdkt_v5_archives(full_model, reset_log2, lengths):
    """GPU lockstep streams in RDKT v5 archives (src/application/codec.rs:540-580, 648-741):
    HEADER (BACKBONE 3 = plugin, PROFILE 0x50, RESET_LOG2) | STREAM | CRC-32 of the
    original data.  The plugin's int8 weights are its configuration (REDUKT_GPU_PROFILE),
    not part of the archive: the reference writes QUANT = F32 for every plugin archive and
    refuses any other (FORMAT-SPEC.md:224-240).  Each archive is parsed and split, its CRC
    checked against the decoded data, and the stream decoded back by the same plugin
    configuration (the period read from the header) to the original tokens byte for byte.
    At RESET_LOG2 8 the files cross resets."""
    files = token_files(50280, lengths, 10 + reset_log2)
    reset_every = 1 << reset_log2
    with Lockstep(full_model, profile=Q8ROW_ALL, slots=4) as ls:
        streams, _ = ls.compress(files, reset_every=reset_every)
    arcs = []
    for f, stm in zip(files, streams):
        payload = f.astype("<u4").tobytes()
        h = archive.default_header(len(payload), backbone=archive.BACKBONE_PLUGIN, quant=0, reset_log2=reset_log2)
        arc = archive.pack(h, stm, payload)
        assert arc[:4] == b"RDKT" and arc[4] == 5 and arc[12:16] == bytes([0x40, 0x50, reset_log2, 3])
        arcs.append(arc)
    # decode side: header -> period and length, stream -> tokens, CRC of the restored data
    heads, body = [], []
    for arc in arcs:
        h, stm, crc = archive.unpack(arc)
        assert h.version == 5 and h.backbone == archive.BACKBONE_PLUGIN and h.quant == 0
        assert h.reset_log2 == reset_log2 and h.has_crc and crc is not None
        heads.append((h, crc))
        body.append(stm)
    assert body == streams
    with Lockstep(full_model, profile=Q8ROW_ALL, slots=3) as ls:
        back, _ = ls.decompress(body, [h.total_bytes // 4 for h, _ in heads], reset_every=heads[0][0].reset_every)
    for f, b, (h, crc) in zip(files, back, heads):
        data = b.astype("<u4").tobytes()
        assert len(data) == h.total_bytes and archive.crc32(data) == crc
        assert np.array_equal(f, b)
    # A flipped bit early in a stream is caught: the decoder fails, or the restored data
    # no longer match the archive's CRC.
    bad = bytearray(arcs[0])
    bad[heads[0][0].header_size + 1] ^= 0x10
    h, stm, crc = archive.unpack(bytes(bad))
    with Lockstep(full_model, profile=Q8ROW_ALL, slots=1) as ls:
        try:
            out, _ = ls.decompress([stm], [h.total_bytes // 4], reset_every=h.reset_every)
            assert archive.crc32(out[0].astype("<u4").tobytes()) != crc
        except LockstepError as e:
            print(f"corrupted stream rejected by the decoder: {e}")
