"""The C++ lockstep driver's schedule on the CPU, over a stand-in plugin (fake_plugin.c)
whose logits numpy can recompute: the coded bytes of every file equal a Python
restatement of the single-file sequence (uniform first token, then the CDF of the
previous forward's logits; src/application/lockstep.rs:16-21, 163-330), with the
plugin's tick schedule (src/infrastructure/plugin_backend/model.rs:44-49); lockstep
equals the single-stream v1 path for any slot and thread count (tests/roundtrip.rs:
681-736); decompress restores the tokens either way."""
import os
import subprocess

import numpy as np
import pytest

from oracle import codec as O
from redukt_amd import codec as C
from redukt_amd.lockstep import Lockstep, LockstepError, LockstepStatus, stream_bound

HERE = os.path.dirname(os.path.abspath(__file__))
VOCAB = 300
M64 = (1 << 64) - 1


@pytest.fixture(scope="module")
def fake(tmp_path_factory):
    d = tmp_path_factory.mktemp("fake_plugin")
    so = str(d / "libfake_plugin.so")
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-ffp-contract=off", "-o", so,
                    os.path.join(HERE, "fake_plugin.c")], check=True)
    w = str(d / "weights.bin")
    np.array([VOCAB], np.uint32).tofile(w)
    return so, w


def _mix(z):
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _mix_np(z):
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _logits(s):
    with np.errstate(over="ignore"):
        v = np.arange(VOCAB, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
    h = _mix_np(np.uint64(s) ^ v)
    return ((h >> np.uint64(40)) % np.uint64(4001)).astype(np.float32) / np.float32(400) - np.float32(5)


def python_encode(tokens, reset_every):
    """One file, exactly the reference's single-file sequence over the stand-in model."""
    enc = O.RangeEncoder()
    s, since, lg = 0, 0, None
    for t, tok in enumerate(tokens):
        enc.encode_symbol(int(tok), O.cdf_uniform(VOCAB) if t == 0 else O.cdf_from_logits(lg))
        if t == len(tokens) - 1:
            break
        if reset_every and since >= reset_every:
            s, since = 0, 0
        since += 1
        s = _mix((s * 0x100000001B3 + int(tok) + 1) & M64)
        lg = _logits(s)
    return enc.finish()


def files(seed=0, lengths=(57, 1, 300, 129, 8, 40)):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, VOCAB, n).astype(np.uint32) for n in lengths]


def test_stream_bound_covers_worst_case():
    # every token at frequency 1 of 2^24: 24 bits each plus truncation, plus the flush
    assert stream_bound(0) == 5 and stream_bound(8) >= 8 * 25 // 8 + 5


def test_lockstep_matches_python_restatement(fake):
    so, w = fake
    fs = files()
    with Lockstep(w, plugin_path=so, slots=3) as ls:
        assert ls.vocab == VOCAB and ls.name == "fake-plugin"
        out, st = ls.compress(fs, reset_every=16)
    for f, b in zip(fs, out):
        assert b == python_encode(f, 16)
    assert st.tokens == sum(len(f) for f in fs) and st.files == len(fs)


@pytest.mark.parametrize("slots,threads", [(0, 0), (1, 1), (2, 0), (4, 3), (7, 0)])
def test_batch_equals_single_and_roundtrip(fake, slots, threads):
    so, w = fake
    fs = files(1)
    with Lockstep(w, plugin_path=so, slots=0) as single:
        ref, _ = single.compress(fs, reset_every=32)
    with Lockstep(w, plugin_path=so, slots=slots, threads=threads) as ls:
        out, _ = ls.compress(fs, reset_every=32)
        assert out == ref
        back, _ = ls.decompress(out, [len(f) for f in fs], reset_every=32)
    for f, b in zip(fs, back):
        assert np.array_equal(f, b)


def test_batched_streams_decode_single_file(fake):
    so, w = fake
    fs = files(2)
    with Lockstep(w, plugin_path=so, slots=4) as ls:
        out, _ = ls.compress(fs, reset_every=0)
    with Lockstep(w, plugin_path=so, slots=0) as single:
        back, _ = single.decompress([out[2]], [len(fs[2])], reset_every=0)
    assert np.array_equal(back[0], fs[2])


def test_reset_period_changes_the_stream(fake):
    so, w = fake
    f = files(3, (200,))
    with Lockstep(w, plugin_path=so, slots=2) as ls:
        a, _ = ls.compress(f, reset_every=0)
        b, _ = ls.compress(f, reset_every=50)
        # decoding with the wrong period does not restore the tokens
        wrong, _ = ls.decompress(b, [200], reset_every=0)
    assert a != b and b[0] == python_encode(f[0], 50) and a[0] == python_encode(f[0], 0)
    assert not np.array_equal(wrong[0], f[0])


def test_per_file_errors(fake):
    so, w = fake
    fs = files(4, (10, 10, 10))
    bad = fs[1].copy()
    bad[4] = VOCAB  # out of the vocabulary
    with Lockstep(w, plugin_path=so, slots=2) as ls:
        with pytest.raises(LockstepError) as e:
            ls.compress([fs[0], bad, np.zeros(0, np.uint32), fs[2]], reset_every=0)
        assert e.value.status == LockstepStatus.CODER
        assert e.value.file_status == [C.CodecStatus.OK, C.CodecStatus.INVALID_ARG, C.CodecStatus.INVALID_ARG,
                                       C.CodecStatus.OK]
        # the healthy files of that batch still coded as if alone
        out, _ = ls.compress([fs[0], fs[2]], reset_every=0)
        assert out[0] == python_encode(fs[0], 0) and out[1] == python_encode(fs[2], 0)


def test_v1_only_plugin_serves_one_stream(fake, monkeypatch):
    so, w = fake
    monkeypatch.setenv("FAKE_PLUGIN_ABI", "1")
    with pytest.raises(LockstepError) as e:
        Lockstep(w, plugin_path=so, slots=4)
    assert e.value.status == LockstepStatus.NEEDS_V2
    f = files(5, (30,))
    with Lockstep(w, plugin_path=so, slots=1) as ls:  # falls back to the v1 global state
        out, _ = ls.compress(f, reset_every=7)
    assert out[0] == python_encode(f[0], 7)


def test_open_errors(fake, tmp_path):
    so, w = fake
    with pytest.raises(LockstepError) as e:
        Lockstep(w, plugin_path=str(tmp_path / "missing.so"), slots=1)
    assert e.value.status == LockstepStatus.PLUGIN_LOAD
    with pytest.raises(LockstepError) as e:
        Lockstep(str(tmp_path / "missing.bin"), plugin_path=so, slots=1)
    assert e.value.status == LockstepStatus.PLUGIN_INIT


@pytest.mark.parametrize("slots", [0, 2])
def test_backbone_failure_marks_unfinished_files(fake, monkeypatch, slots):
    # forward fails mid-run: files finished before it keep OK and their bytes; every file in
    # flight or never admitted reports INCOMPLETE, never OK.
    so, w = fake
    fs = files(6, (3, 40, 40, 40, 40))
    monkeypatch.setenv("FAKE_PLUGIN_FAIL_AFTER", "12")
    with Lockstep(w, plugin_path=so, slots=slots) as ls:
        with pytest.raises(LockstepError) as e:
            ls.compress(fs, reset_every=0)
    assert e.value.status == LockstepStatus.FORWARD
    st = e.value.file_status
    assert st[0] == C.CodecStatus.OK
    assert all(s == C.CodecStatus.INCOMPLETE for s in st[1:]), st


def test_decompress_rejects_mismatched_lengths(fake):
    so, w = fake
    with Lockstep(w, plugin_path=so, slots=2) as ls:
        with pytest.raises(ValueError):
            ls.decompress([b"\x00" * 8, b"\x00" * 8], [4])


def test_device_cdf_needs_the_plugin_symbol(fake):
    # the stand-in plugin exports no forward_batch_cdf: the driver keeps the host CDF and
    # refuses to switch
    so, w = fake
    with Lockstep(w, plugin_path=so, slots=3) as ls:
        assert not ls.device_cdf
        out, _ = ls.compress(files(), reset_every=16)
    with pytest.raises(LockstepError):
        Lockstep(w, plugin_path=so, slots=3, device_cdf=True)
    with Lockstep(w, plugin_path=so, slots=3, device_cdf=False) as ls:
        assert ls.compress(files(), reset_every=16)[0] == out


@pytest.mark.parametrize("kind", ["mamba", "rwkv7"])
def test_oracle_plugin_round_trip_on_the_cpu(oracle_plugin, tmp_path, kind):
    """The CPU oracle behind the plugin ABI (tests/oracle_plugin.c) drives the lockstep
    coder end to end on the host: batched compress, then decompress, byte-exact, for both
    model kinds the plugin tells apart by the file header; batched and single-stream
    coding give the same bytes."""
    from redukt_amd import rbin, rwkv, synth

    path = str(tmp_path / f"{kind}.rbin")
    if kind == "mamba":
        synth.write_synthetic_mamba(path, rbin.MambaDims(vocab=300, d_model=64, n_layer=2), seed=4)
        vocab = 300
    else:
        dims = rwkv.RwkvDims(vocab=260, d_model=64, n_layer=2, head_size=64, d_ffn=128, lora_w=8, lora_a=8,
                             lora_v=8, lora_g=16)
        rwkv.write_synthetic(path, dims, seed=4)
        vocab = 260
    rng = np.random.default_rng(6)
    files = [rng.integers(0, vocab, k).astype(np.uint32) for k in (70, 1, 40)]
    with Lockstep(path, plugin_path=oracle_plugin, slots=2) as ls:
        streams, _ = ls.compress(files, reset_every=32)
        back, _ = ls.decompress(streams, [len(f) for f in files], reset_every=32)
    for f, b in zip(files, back):
        assert np.array_equal(f, b)
    with Lockstep(path, plugin_path=oracle_plugin, slots=0) as single:
        one, _ = single.compress(files, reset_every=32)
    assert one == streams


# The device-CDF paths over the stand-in plugin built with its CDF entry points
# (-DFAKE_PLUGIN_CDF: every CDF is the host library's): host CDFs, whole device rows,
# the coder's values per stream (compression) with the decoder's search (decompression),
# and compression queued a step ahead (REDUKT_LOCKSTEP_PIPELINE) all code the bytes of the
# Python restatement, with the same per-file errors and the same statuses when the
# backbone fails.
PATHS = {"host": (False, "1", "1"), "rows": (True, "0", "1"), "sym-find": (True, "1", "0"),
         "pipelined": (True, "1", "1")}


@pytest.fixture(scope="module")
def fake_cdf(tmp_path_factory):
    d = tmp_path_factory.mktemp("fake_plugin_cdf")
    so = str(d / "libfake_plugin_cdf.so")
    host = os.path.dirname(os.path.abspath(C.DEFAULT_LIB))
    subprocess.run(["gcc", "-O2", "-shared", "-fPIC", "-ffp-contract=off", "-DFAKE_PLUGIN_CDF", "-o", so,
                    os.path.join(HERE, "fake_plugin.c"), "-L", host, "-lredukt_host", f"-Wl,-rpath,{host}"],
                   check=True)
    w = str(d / "weights.bin")
    np.array([VOCAB], np.uint32).tofile(w)
    return so, w


def _path(monkeypatch, name):
    dev, sym, pipe = PATHS[name]
    monkeypatch.setenv("REDUKT_LOCKSTEP_CDF_SYM", sym)
    monkeypatch.setenv("REDUKT_LOCKSTEP_PIPELINE", pipe)
    return dev


@pytest.mark.parametrize("slots", [1, 2, 3, 7])
@pytest.mark.parametrize("name", list(PATHS))
def test_device_cdf_paths_equal_the_restatement(fake_cdf, monkeypatch, slots, name):
    so, w = fake_cdf
    fs = files(7)
    dev = _path(monkeypatch, name)
    with Lockstep(w, plugin_path=so, slots=slots, device_cdf=dev) as ls:
        assert ls.device_cdf == dev
        out, st = ls.compress(fs, reset_every=16)
        assert out == [python_encode(f, 16) for f in fs]
        assert st.tokens == sum(len(f) for f in fs) and st.files == len(fs)
        back, _ = ls.decompress(out, [len(f) for f in fs], reset_every=16)
    for f, b in zip(fs, back):
        assert np.array_equal(f, b)


@pytest.mark.parametrize("name", list(PATHS))
def test_device_cdf_paths_per_file_errors(fake_cdf, monkeypatch, name):
    so, w = fake_cdf
    fs = files(4, (10, 10, 10))
    bad = fs[1].copy()
    bad[4] = VOCAB
    dev = _path(monkeypatch, name)
    with Lockstep(w, plugin_path=so, slots=2, device_cdf=dev) as ls:
        with pytest.raises(LockstepError) as e:
            ls.compress([fs[0], bad, np.zeros(0, np.uint32), fs[2]], reset_every=3)
        assert e.value.status == LockstepStatus.CODER
        assert e.value.file_status == [C.CodecStatus.OK, C.CodecStatus.INVALID_ARG, C.CodecStatus.INVALID_ARG,
                                       C.CodecStatus.OK]
        out, _ = ls.compress([fs[0], fs[2]], reset_every=3)
        assert out[0] == python_encode(fs[0], 3) and out[1] == python_encode(fs[2], 3)


@pytest.mark.parametrize("name", list(PATHS))
def test_device_cdf_paths_backbone_failure(fake_cdf, monkeypatch, name):
    # the 13th forward fails in the iteration in which file 0 codes its last token: file 0
    # still finishes (its coding comes before that forward), the others are INCOMPLETE
    so, w = fake_cdf
    fs = files(6, (13, 40, 40))
    dev = _path(monkeypatch, name)
    monkeypatch.setenv("FAKE_PLUGIN_FAIL_AFTER", "12")
    with Lockstep(w, plugin_path=so, slots=2, device_cdf=dev) as ls:
        with pytest.raises(LockstepError) as e:
            ls.compress(fs, reset_every=0)
    assert e.value.status == LockstepStatus.FORWARD
    assert e.value.file_status == [C.CodecStatus.OK, C.CodecStatus.INCOMPLETE, C.CodecStatus.INCOMPLETE]
