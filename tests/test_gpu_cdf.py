"""The device CDF (logits -> u32 cumulative frequencies on the GPU) against the host coding
path, through the C ABI.

The range coder's frequencies depend on the last bit of every f64 operation of the CDF,
so the bar is bit-exact equality with `redukt_cdf_from_logits` (libredukt_host.so), which
the CPU tests pin to the oracle and the reference's exp goldens:

* crafted rows through `redukt_backend_cdf_from_logits_device`: Gaussian logits at
  several scales, vocabularies 1, 2, 255-257 (around the terms the sums add one by one),
  8,192 and 8,193 (one round's window), 50,280, 50,281 (odd: the unpaired load path) and
  65,536, many-way ties for the maximum, a flat row (every share rounds up and the
  fix-up wraps the last frequency, a reference quirk), -inf entries, rows whose exps
  underflow into subnormals, a row with NaNs;
* `redukt_backend_forward_batch_cdf` on Mamba-130M (int8 per-row) and RWKV-7 0.1B
  against the host CDF of the same step's logits from `forward_batch` (batch invariance
  makes a stream's logits the same on any slot);
* `redukt_backend_forward_batch_cdf_sym` and `_find` (what the coder reads of each row for
  a known symbol or a decoder target) against the full rows and the host search;
* the driver's lockstep bytes with the device CDF equal those with the host CDF, and
  damaged archives decode to the same tokens on every path.
"""
import numpy as np
import pytest

from redukt_amd import codec, ffi, hip, lockstep, rwkv, synth

pytestmark = pytest.mark.gpu

Q8ROW_ALL = ffi.PROFILE_Q8_ROW | ffi.PROFILE_Q8_SMALL


def crafted_rows():
    rng = np.random.default_rng(2024)
    rows = []
    for n, scale in ((50280, 1.0), (50280, 8.0), (50280, 0.05), (65536, 3.0), (256, 2.0), (50281, 1.5),
                     (2, 1.0), (1, 1.0), (255, 1.0), (257, 1.0), (8192, 2.0), (8193, 0.5)):
        rows.append(("gauss", (rng.standard_normal(n) * scale).astype(np.float32)))
    t = (rng.standard_normal(50280)).astype(np.float32)
    t[rng.choice(50280, 37, replace=False)] = t.max() + 1.0       # 37 equal maxima
    rows.append(("ties", t))
    rows.append(("flat", np.zeros(50280, np.float32)))             # every share rounds up
    t = (rng.standard_normal(50280) * 2).astype(np.float32)
    t[::7] = -np.inf
    rows.append(("neg-inf", t))
    t = (rng.standard_normal(50280) * 300).astype(np.float32)       # exps down to subnormal and 0
    rows.append(("subnormal", t))
    t = (rng.standard_normal(4096)).astype(np.float32)
    t[[5, 100, 4000]] = np.nan
    rows.append(("nan", t))
    return rows


@pytest.fixture(scope="module")
def backend(full_model):
    with ffi.PluginBackend(full_model, profile=Q8ROW_ALL) as be:
        yield be


ROWS = crafted_rows()


@pytest.mark.parametrize("case", range(len(ROWS)), ids=[f"{i}-{r[0]}-{r[1].size}" for i, r in enumerate(ROWS)])
def test_device_cdf_equals_host_cdf_on_crafted_rows(backend, case):
    name, row = ROWS[case]
    n = row.size
    host = codec.cdf_from_logits(row)
    reps = np.stack([row, row[::-1].copy()]) if n > 1 else row[None]
    d_l = hip.DeviceBuffer.from_array(np.ascontiguousarray(reps, np.float32))
    d_c = hip.DeviceBuffer(reps.shape[0] * (n + 1) * 4)
    try:
        assert backend.cdf_from_logits_device(d_l.ptr, reps.shape[0], n, d_c.ptr) == ffi.BackendResult.OK
        hip.stream_sync(backend.stream())
        got = d_c.download(np.uint32, reps.shape[0] * (n + 1)).reshape(reps.shape[0], n + 1)
    finally:
        d_l.close()
        d_c.close()
    assert np.array_equal(got[0], host), (name, int(np.flatnonzero(got[0] != host)[0]))
    if reps.shape[0] > 1:
        assert np.array_equal(got[1], codec.cdf_from_logits(reps[1])), name
    assert got[0, 0] == 0 and got[0, -1] == (1 << 24)


def test_device_cdf_rejects_bad_sizes(backend):
    assert backend.cdf_from_logits_device(0, 1, 0, 0) == ffi.BackendResult.INVALID_ARGUMENT
    assert backend.cdf_from_logits_device(0, 1, 1 << 24, 0) == ffi.BackendResult.INVALID_ARGUMENT
    assert backend.cdf_from_logits_device(0, 0, 10, 0) == ffi.BackendResult.OK


def step_pair(be, n, steps, seed):
    """forward_batch_cdf on slots [0, n) and forward_batch on slots [n, 2n) with the same
    tokens: the device CDFs and the host CDFs of the logits, step by step."""
    rng = np.random.default_rng(seed)
    V = be.vocab
    for t in range(steps):
        toks = [int(x) for x in rng.integers(0, min(V, 50280), n)]
        cdf = np.empty((n, V + 1), np.uint32)
        be.forward_batch_cdf(list(range(n)), toks, cdf)
        logits = np.empty((n, V), np.float32)
        be.forward_batch(list(range(n, 2 * n)), toks, logits)
        host = codec.cdf_from_logits_batch(logits)
        bad = [r for r in range(n) if not np.array_equal(cdf[r], host[r])]
        assert not bad, (t, bad[:5])


def test_forward_batch_cdf_mamba130m(backend):
    backend.batch_init(64)
    step_pair(backend, 32, 3, seed=9)


def test_forward_batch_cdf_rejects_bad_arguments(backend):
    backend.batch_init(8)
    out = np.empty((2, backend.vocab + 1), np.uint32)
    with pytest.raises(ffi.BackendError):
        backend.forward_batch_cdf([0, 0], [1, 2], out)          # repeated slot
    code = backend.lib.lib.redukt_backend_forward_batch_cdf(
        1, ffi._ptr(np.zeros(1, np.uint32), ffi.ctypes.c_uint32), ffi._ptr(np.zeros(1, np.uint32), ffi.ctypes.c_uint32),
        ffi._ptr(out, ffi.ctypes.c_uint32), backend.vocab)      # cdf_len one short
    assert code == ffi.BackendResult.INVALID_ARGUMENT


def test_forward_batch_cdf_sym_equals_the_rows(backend):
    # The coder's three values per stream for a known next symbol equal the full device CDF
    # row's entries (the same tokens on other slots), symbols 0 and V - 1 included.
    backend.batch_init(64)
    V = backend.vocab
    rng = np.random.default_rng(12)
    n = 29
    for t in range(3):
        toks = [int(x) for x in rng.integers(0, V, n)]
        syms = [int(x) for x in rng.integers(0, V, n)]
        syms[0], syms[-1] = 0, V - 1
        rows = np.empty((n, V + 1), np.uint32)
        backend.forward_batch_cdf(list(range(n)), toks, rows)
        got = np.empty(3 * n, np.uint32)
        assert backend.forward_batch_cdf_sym(list(range(n, 2 * n)), toks, syms, got) == ffi.BackendResult.OK
        want = np.stack([[rows[b, syms[b]], rows[b, syms[b] + 1], rows[b, V]] for b in range(n)]).reshape(-1)
        assert np.array_equal(got, want), t


def test_forward_batch_cdf_sym_rejects_bad_arguments(backend):
    backend.batch_init(8)
    V = backend.vocab
    got = np.empty(6, np.uint32)
    assert backend.forward_batch_cdf_sym([0, 1], [1, 2], [3, V], got) == ffi.BackendResult.INVALID_ARGUMENT
    assert backend.forward_batch_cdf_sym([0, 0], [1, 2], [3, 4], got) == ffi.BackendResult.INVALID_ARGUMENT
    code = backend.lib.lib.redukt_backend_forward_batch_cdf_sym(
        2, ffi._ptr(np.array([0, 1], np.uint32), ffi.ctypes.c_uint32),
        ffi._ptr(np.array([1, 2], np.uint32), ffi.ctypes.c_uint32),
        ffi._ptr(np.array([3, 4], np.uint32), ffi.ctypes.c_uint32), ffi._ptr(got, ffi.ctypes.c_uint32), V + 1)
    assert code == ffi.BackendResult.INVALID_ARGUMENT   # vocab_size not the model's


def test_forward_batch_cdf_sym_queued_equals_the_direct_call(backend):
    # Queued calls (two in flight) give the direct call's values for the same tokens on
    # other slots over three steps; a third call in flight, an unknown ticket and a count
    # other than the submitted one are refused without disturbing the calls in flight.
    backend.batch_init(64)
    V = backend.vocab
    rng = np.random.default_rng(14)
    n = 23
    toks = [[int(x) for x in rng.integers(0, V, n)] for _ in range(3)]
    syms = [[int(x) for x in rng.integers(0, V, n)] for _ in range(3)]
    want = []
    for t in range(3):
        w = np.empty(3 * n, np.uint32)
        assert backend.forward_batch_cdf_sym(list(range(n)), toks[t], syms[t], w) == ffi.BackendResult.OK
        want.append(w)
    q = list(range(n, 2 * n))
    rc0, t0 = backend.forward_batch_cdf_sym_submit(q, toks[0], syms[0])
    rc1, t1 = backend.forward_batch_cdf_sym_submit(q, toks[1], syms[1])
    assert rc0 == rc1 == ffi.BackendResult.OK and t0 != t1 and t0 > 0
    assert backend.forward_batch_cdf_sym_submit(q, toks[2], syms[2])[0] == ffi.BackendResult.INVALID_ARGUMENT
    got = np.empty(3 * n, np.uint32)
    assert backend.forward_batch_cdf_sym_wait(t0, np.empty(3 * (n - 1), np.uint32)) == ffi.BackendResult.INVALID_ARGUMENT
    assert backend.forward_batch_cdf_sym_wait(t0 + t1 + 7, got) == ffi.BackendResult.INVALID_ARGUMENT
    assert backend.forward_batch_cdf_sym_wait(t0, got) == ffi.BackendResult.OK
    assert np.array_equal(got, want[0])
    rc2, t2 = backend.forward_batch_cdf_sym_submit(q, toks[2], syms[2])
    assert rc2 == ffi.BackendResult.OK
    assert backend.forward_batch_cdf_sym_wait(t1, got) == ffi.BackendResult.OK
    assert np.array_equal(got, want[1])
    assert backend.forward_batch_cdf_sym_wait(t2, got) == ffi.BackendResult.OK
    assert np.array_equal(got, want[2])
    assert backend.forward_batch_cdf_sym_wait(t0, got) == ffi.BackendResult.INVALID_ARGUMENT   # already collected
    bad = list(q)
    bad[3] = bad[2]
    assert backend.forward_batch_cdf_sym_submit(bad, toks[0], syms[0])[0] == ffi.BackendResult.INVALID_ARGUMENT
    # a call in flight across batch_init is dropped: its ticket is refused, and a new
    # pool's tickets are new numbers
    rc3, t3 = backend.forward_batch_cdf_sym_submit(q, toks[0], syms[0])
    assert rc3 == ffi.BackendResult.OK
    backend.batch_init(64)
    assert backend.forward_batch_cdf_sym_wait(t3, got) == ffi.BackendResult.INVALID_ARGUMENT
    rc4, t4 = backend.forward_batch_cdf_sym_submit(q, toks[0], syms[0])
    assert rc4 == ffi.BackendResult.OK and t4 > t3
    assert backend.forward_batch_cdf_sym_wait(t4, got) == ffi.BackendResult.OK


def test_forward_batch_cdf_find_equals_the_host_search(backend):
    # The symbol the device finds for a decoder target, with its two bounds and the total,
    # equals the host search (redukt_cdf_lookup) over the full device CDF row of the same
    # tokens on other slots: targets 0 and total - 1, each bound of random symbols, random
    # values, and targets at and beyond the total (s = V, both bounds the total).
    backend.batch_init(64)
    V = backend.vocab
    T = 1 << 24
    rng = np.random.default_rng(13)
    n = 31
    for t in range(3):
        toks = [int(x) for x in rng.integers(0, V, n)]
        rows = np.empty((n, V + 1), np.uint32)
        backend.forward_batch_cdf(list(range(n)), toks, rows)
        assert np.all(rows[:, V] == T)
        syms = rng.integers(0, V, n)
        targets = rng.integers(0, T, n).astype(np.uint32)
        targets[:4] = [0, T - 1, T, 2**32 - 1]
        for b in range(4, 12):
            targets[b] = rows[b, syms[b]]            # a symbol's first value
        for b in range(12, 20):
            targets[b] = rows[b, syms[b] + 1] - 1    # a symbol's last value
        got = np.empty(4 * n, np.uint32)
        assert backend.forward_batch_cdf_find(list(range(n, 2 * n)), toks, targets, got) == ffi.BackendResult.OK
        want = []
        for b in range(n):
            s = codec.lookup(rows[b], int(targets[b]))
            want += [s, rows[b, s], rows[b, s + 1], T] if s < V else [V, T, T, T]
        assert np.array_equal(got, np.array(want, np.uint32)), t
        assert got[0] == 0 and got[4 * 2] == V and got[4 * 3] == V


def test_forward_batch_cdf_find_rejects_bad_arguments(backend):
    backend.batch_init(8)
    V = backend.vocab
    got = np.empty(8, np.uint32)
    assert backend.forward_batch_cdf_find([0, 1], [1, V], [3, 4], got) == ffi.BackendResult.INVALID_ARGUMENT
    assert backend.forward_batch_cdf_find([0, 0], [1, 2], [3, 4], got) == ffi.BackendResult.INVALID_ARGUMENT
    code = backend.lib.lib.redukt_backend_forward_batch_cdf_find(
        2, ffi._ptr(np.array([0, 1], np.uint32), ffi.ctypes.c_uint32),
        ffi._ptr(np.array([1, 2], np.uint32), ffi.ctypes.c_uint32),
        ffi._ptr(np.array([3, 4], np.uint32), ffi.ctypes.c_uint32), ffi._ptr(got, ffi.ctypes.c_uint32), V - 1)
    assert code == ffi.BackendResult.INVALID_ARGUMENT   # vocab_size not the model's


# The tests below open backends of their own: the library holds one model at a time, so
# they come after every test of the shared `backend` fixture.
def test_forward_batch_cdf_rwkv7(tmp_path):
    p = str(tmp_path / "rwkv.rbin")
    rwkv.write_synthetic(p, rwkv.RWKV7_0_1B, seed=1)
    with ffi.PluginBackend(p, profile=2) as be:
        be.batch_init(16)
        step_pair(be, 8, 2, seed=3)


def test_lockstep_device_cdf_bytes_equal_host_cdf(full_model, monkeypatch):
    # Host CDFs, device CDF rows, and the device paths that hand back only what the coder
    # reads (three values for compression's known symbol, the symbol found and its bounds
    # for decompression's target), with compression waiting for each step or queueing the
    # next one first (the default): the same archives, each decoding to its file.  Damaged archives (bytes flipped, a stream cut short, one empty, more tokens
    # asked for than were coded) drive the decoders through arbitrary states: all three
    # decode them to the same tokens.
    rng = np.random.default_rng(77)
    files = [[int(x) for x in synth.zipf_tokens(rng, 50280, (L,))] for L in (40, 17, 64, 1, 33)]
    outs, bad = {}, {}
    for dev, sym, pipe in ((False, "1", "1"), (True, "0", "1"), (True, "1", "0"), (True, "1", "1")):
        monkeypatch.setenv("REDUKT_LOCKSTEP_CDF_SYM", sym)
        monkeypatch.setenv("REDUKT_LOCKSTEP_PIPELINE", pipe)
        with lockstep.Lockstep(full_model, ffi.DEFAULT_LIB, profile=Q8ROW_ALL, slots=3, device_cdf=dev) as ls:
            assert ls.device_cdf == dev
            streams, _ = ls.compress(files)
            back, _ = ls.decompress(streams, [len(f) for f in files])
            assert [b.tolist() for b in back] == files
            outs[(dev, sym, pipe)] = streams
            damaged = [bytes(x ^ 0x5A if i % 3 == 1 else x for i, x in enumerate(streams[0])), streams[2][:5], b"",
                       streams[3], streams[4]]
            got, _ = ls.decompress(damaged, [40, 64, 20, 30, 33])
            bad[(dev, sym, pipe)] = [g.tolist() for g in got]
    ref = outs[(False, "1", "1")]
    assert all(o == ref for o in outs.values())
    assert all(b == bad[(False, "1", "1")] for b in bad.values())
    assert bad[(False, "1", "1")][0] != files[0] and bad[(False, "1", "1")][4] == files[4]
