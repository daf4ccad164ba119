"""The allocation-free device step (redukt_backend_forward_batch_device_noalloc) against
the existing device step (redukt_backend_forward_batch_device), through the C ABI: the
same slots and tokens from the same state give bit-identical logits (and probabilities)
and leave bit-identical recurrent state, on two calls in a row, the second with fewer
streams; a batch that does not fit the library's scratch is refused and changes nothing."""
import numpy as np
import pytest

from redukt_amd import ffi, hip, rbin, synth

pytestmark = pytest.mark.gpu

Q8ROW_ALL = ffi.PROFILE_Q8_ROW | ffi.PROFILE_Q8_SMALL


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _call(be, noalloc, slots, toks, probs=False):
    v = be.vocab
    d_s = hip.DeviceBuffer.from_array(np.array(slots, np.uint32))
    d_t = hip.DeviceBuffer.from_array(np.array(toks, np.uint32))
    d_o = hip.DeviceBuffer(len(slots) * v * 4)
    try:
        if noalloc:
            rc = be.forward_batch_device_noalloc(len(slots), d_s.ptr, d_t.ptr, d_o.ptr, probs=probs)
            assert rc == ffi.BackendResult.OK, rc
        else:
            be.forward_batch_device(len(slots), d_s.ptr, d_t.ptr, d_o.ptr, probs=probs)
        assert be.device_status() == ffi.BackendResult.OK
        return d_o.download(np.float32, len(slots) * v).reshape(len(slots), v)
    finally:
        for b in (d_s, d_t, d_o):
            b.close()


def _run(be, noalloc, calls, probs, state_slots, dims):
    be.batch_reset(None)
    outs = [_call(be, noalloc, s, t, probs) for s, t in calls]
    states = [[be.get_state(s, l, dims.d_inner, dims.d_conv) for l in (0, dims.n_layer - 1)] for s in state_slots]
    return outs, states


@pytest.mark.parametrize("which,profile,probs", [("small", 0, False), ("small", 6, True), ("m130", Q8ROW_ALL, False),
                                                  ("small", ffi.PROFILE_Q8_G64 | ffi.PROFILE_EXACT | ffi.PROFILE_FMA, False)])
def test_noalloc_step_equals_device_step(tmp_path, full_model, which, profile, probs):
    if which == "small":
        dims = rbin.MambaDims(vocab=1000, d_model=96, n_layer=3)
        path = str(tmp_path / "small.rbin")
        synth.write_synthetic_mamba(path, dims, seed=12)
        n1, n2, cap = 200, 37, 260
    else:
        dims, path = rbin.MAMBA_130M, full_model
        n1, n2, cap = 128, 19, 300
    rng = np.random.default_rng(21)
    with ffi.PluginBackend(path, profile=profile) as be:
        v = be.vocab
        be.batch_init(cap)
        s1 = [int(s) for s in rng.permutation(cap)[:n1]]
        s2 = [int(s) for s in rng.permutation(s1)[:n2]]      # the second call advances some of them again
        calls = [(s1, [int(x) for x in rng.integers(0, v, n1)]), (s2, [int(x) for x in rng.integers(0, v, n2)])]
        watch = [s2[0], s1[-1], next(s for s in range(cap) if s not in s1)]
        ref, ref_state = _run(be, False, calls, probs, watch, dims)
        got, got_state = _run(be, True, calls, probs, watch, dims)
        for r, g in zip(ref, got):
            assert np.array_equal(bits(r), bits(g))
        for a, b in zip(ref_state, got_state):
            for (c0, x0), (c1, x1) in zip(a, b):
                assert np.array_equal(c0, c1) and np.array_equal(x0, x1)


def test_noalloc_refuses_a_batch_beyond_its_scratch(full_model):
    with ffi.PluginBackend(full_model, profile=Q8ROW_ALL) as be:
        v = be.vocab
        be.batch_init(1024)
        before = be.get_state(5, 0, 1536, 4)
        n = 1000                                             # 44.7 MB of scratch at Mamba-130M
        d_s = hip.DeviceBuffer.from_array(np.arange(n, dtype=np.uint32))
        d_t = hip.DeviceBuffer.from_array(np.zeros(n, np.uint32))
        d_o = hip.DeviceBuffer(n * v * 4)
        try:
            rc = be.forward_batch_device_noalloc(n, d_s.ptr, d_t.ptr, d_o.ptr)
            assert rc == ffi.BackendResult.INVALID_ARGUMENT
            assert be.device_status() == ffi.BackendResult.OK
            after = be.get_state(5, 0, 1536, 4)
            assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])
        finally:
            for b in (d_s, d_t, d_o):
                b.close()
