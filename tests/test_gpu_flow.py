"""The persistent step kernel (every Mamba layer of a step in one cooperative launch) on
the GPU, through the C ABI.

The kernel runs the per-layer kernels' bodies as tasks (same tiles, k-splits and
summation orders), so a step through it must give the per-layer path's bits exactly:

* logits, probabilities and recurrent state bit for bit equal to the per-layer path
  (REDUKT_GPU_FLOW=0) at 16 (tasks in ticket order), 150 (a last group of 6 streams; tasks
  assigned statically, six steps: a stale hand-over read shows as one stream's bits
  differing) and 1024 streams (ticket order, two workgroups per CU), for the weight profiles
  it serves (int8 per-row with F32 or int8 x_proj/dt_proj, fast or exact scan decay), over
  several steps with scattered slots;
* parity with the CPU oracle at 128 streams (max |logit error| <= 1e-3, probability L1
  <= 1e-4);
* the device-side argument check of forward_batch_device contains bad entries as on the
  per-layer path, and a clean run leaves the error word clear (no wait timed out, every
  workgroup on the XCD the kernel assumed);
* profiles it does not serve (F32, group-64 int8) still run, on the per-layer path;
* the kernel's probe class brackets its launch with a pair of events.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, hip, synth

pytestmark = pytest.mark.gpu

TOL_ABS = 1e-3
TOL_L1 = 1e-4
Q8ROW = ffi.PROFILE_Q8_ROW
Q8ROW_ALL = ffi.PROFILE_Q8_ROW | ffi.PROFILE_Q8_SMALL
EXACT = ffi.PROFILE_EXACT_SCAN
KC_FLOW = ffi.KC_FLOW
VOCAB = 50280


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def probs64(logits):
    x = np.asarray(logits, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def backend(path, profile, flow):
    os.environ["REDUKT_GPU_FLOW"] = "1" if flow else "0"
    try:
        return ffi.PluginBackend(path, profile=profile)
    finally:
        del os.environ["REDUKT_GPU_FLOW"]


class FlowProbe:
    """Events around every launch of the persistent kernel: `launches()` says how many
    steps actually ran it (a step that fell back to the per-layer path records none)."""

    def __init__(self, be, cap):
        self.be = be
        self.evs = [hip.Event() for _ in range(2 * cap)]
        self.arr = (ctypes.c_void_p * len(self.evs))(*[e.h for e in self.evs])
        be.probe_kernel(KC_FLOW, self.arr)

    def launches(self):
        used = self.be.probe_used()
        self.be.probe_kernel(0, None)
        hip.stream_sync(self.be.stream())
        us = [1e3 * self.evs[2 * i].elapsed_ms(self.evs[2 * i + 1]) for i in range(used // 2)]
        for e in self.evs:
            e.close()
        return used // 2, us


def run_sequence(path, profile, flow, n, steps, seed, probs=False, expect_flow=None):
    """`steps` steps of n streams on scattered slots of an (n + 5)-slot pool; returns the
    outputs, the conv and SSM state of three streams at the first and last layer, and
    the device status afterwards.  With flow on, checks that every step ran the
    persistent kernel (expect_flow, default flow) or none did."""
    rng = np.random.default_rng(seed)
    slots = [int(s) for s in rng.permutation(n + 5)[:n]]
    toks = synth.zipf_tokens(rng, VOCAB, (steps, n))
    expect_flow = flow if expect_flow is None else expect_flow
    with backend(path, profile, flow) as be:
        be.batch_init(n + 5)
        probe = FlowProbe(be, steps) if flow else None
        outs = []
        for t in range(steps):
            g = np.empty((n, be.vocab), np.float32)
            be.forward_batch(slots, [int(x) for x in toks[t]], g, probs=probs)
            outs.append(g)
        if probe is not None:
            ran, _ = probe.launches()
            assert ran == (steps if expect_flow else 0), (ran, steps)
        states = []
        for i in sorted({0, n // 2, n - 1}):
            for layer in (0, 23):
                states.extend(be.get_state(slots[i], layer, 1536, 4))
        status = be.device_status()
    return outs, states, status


@pytest.mark.parametrize("n,profile,steps", [(16, Q8ROW_ALL, 3), (150, Q8ROW_ALL, 6), (150, Q8ROW, 2),
                                             (150, Q8ROW_ALL | EXACT, 2), (1024, Q8ROW_ALL, 2)])
def test_flow_equals_per_layer_path(full_model, n, profile, steps):
    ref_out, ref_st, ref_status = run_sequence(full_model, profile, False, n, steps, seed=n + profile)
    out, st, status = run_sequence(full_model, profile, True, n, steps, seed=n + profile)
    assert ref_status == ffi.BackendResult.OK and status == ffi.BackendResult.OK, (ref_status, status)
    for t, (a, b) in enumerate(zip(ref_out, out)):
        same = np.all(bits(a) == bits(b), axis=1)
        assert same.all(), f"step {t}: streams {np.flatnonzero(~same)[:8].tolist()} differ"
    for i, (a, b) in enumerate(zip(ref_st, st)):
        assert np.array_equal(bits(a), bits(b)), f"state array {i}"


def test_flow_probabilities_equal_per_layer_path(full_model):
    ref, _, _ = run_sequence(full_model, Q8ROW_ALL, False, 64, 2, seed=11, probs=True)
    got, _, status = run_sequence(full_model, Q8ROW_ALL, True, 64, 2, seed=11, probs=True)
    assert status == ffi.BackendResult.OK
    for a, b in zip(ref, got):
        assert np.array_equal(bits(a), bits(b))
    assert np.allclose(got[-1].astype(np.float64).sum(axis=1), 1.0, atol=1e-5)


def test_flow_oracle_parity_128_streams(full_model):
    n, steps = 128, 2
    rng = np.random.default_rng(23)
    toks = synth.zipf_tokens(rng, VOCAB, (steps, n))
    with backend(full_model, Q8ROW_ALL, True) as be:
        orc = O.MambaOracle(full_model, Q8ROW_ALL, cap=n)
        be.batch_init(n)
        slots = list(range(n))
        g = np.empty((n, be.vocab), np.float32)
        probe = FlowProbe(be, steps)
        for t in range(steps):
            tl = [int(x) for x in toks[t]]
            be.forward_batch(slots, tl, g)
            c = orc.forward(slots, tl)
            err = float(np.max(np.abs(g.astype(np.float64) - c)))
            l1 = float(np.max(np.abs(probs64(g) - probs64(c)).sum(axis=-1)))
            assert err <= TOL_ABS and l1 <= TOL_L1, f"step {t}: max|dlogit|={err:.3e} L1={l1:.3e}"
        assert probe.launches()[0] == steps
        for s in (0, 127):
            gc, gs = be.get_state(s, 23, 1536, 4)
            cc, cs = orc.state(s, 23)
            np.testing.assert_allclose(gc, cc, rtol=1e-3, atol=1e-4)
            np.testing.assert_allclose(gs, cs, rtol=1e-3, atol=1e-4)
        assert be.device_status() == ffi.BackendResult.OK
        orc.close()


def test_flow_device_check_contains_bad_entries(full_model):
    n = 40
    with backend(full_model, Q8ROW_ALL, True) as be:
        be.batch_init(48)
        warm = np.empty((48, be.vocab), np.float32)
        be.forward_batch(list(range(48)), [(7 * s + 3) % VOCAB for s in range(48)], warm)
        before = {s: be.get_state(s, 5, 1536, 4) for s in (41, 42, 47)}
        slots = list(range(n))
        slots[3] = 60            # out of range
        slots[9] = slots[8]      # repeated: the later entry is routed to the scratch slot
        toks = [(11 * s + 1) % VOCAB for s in range(n)]
        toks[17] = VOCAB + 2     # token out of range
        d_s = hip.DeviceBuffer.from_array(np.array(slots, np.uint32))
        d_t = hip.DeviceBuffer.from_array(np.array(toks, np.uint32))
        d_o = hip.DeviceBuffer(n * be.vocab * 4)
        try:
            probe = FlowProbe(be, 1)
            be.forward_batch_device(n, d_s.ptr, d_t.ptr, d_o.ptr)
            assert probe.launches()[0] == 1
            assert be.device_status() == ffi.BackendResult.INVALID_ARGUMENT
            for s, (c0, x0) in before.items():
                c1, x1 = be.get_state(s, 5, 1536, 4)
                assert np.array_equal(bits(c0), bits(c1)) and np.array_equal(bits(x0), bits(x1)), s
            be.forward_batch(list(range(n)), [(5 * s) % VOCAB for s in range(n)], warm[:n])
            assert be.device_status() == ffi.BackendResult.OK
        finally:
            for b in (d_s, d_t, d_o):
                b.close()


@pytest.mark.parametrize("profile", [ffi.PROFILE_F32, ffi.PROFILE_Q8_G64])
def test_profiles_without_flow_still_run(full_model, profile):
    ref, _, _ = run_sequence(full_model, profile, False, 32, 1, seed=5)
    got, _, status = run_sequence(full_model, profile, True, 32, 1, seed=5, expect_flow=False)
    assert status == ffi.BackendResult.OK
    assert np.array_equal(bits(ref[0]), bits(got[0]))


def test_flow_probe_brackets_the_launch(full_model):
    with backend(full_model, Q8ROW_ALL, True) as be:
        n = 64
        be.batch_init(n)
        g = np.empty((n, be.vocab), np.float32)
        be.forward_batch(list(range(n)), list(range(n)), g)
        probe = FlowProbe(be, 3)
        for t in range(2):
            be.forward_batch(list(range(n)), [(t + s) % VOCAB for s in range(n)], g)
        ran, us = probe.launches()
        assert ran == 2 and all(0.0 < u < 1e5 for u in us), (ran, us)
        assert be.device_status() == ffi.BackendResult.OK
