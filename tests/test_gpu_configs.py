"""The benchmark workloads at their full sizes, on the GPU, against the CPU oracle.

Each test runs one of the workload configurations through the C ABI and compares every
stream's output with the oracle (a C restatement of the reference CPU path) on the same
seeded weights and tokens: max |logit error| <= 1e-3 and probability-vector L1 <= 1e-4.

* Mamba-130M F32, one stream, 1024 tokens through the v1 entry point
  (redukt_backend_forward), compared at every token: recurrent-state drift over the
  whole horizon.
* Mamba-130M int8 per-row, 32 lockstep streams, 256 steps, every step compared, on the
  matrix-core tier and on the wavefront-GEMV tier.
* Mamba-130M F32, 128 streams, probability vector through forward_batch_probs
  (softmax_into, src/domain/tensor.rs:1917-1933), every row; one stream alone equals the
  same stream inside the 128-stream batch, bit for bit (PLUGIN-FFI-V2.md:97-101).
* Mamba-130M int8 per-row, 1024 streams, every row; one stream's bits alone == in the
  batch; on both tiers.
* RWKV-7 0.1B at its real vocabulary (65,536), 64 streams, F32 and int8 weight-only.
"""
import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, hip, rwkv, synth

pytestmark = pytest.mark.gpu

TOL_ABS = 1e-3
TOL_L1 = 1e-4
Q8ROW_ALL = ffi.PROFILE_Q8_ROW | ffi.PROFILE_Q8_SMALL


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def probs64(logits):
    x = np.asarray(logits, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def parity(gpu, cpu):
    err = float(np.max(np.abs(gpu.astype(np.float64) - cpu)))
    l1 = float(np.max(np.abs(probs64(gpu) - probs64(cpu)).sum(axis=-1)))
    return err, l1


def test_mamba130m_f32_single_stream_1024_tokens(full_model):
    n_tok = 1024
    rng = np.random.default_rng(101)
    seq = [int(t) for t in synth.zipf_tokens(rng, 50280, (n_tok,))]
    with ffi.PluginBackend(full_model, profile=0) as be:
        orc = O.MambaOracle(full_model, 0, cap=1)
        out = np.empty(be.vocab, np.float32)
        be.lib.lib.redukt_backend_reset_state()
        worst = (0.0, 0.0)
        for t, tok in enumerate(seq):
            rc = be.lib.lib.redukt_backend_forward(tok, out.ctypes.data_as(ffi._f32p), be.vocab)
            assert rc == ffi.BackendResult.OK
            c = orc.forward([0], [tok])[0]
            err, l1 = parity(out[None], c[None])
            assert err <= TOL_ABS and l1 <= TOL_L1, f"token {t}: max|dlogit|={err:.3e} L1={l1:.3e}"
            worst = max(worst, (err, l1))
        orc.close()
    print(f"Mamba-130M F32 v1, {n_tok} tokens: worst max|dlogit|={worst[0]:.3e} L1={worst[1]:.3e}")


TIERS = [pytest.param(0, id="matrix-core"), pytest.param(ffi.PROFILE_GEMV, id="gemv")]


@pytest.mark.parametrize("tier", TIERS)
def test_mamba130m_q8_32_streams_256_steps(full_model, tier):
    n, steps = 32, 256
    rng = np.random.default_rng(102)
    toks = synth.zipf_tokens(rng, 50280, (steps, n))
    print(f"int8 per-row, {n} streams x {steps} steps, tier bits {tier}", flush=True)
    with ffi.PluginBackend(full_model, profile=Q8ROW_ALL | tier) as be:
        orc = O.MambaOracle(full_model, Q8ROW_ALL, cap=n)
        be.batch_init(n)
        slots = list(range(n))
        g = np.empty((n, be.vocab), np.float32)
        worst = (0.0, 0.0)
        for t in range(steps):
            tl = [int(x) for x in toks[t]]
            be.forward_batch(slots, tl, g)
            c = orc.forward(slots, tl)
            err, l1 = parity(g, c)
            assert err <= TOL_ABS and l1 <= TOL_L1, f"step {t}: max|dlogit|={err:.3e} L1={l1:.3e}"
            worst = max(worst, (err, l1))
        # the recurrent state after the whole horizon
        for s in (0, 31):
            for layer in (0, 23):
                gc, gs = be.get_state(s, layer, 1536, 4)
                cc, cs = orc.state(s, layer)
                np.testing.assert_allclose(gc, cc, rtol=1e-3, atol=1e-4)
                np.testing.assert_allclose(gs, cs, rtol=1e-3, atol=1e-4)
        orc.close()
    print(f"Mamba-130M int8 per-row, {n} streams x {steps} steps: worst max|dlogit|={worst[0]:.3e} L1={worst[1]:.3e}")


def test_mamba130m_f32_128_streams_probability_vector(full_model):
    n, steps = 128, 2
    rng = np.random.default_rng(103)
    toks = synth.zipf_tokens(rng, 50280, (steps, n))
    with ffi.PluginBackend(full_model, profile=0) as be:
        orc = O.MambaOracle(full_model, 0, cap=n)
        be.batch_init(n + 1)
        slots = list(range(n))
        p = np.empty((n, be.vocab), np.float32)
        worst = 0.0
        for t in range(steps):
            tl = [int(x) for x in toks[t]]
            be.forward_batch(slots, tl, p, probs=True)
            c = orc.forward(slots, tl)
            ref = np.stack([O.softmax(r) for r in c]).astype(np.float64)
            l1 = np.abs(p.astype(np.float64) - ref).sum(axis=1)
            assert np.all(l1 <= TOL_L1), (t, float(l1.max()))
            assert np.all(np.abs(p.astype(np.float64).sum(axis=1) - 1.0) < 1e-5)
            worst = max(worst, float(l1.max()))
        orc.close()
        # Stream 77 of a fresh 128-stream batch (slot n, never used above) against the same
        # stream alone: the F32 out_proj takes two stream groups per workgroup from 80
        # streams, one below; the probabilities must not depend on that.
        seq = [int(x) for x in synth.zipf_tokens(rng, 50280, (2,))]
        be.batch_reset(None)
        alone = []
        for tok in seq:
            a = np.empty((1, be.vocab), np.float32)
            be.forward_batch([n], [tok], a, probs=True)
            alone.append(a[0].copy())
        be.batch_reset(None)
        others = [int(s) for s in rng.permutation(n)[: n - 1]]
        for i, tok in enumerate(seq):
            sl = others[:77] + [n] + others[77:]
            tl = [int(x) for x in synth.zipf_tokens(rng, 50280, (n,))]
            tl[77] = tok
            be.forward_batch(sl, tl, p, probs=True)
            assert np.array_equal(bits(p[77]), bits(alone[i])), i
    print(f"Mamba-130M F32, {n} streams, probability vector: worst L1={worst:.3e}")


@pytest.mark.parametrize("tier", TIERS)
def test_mamba130m_q8_1024_streams(full_model, tier):
    """The large-batch workload (1024 streams), on the matrix-core tier and on the
    wavefront-GEMV tier, whose projections are then 1024-column skinny GEMMs computed as
    dot products on the vector ALUs: every row against the oracle, one stream alone equal
    to the same stream inside the batch."""
    n = 1024
    rng = np.random.default_rng(104)
    toks = synth.zipf_tokens(rng, 50280, (2, n))
    print(f"int8 per-row, {n} streams, tier bits {tier}", flush=True)
    with ffi.PluginBackend(full_model, profile=Q8ROW_ALL | tier) as be:
        orc = O.MambaOracle(full_model, Q8ROW_ALL, cap=n)
        be.batch_init(n + 1)
        slots = list(range(n))
        g = np.empty((n, be.vocab), np.float32)
        worst = (0.0, 0.0)
        for t in range(2):
            tl = [int(x) for x in toks[t]]
            be.forward_batch(slots, tl, g)
            c = orc.forward(slots, tl)
            err, l1 = parity(g, c)
            assert err <= TOL_ABS and l1 <= TOL_L1, f"step {t}: max|dlogit|={err:.3e} L1={l1:.3e}"
            worst = max(worst, (err, l1))
        orc.close()
        # one stream alone == the same stream at position 1000 of a 1024-stream batch
        tok = int(toks[0, 5])
        be.batch_reset(None)
        alone = np.empty((1, be.vocab), np.float32)
        be.forward_batch([n], [tok], alone)
        be.batch_reset(None)
        sl = [int(s) for s in rng.permutation(n)[: n - 1]]
        sl.insert(1000, n)
        tl = [int(x) for x in synth.zipf_tokens(rng, 50280, (n,))]
        tl[1000] = tok
        be.forward_batch(sl, tl, g)
        assert np.array_equal(bits(g[1000]), bits(alone[0]))
    print(f"Mamba-130M int8 per-row, {n} streams: worst max|dlogit|={worst[0]:.3e} L1={worst[1]:.3e}")


@pytest.fixture(scope="module")
def rwkv_0_1b(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("rwkv_0_1b") / "rwkv7_0_1b.rbin")
    rwkv.write_synthetic(p, rwkv.RWKV7_0_1B, seed=0)
    return p


@pytest.mark.parametrize("profile", [0, 2])
def test_rwkv7_0_1b_64_streams_full_vocab(rwkv_0_1b, profile):
    n, steps = 64, 3
    rng = np.random.default_rng(105)
    toks = rng.integers(0, 256, size=(steps, n))   # byte-level ids
    with ffi.PluginBackend(rwkv_0_1b, profile=profile) as be:
        assert be.vocab == 65536
        orc = O.RwkvOracle(rwkv_0_1b, profile, cap=n)
        be.batch_init(n)
        slots = list(range(n))
        g = np.empty((n, be.vocab), np.float32)
        worst = (0.0, 0.0)
        for t in range(steps):
            tl = [int(x) for x in toks[t]]
            be.forward_batch(slots, tl, g)
            c = orc.forward(slots, tl)
            err, l1 = parity(g, c)
            assert err <= TOL_ABS and l1 <= TOL_L1, f"step {t}: max|dlogit|={err:.3e} L1={l1:.3e}"
            worst = max(worst, (err, l1))
        orc.close()
    print(f"RWKV-7 0.1B profile {profile}, {n} streams, vocab 65536: worst max|dlogit|={worst[0]:.3e} "
          f"L1={worst[1]:.3e}")
