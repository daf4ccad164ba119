"""Mamba-130M over 4,100 tokens, across the 4096-token reset that the host's tick schedule
(plugin_backend/model.rs:44-49) sends, compared with the oracle at every token; the oracle
resets on its own schedule (MambaState::maybe_periodic_reset, model.rs:315-320).

* The reference-order tier (int8 groups of 64, numeric contract 2), one stream: every logit
  of every token bit-identical to the oracle.
* The default matrix-core tier at the 32-stream int8 per-row workload (32 lockstep streams
  x 4,100 tokens of independent Zipf(1.1) ids, every projection int8 with per-row scales):
  one stream of the batch compared with the oracle's single stream at every token within
  max |logit error| <= 1e-3 and probability L1 <= 1e-4, its recurrent state after the
  horizon, and after the reset the stream's logits equal a fresh stream's fed the same
  tokens, bit for bit.

* cfg3's workload at its full horizon: F32, 128 lockstep streams x 2,048 tokens with the
  probability vector handed back every step, 8 streams against the oracle's softmax at every
  token (L1 <= 1e-4).
* cfg5's workload at its full horizon: int8 per-row, 1,024 lockstep streams x 512 tokens in
  two parts of 512, 8 streams across both parts against the oracle at every token.

Each test is up to about a minute of oracle steps on 16 host threads.
"""
import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, rbin, synth

pytestmark = pytest.mark.gpu

TOL_ABS = 1e-3
TOL_L1 = 1e-4
Q8ROW_ALL = ffi.PROFILE_Q8_ROW | ffi.PROFILE_Q8_SMALL
N_TOK = 4100
RESET = 4096


def probs64(logits):
    x = np.asarray(logits, np.float64)
    e = np.exp(x - x.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def test_mamba130m_reference_order_4100_tokens_across_the_reset(full_model):
    orc = O.MambaOracle(full_model, ffi.PROFILE_Q8_G64 | O.ORC_PROFILE_FMA, cap=1)
    orc.set_reset_every(RESET)
    toks = [int(x) for x in synth.zipf_tokens(np.random.default_rng(3), rbin.MAMBA_130M.vocab, (N_TOK,))]
    print("reference-order tier, 1 stream x 4100 tokens", flush=True)
    with ffi.PluginBackend(full_model, profile=ffi.PROFILE_Q8_G64 | ffi.PROFILE_EXACT | ffi.PROFILE_FMA) as be:
        be.prepare_streams(1)
        st = be.create_state()
        st.set_reset_every(RESET)
        g = np.empty((1, be.vocab), np.float32)
        for i, t in enumerate(toks):
            st.tick()
            be.forward_batch([st.slot], [t], g)
            c = orc.forward([0], [t])
            assert np.array_equal(g.view(np.uint32), np.ascontiguousarray(c, np.float32).view(np.uint32)), i
    orc.close()


def test_mamba130m_q8row_32_streams_4100_tokens_across_the_reset(full_model):
    n, watch = 32, 13
    rng = np.random.default_rng(106)
    toks = synth.zipf_tokens(rng, rbin.MAMBA_130M.vocab, (N_TOK, n))
    orc = O.MambaOracle(full_model, Q8ROW_ALL, cap=1)
    orc.set_reset_every(RESET)
    print(f"default tier int8 per-row, {n} streams x {N_TOK} tokens, stream {watch} against the oracle", flush=True)
    with ffi.PluginBackend(full_model, profile=Q8ROW_ALL) as be:
        be.prepare_streams(n)
        states = [be.create_state() for _ in range(n)]
        for s in states:
            s.set_reset_every(RESET)
        slots = [s.slot for s in states]
        g = np.empty((n, be.vocab), np.float32)
        worst = (0.0, 0.0, -1)
        for t in range(N_TOK):
            tl = [int(x) for x in toks[t]]
            be.forward_multi(tl, states, g)   # ticks every state, then one forward_batch
            c = orc.forward([0], [tl[watch]])[0]
            err = float(np.max(np.abs(g[watch].astype(np.float64) - c)))
            l1 = float(np.abs(probs64(g[watch]) - probs64(c)).sum())
            assert err <= TOL_ABS and l1 <= TOL_L1, f"token {t}: max|dlogit|={err:.3e} L1={l1:.3e}"
            if (err, l1) > worst[:2]:
                worst = (err, l1, t)
            if t in (RESET - 1, N_TOK - 1):
                for layer in (0, 11, 23):
                    gc, gs = be.get_state(slots[watch], layer, 1536, 4)
                    cc, cs = orc.state(0, layer)
                    np.testing.assert_allclose(gc, cc, rtol=1e-3, atol=1e-4)
                    np.testing.assert_allclose(gs, cs, rtol=1e-3, atol=1e-4)
        # after the reset the batch restarted from zero state: a fresh single stream fed
        # the same four tokens reaches the same logits, bit for bit (batch invariance)
        last = np.array(g[watch])
        be.batch_init(1)
        one = np.empty((1, be.vocab), np.float32)
        for t in range(RESET, N_TOK):
            be.forward_batch([0], [int(toks[t, watch])], one)
        assert np.array_equal(one[0].view(np.uint32), last.view(np.uint32))
    orc.close()
    print(f"stream {watch}: worst max|dlogit|={worst[0]:.3e} L1={worst[1]:.3e} (token {worst[2]})")


def test_mamba130m_f32_128_streams_2048_tokens_probability_vector(full_model):
    # cfg3's workload at its full horizon: Mamba-130M F32, 128 lockstep streams x 2,048
    # Zipf(1.1) tokens, the probability vector handed back every step; every 16th stream
    # (8 of them) against the oracle's softmax at every token (L1 <= 1e-4, rows summing to 1).
    n, steps = 128, 2048
    watch = list(range(0, n, 16))
    toks = synth.zipf_tokens(np.random.default_rng(303), rbin.MAMBA_130M.vocab, (steps, n))
    orc = O.MambaOracle(full_model, 0, cap=len(watch))
    print(f"F32, {n} streams x {steps} tokens, probabilities of streams {watch} against the oracle", flush=True)
    with ffi.PluginBackend(full_model, profile=0) as be:
        be.batch_init(n)
        p = np.empty((n, be.vocab), np.float32)
        worst = 0.0
        for t in range(steps):
            tl = [int(x) for x in toks[t]]
            be.forward_batch(list(range(n)), tl, p, probs=True)
            c = orc.forward(list(range(len(watch))), [tl[s] for s in watch])
            ref = np.stack([O.softmax(r) for r in c]).astype(np.float64)
            got = p[watch].astype(np.float64)
            l1 = np.abs(got - ref).sum(axis=1)
            assert np.all(l1 <= TOL_L1), (t, float(l1.max()))
            assert np.all(np.abs(got.sum(axis=1) - 1.0) < 1e-5), t
            worst = max(worst, float(l1.max()))
            if t % 512 == 511:
                print(f"token {t + 1}: worst L1 so far {worst:.2e}", flush=True)
    orc.close()


def test_mamba130m_q8row_1024_streams_512_tokens(full_model):
    # cfg5's workload at its full horizon: Mamba-130M int8 per-row on every projection,
    # 1,024 lockstep streams x 512 Zipf(1.1) tokens (two parts of 512 streams, every
    # projection a 512-column skinny GEMM); 8 streams spread over both parts against the
    # oracle at every token.
    n, steps = 1024, 512
    watch = [0, 137, 300, 511, 512, 700, 901, 1023]
    toks = synth.zipf_tokens(np.random.default_rng(505), rbin.MAMBA_130M.vocab, (steps, n))
    orc = O.MambaOracle(full_model, Q8ROW_ALL, cap=len(watch))
    print(f"int8 per-row, {n} streams x {steps} tokens, streams {watch} against the oracle", flush=True)
    with ffi.PluginBackend(full_model, profile=Q8ROW_ALL) as be:
        be.batch_init(n)
        g = np.empty((n, be.vocab), np.float32)
        worst = (0.0, 0.0)
        for t in range(steps):
            tl = [int(x) for x in toks[t]]
            be.forward_batch(list(range(n)), tl, g)
            c = orc.forward(list(range(len(watch))), [tl[s] for s in watch])
            err = float(np.max(np.abs(g[watch].astype(np.float64) - c)))
            l1 = float(np.max(np.abs(probs64(g[watch]) - probs64(c)).sum(axis=-1)))
            assert err <= TOL_ABS and l1 <= TOL_L1, f"token {t}: max|dlogit|={err:.3e} L1={l1:.3e}"
            worst = (max(worst[0], err), max(worst[1], l1))
            if t % 128 == 127:
                print(f"token {t + 1}: worst max|dlogit| {worst[0]:.2e} L1 {worst[1]:.2e}", flush=True)
    orc.close()
