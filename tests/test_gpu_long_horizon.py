"""Mamba-130M on the reference-order tier (int8 groups of 64, numeric contract 2) for one
stream over 4,100 tokens, across the 4096-token reset that the host's tick schedule
(plugin_backend/model.rs:44-49) sends: every logit of every token bit-identical to the
oracle, which resets on its own schedule (MambaState::maybe_periodic_reset, model.rs:315-320).

About 80 s, nearly all of it the oracle's single-stream steps, so it runs only when
REDUKT_LONG_TESTS=1 is set:  REDUKT_LONG_TESTS=1 python -m pytest tests/test_gpu_long_horizon.py
"""
import os

import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, rbin, synth

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("REDUKT_LONG_TESTS") != "1",
                                 reason="80 s of oracle steps; set REDUKT_LONG_TESTS=1")]


def test_mamba130m_reference_order_4100_tokens_across_the_reset(full_model):
    orc = O.MambaOracle(full_model, ffi.PROFILE_Q8_G64 | O.ORC_PROFILE_FMA, cap=1)
    orc.set_reset_every(4096)
    toks = [int(x) for x in synth.zipf_tokens(np.random.default_rng(3), rbin.MAMBA_130M.vocab, (4100,))]
    with ffi.PluginBackend(full_model, profile=ffi.PROFILE_Q8_G64 | ffi.PROFILE_EXACT | ffi.PROFILE_FMA) as be:
        be.prepare_streams(1)
        st = be.create_state()
        st.set_reset_every(4096)
        g = np.empty((1, be.vocab), np.float32)
        for i, t in enumerate(toks):
            st.tick()
            be.forward_batch([st.slot], [t], g)
            c = orc.forward([0], [t])
            assert np.array_equal(g.view(np.uint32), np.ascontiguousarray(c, np.float32).view(np.uint32)), i
    orc.close()
