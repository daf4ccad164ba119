import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP library through the C ABI")


@pytest.fixture(scope="session")
def full_model(tmp_path_factory):
    """Mamba-130M (d 768, 24 layers, vocab 50280) with synthetic seed-0 weights, shared by
    every GPU module of the session."""
    from redukt_amd import rbin, synth

    p = str(tmp_path_factory.mktemp("mamba130m") / "model.rbin")
    synth.write_synthetic_mamba(p, rbin.MAMBA_130M, seed=0)
    return p


# Worker pools stay within one GPU's share of host cores (16), whatever the machine
# reports: the oracle's GEMV threads and the host library's coding threads.
os.environ.setdefault("ORACLE_THREADS", str(min(os.cpu_count() or 1, 16)))
os.environ.setdefault("REDUKT_HOST_THREADS", str(min(os.cpu_count() or 1, 16)))
