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


@pytest.fixture(scope="session")
def oracle_plugin(tmp_path_factory):
    """The CPU oracle behind the reference's plugin ABI (tests/oracle_plugin.c), for Mamba
    and RWKV-7 files.  Linked -z nodelete: the driver unloads a plugin when it closes, and
    the oracle's worker threads must not outlive the code and state of an unloaded copy."""
    import subprocess

    here = os.path.join(ROOT, "tests")
    d = tmp_path_factory.mktemp("oracle_plugin")
    so = str(d / "liboracle_plugin.so")
    odir = os.path.join(ROOT, "oracle")
    subprocess.run(["gcc", "-O2", "-std=gnu11", "-shared", "-fPIC", "-I", odir, os.path.join(here, "oracle_plugin.c"),
                    "-o", so, "-L", odir, "-loracle", "-Wl,-rpath," + odir, "-Wl,-z,nodelete"], check=True)
    return so


# Worker pools stay within one GPU's share of host cores (16), whatever the machine
# reports: the oracle's GEMV threads and the host library's coding threads.
os.environ.setdefault("ORACLE_THREADS", str(min(os.cpu_count() or 1, 16)))
os.environ.setdefault("REDUKT_HOST_THREADS", str(min(os.cpu_count() or 1, 16)))
