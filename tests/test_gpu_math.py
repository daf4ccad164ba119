"""The portable element-wise functions as the GPU computes them (redukt_backend_eval_math)
against the CPU oracle's, bit for bit: exp, lane exp, ln, softplus, lane sigmoid and
sigmoid (src/domain/tensor.rs:765-885).  Every element-wise phase of both steps is built
from these, so a fused multiply-add or any other deviation in them shows up here."""
import numpy as np
import pytest

from oracle import oracle as O
from redukt_amd import ffi, hip

pytestmark = pytest.mark.gpu


def inputs():
    rng = np.random.default_rng(3)
    special = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 20.0, 20.000002, 19.999998, 88.37626, 88.5, -87.33654,
                        -87.5, -103.0, 1e-30, -1e-30, 1e-45, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan,
                        2.0 ** -126, 7.0, -7.0, 0.6931472, 1e-7, -1e-7], np.float32)
    return np.concatenate([special, rng.normal(0, 4, 20000).astype(np.float32),
                           rng.uniform(-100, 100, 20000).astype(np.float32),
                           rng.uniform(1e-6, 50, 20000).astype(np.float32),
                           np.linspace(-30, 30, 20001, dtype=np.float32)])


CPU = {"exp": O.expf, "lane_exp": O.lane_expf, "ln": O.lnf, "softplus": O.softplus, "sigmoid": O.sigmoidf,
       "lane_sigmoid": lambda v: O.lib().orc_lane_sigmoidf(v)}


@pytest.mark.parametrize("fn", sorted(ffi.MATH_FNS))
def test_device_math_is_bit_identical_to_the_oracle(fn):
    assert hip.device_count() > 0, "no GPU visible"
    lib = ffi.PluginLibrary()
    assert lib.has_v3
    x = inputs()
    if fn == "ln":
        x = np.concatenate([np.abs(x), np.array([0.0, -1.0, 1.0], np.float32)])
    gpu = lib.eval_math(fn, x)
    cpu = np.array([CPU[fn](float(v)) for v in x], np.float32)
    both_nan = np.isnan(gpu) & np.isnan(cpu)
    diff = (gpu.view(np.uint32) != cpu.view(np.uint32)) & ~both_nan
    idx = np.flatnonzero(diff)
    assert idx.size == 0, f"{fn}: {idx.size} of {x.size} differ, e.g. x={x[idx[:5]]} gpu={gpu[idx[:5]]} cpu={cpu[idx[:5]]}"
