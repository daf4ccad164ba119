"""bench.py host logic, without a GPU: the one-GPU contract and the byte model behind
step_GBps / roofline.achieved.

The weight and state figures are the ones computed for Mamba-130M from the model shape
(24 layers, d 768, d_inner 1536, d_state 16, d_conv 4, dt_rank 48, vocab 50280, tied head):
the F32 step reads 516,541,440 weight bytes, the int8 per-row profile (in_proj, x_proj,
dt_proj, out_proj and head quantised, one f32 scale per row) 132,461,472, the reference's
group-64 profile on in_proj, out_proj and head 153,614,208; each stream reads and writes
2 x (442,368 + 2,359,296) bytes of recurrent state per step, writes 201,120 bytes of logits
and reads one 3,072-byte embedding row.
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from redukt_amd import rbin  # noqa: E402

M130 = rbin.MAMBA_130M
PER_STREAM = 2 * (442_368 + 2_359_296) + 201_120 + 3_072


@pytest.mark.parametrize("profile,weights", [(0, 516_541_440), (6, 132_461_472), (1, 153_614_208)])
def test_step_bytes_match_the_model_figures(profile, weights):
    assert bench.step_bytes(M130, profile, 0) == weights
    for n in (1, 32, 128, 1024):
        assert bench.step_bytes(M130, profile, n) == weights + n * PER_STREAM


@pytest.mark.parametrize("profile", [0, 1, 2, 6])
def test_launch_bytes_cover_the_step_weights(profile):
    # With no streams only weights and per-layer vectors move: one launch of each layer
    # kernel per layer plus the head reads exactly the step's weight bytes.  (With streams
    # the launches also count the activations they pass to each other, which the step
    # figure leaves out.)
    a = bench.algorithmic_bytes(M130, profile, 0)
    total = a["embed"] + M130.n_layer * (a["mix_in"] + a["scan"] + a["mix_out"]) + a["head"]
    assert total == bench.step_bytes(M130, profile, 0)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr or "one process per GPU" in r.stderr
