"""bench.py's CPU library figure evaluates the same model as the oracle.

`cpu_library` times the benchmark model through torch's CPU conv2d; its graph
walk (bench.torch_cpu_runner) must compute the model the oracle computes in
fp32 throughout, or the figure would time a different network.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

from arthip_amd import models
from oracle.model import run_model

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402


@pytest.mark.parametrize("builder,hw", [(models.r8f64, (12, 20)), (models.shipped_like, (10, 18)),
                                        (models.c4f32, (8, 12)), (models.r16f96, (6, 10))])
def test_torch_runner_matches_the_fp32_oracle(builder, hw):
    spec = builder(seed=0)
    x = models.synthetic_input((1, spec.in_channels) + hw, seed=1)
    got = bench.torch_cpu_runner(spec.model, x)().numpy()
    want = run_model(spec.model, x, round_fp16=False)
    assert got.shape == want.shape
    rel = np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2))
    assert rel < 1e-4, rel


def test_launch_work_counts_each_distinct_tensor_once():
    """A fused R8F64 block's residual is its own input: input + output, 531 MB at
    1080p; the last block adds the global skip (796 MB). A shipped-architecture
    block (the last two convs of a 3-conv block) reads its input, the block's
    residual (another tensor) and writes its output: 796 MB."""
    px = 1080 * 1920
    act = 2.0 * px * 64
    w2 = 2 * 18.0 * 64 * 64
    r8 = models.r8f64(seed=0)
    steps = ["direct_conv"] + ["winograd_block"] * 8 + ["winograd_conv"]
    got = [x["bytes"] for x in bench.launch_work(r8, steps, px)]
    assert got[1:8] == [2 * act + w2] * 7
    assert got[8] == 3 * act + w2
    sh = models.shipped_like(seed=0)
    steps = ["direct_conv"] + ["winograd_conv", "winograd_block"] * 8 + ["winograd_conv"] * 2
    got = [x["bytes"] for x in bench.launch_work(sh, steps, px)]
    assert got[2] == 3 * act + w2
    assert got[1] == 2 * act + 18.0 * 64 * 64


def test_end_to_end_reports_a_failed_filter_child(monkeypatch):
    """The VapourSynth-path rate runs in a child process; if the child fails,
    the bench line carries null and the error instead of failing as a whole."""
    import subprocess

    class Res:
        returncode = 1
        stdout = ""
        stderr = "no device"

    class Spec:
        in_channels = 1
        name = "r8f64"

    class Eng:
        def run(self, x):
            return x

    monkeypatch.setattr(subprocess, "run", lambda *a, **k: Res())
    out = bench.end_to_end(Spec(), Eng(), np.zeros((1, 1, 8, 8), np.float16), 2, 4)
    assert out["vs_filter_fps"] is None
    assert "exit 1" in out["vs_filter_error"] and "no device" in out["vs_filter_error"]
