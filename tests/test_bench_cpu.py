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
