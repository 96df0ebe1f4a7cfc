"""The ONNX Runtime execution provider's capability and compile on the GPU.

Mirrors tests/correctness/test_ep.py without ONNX Runtime (not installed):
- an unusable device claims nothing (P1-6);
- a claimed run compiled into an engine (arthip_engine_build_subgraph) gives
  the same bits as the whole model when the run is the whole model (the
  shipped luma model, the fp32-boundary fixture of P1-4);
- a model split by an unsupported node runs as ONNX Runtime would run it
  (claimed runs on the GPU, the rest on the CPU) and matches the oracle.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from arthip_amd import onnx_proto as op
from arthip_amd.engine import Engine, get_capability
from tests.fixtures import _conv, _half, _model, fused_node_graph, kern

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_invalid_device_refuses_capability(fixtures):
    m = fixtures.get("ep_conv_fp32io").model
    assert get_capability(m, device_id=999) == []
    assert get_capability(m, device_id=0) == [[0, 1, 2]]


def test_whole_model_run_equals_the_engine():
    m = op.load(GOLDEN / "ArtCNN_R8F64_fp16.onnx")
    (run,) = get_capability(m, device_id=0)
    x = np.load(GOLDEN / "shipped_luma_48x64.npz")["x"]
    with Engine(0) as a, Engine(0) as b:
        got = a.build_subgraph(m, run).run(x)
        want = b.build(m).run(x)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_fp32_boundary_run(fixtures):
    fx = fixtures.get("ep_conv_fp32io")
    (run,) = get_capability(fx.model, device_id=0)
    rng = np.random.default_rng(2)
    for h, w in ((16, 16), (4, 4)):  # a second, smaller shape re-plans
        x = rng.uniform(-1, 1, (1, 1, h, w)).astype(np.float32)
        with Engine(0) as a, Engine(0) as b:
            got = a.build_subgraph(fx.model, run).run(x)
            want = b.build(fx.model).run(x)
        assert got.dtype == np.float32 and got.shape == (1, 1, h, w)
        np.testing.assert_array_equal(got, want)


def test_split_model_runs_like_the_fallback():
    from oracle.model import run_model
    w1, w2 = kern(31, 8, 4), kern(32, 4, 8)
    nodes = [_conv("x", "w1", None, "a"),
             op.node("Cast", ["a"], ["a32"], to=op.FLOAT),
             op.node("Cast", ["a32"], ["a16"], to=op.FLOAT16),
             _conv("a16", "w2", None, "y")]
    m = _model(nodes, "x", [1, 4, "h", "w"], op.FLOAT16, "y", [1, 4, "h", "w"], op.FLOAT16,
               [_half("w1", w1), _half("w2", w2)])
    runs = get_capability(m, device_id=0)
    assert runs == [[0], [3]]
    x = np.random.default_rng(3).uniform(-1, 1, (1, 4, 20, 28)).astype(np.float16)
    with Engine(0) as e1, Engine(0) as e2:
        a = e1.build_subgraph(m, runs[0]).run(x)
        a16 = a.astype(np.float32).astype(np.float16)  # the two Casts, on the CPU
        y = e2.build_subgraph(m, runs[1]).run(a16)
    want = run_model(m, x)
    assert y.shape == want.shape
    assert np.abs(y.astype(np.float64) - want).max() <= 2e-2


@pytest.mark.parametrize("which", ["shipped", "fp32io"])
def test_compile_from_the_fused_node_graph(which, fixtures):
    """Compile as the EP shim does it: the fused node's own graph, serialized on
    its own, built over all of its nodes, gives the same bits as the run built
    from the whole model."""
    if which == "shipped":
        m = op.load(GOLDEN / "ArtCNN_R8F64_fp16.onnx")
        x = np.load(GOLDEN / "shipped_luma_48x64.npz")["x"]
    else:
        m = op.load(fixtures.get("ep_conv_fp32io").model)
        x = np.random.default_rng(4).uniform(-1, 1, (1, 1, 18, 30)).astype(np.float32)
    (run,) = get_capability(m, device_id=0)
    sub = fused_node_graph(m, run)
    with Engine(0) as a, Engine(0) as b:
        got = a.build_subgraph(sub, list(range(len(sub.graph.nodes)))).run(x)
        want = b.build_subgraph(m, run).run(x)
    assert got.dtype == want.dtype and got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
