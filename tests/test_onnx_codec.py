"""The package's own ONNX protobuf codec (arthip_amd/onnx_proto.py) and the
engine's independent C++ decoder (arthip_amd/csrc/onnx.cc) on CPU."""

from __future__ import annotations

import collections
from pathlib import Path

import numpy as np
import pytest

from arthip_amd import models
from arthip_amd import onnx_proto as op
from arthip_amd.engine import Engine, EngineError

GOLDEN = Path(__file__).resolve().parent / "golden"
SHIPPED = GOLDEN / "ArtCNN_R8F64_fp16.onnx"


def test_roundtrip_preserves_fields():
    w = np.arange(2 * 3 * 3 * 3, dtype=np.float32).reshape(2, 3, 3, 3) / 7
    m = op.Model(graph=op.Graph(
        nodes=[op.node("Conv", ["x", "w"], ["y"], pads=[1, 1, 1, 1], strides=[1, 1],
                       auto_pad="NOTSET", alpha=0.5)],
        initializers=[op.tensor("w", w), op.tensor("th", w[0].astype(np.float16), typed_half=True),
                      op.Tensor(name="fd", dims=[3], data_type=op.FLOAT, float_data=[1.5, -2.0, 3.25]),
                      op.Tensor(name="neg", dims=[2], data_type=op.INT64, int64_data=[-1, 7])],
        inputs=[op.value_info("x", op.FLOAT16, [1, 3, "H", "W"])],
        outputs=[op.value_info("y", op.FLOAT16, [1, 2, None, 5])]))
    d = op.decode_model(op.encode_model(m))
    g = d.graph
    n = g.nodes[0]
    assert (n.op_type, n.inputs, n.outputs) == ("Conv", ["x", "w"], ["y"])
    assert n.attr("pads") == [1, 1, 1, 1] and n.attr("auto_pad") == "NOTSET"
    assert n.attr("alpha") == pytest.approx(0.5)
    t = {x.name: x for x in g.initializers}
    np.testing.assert_array_equal(t["w"].to_numpy(), w)
    np.testing.assert_array_equal(t["th"].to_numpy(), w[0].astype(np.float16))
    assert t["th"].int32_data and not t["th"].raw_data
    np.testing.assert_array_equal(t["fd"].to_numpy(), [1.5, -2.0, 3.25])
    np.testing.assert_array_equal(t["neg"].to_numpy(), [-1, 7])
    assert g.inputs[0].shape == [1, 3, "H", "W"] and g.inputs[0].elem_type == op.FLOAT16


def test_decodes_shipped_model():
    m = op.load(SHIPPED)
    c = collections.Counter(n.op_type for n in m.graph.nodes)
    # Structure of the shipped luma model: 70 nodes.
    assert len(m.graph.nodes) == 70
    assert c == {"Conv": 27, "Sigmoid": 16, "Mul": 16, "Add": 9, "DepthToSpace": 1, "Clip": 1}
    assert m.graph.inputs[0].elem_type == op.FLOAT16
    w0 = {t.name: t for t in m.graph.initializers}["kernel_oih_0"].to_numpy()
    assert w0.shape == (64, 1, 3, 3) and w0.dtype == np.float16


def test_reencoded_shipped_model_builds_identically():
    a = Engine(0).build(SHIPPED).describe()
    b = Engine(0).build(op.encode_model(op.load(SHIPPED))).describe()
    assert a == b


def test_cpp_decoder_rejects_malformed_bytes():
    good = models.c4f32().bytes()
    with pytest.raises(EngineError, match="failed to parse model file"):
        Engine(0).build(good[: len(good) // 2])
    with pytest.raises(EngineError, match="failed to parse model file"):
        Engine(0).build(b"\xff\xff\xff\xff\xff\xff\xff\xff\xff\xff\xff")


def test_cpp_decoder_accepts_unpacked_repeated_fields(monkeypatch):
    """Repeated scalars may be serialized one value per key (proto2 style); both
    decoders must accept that as well as the packed form."""
    packed = op.encode_attribute

    def unpacked(a):
        if a.type != op.A_INTS:
            return packed(a)
        return (op._str(1, a.name) + op._int(20, a.type) +
                b"".join(op._int(8, v) for v in a.ints))

    spec = models.c4f32()
    want = Engine(0).build(spec.bytes()).describe()
    monkeypatch.setattr(op, "encode_attribute", unpacked)
    raw = op.encode_model(spec.model)
    monkeypatch.undo()
    assert raw != spec.bytes()
    assert Engine(0).build(raw).describe() == want
    assert op.decode_model(raw).graph.nodes[0].attr("pads") == [1, 1, 1, 1]
