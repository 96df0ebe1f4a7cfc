"""Graph building through the C ABI on the CPU (no GPU needed): validation
messages, fusion decisions and shape propagation, mirroring the reference's
Build / PropagateShapes semantics (src/vapoursynth/hip_engine.cc:197-736)."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

from arthip_amd import models
from arthip_amd.engine import Engine, EngineError

SHIPPED = Path(__file__).resolve().parent / "golden" / "ArtCNN_R8F64_fp16.onnx"


def ops_of(eng: Engine) -> list[str]:
    return [l for l in eng.describe().splitlines() if l.startswith("op")]


@pytest.mark.parametrize("name,match", [
    ("conv_1x1", "3x3"),
    ("conv_short_bias", "bias"),
    ("conv_external", "external data"),
    ("add_const", "not an activation produced"),
    ("conv_pads_asym", "pads"),
    ("clip_dynamic_bound", "dynamic Clip bounds"),
    ("conv_m160", "128 output channels"),
    ("conv_c128", "96 input channels"),
])
def test_rejections(fixtures, name, match):
    with pytest.raises(EngineError, match=match):
        Engine(0).build(fixtures.get(name).model)


def test_broadcast_fails_shape_propagation(fixtures):
    e = Engine(0).build(fixtures.get("add_broadcast").model)
    with pytest.raises(EngineError, match="shape propagation failed"):
        e.output_shape((1, 4, 16, 16))


@pytest.mark.parametrize("shape", [(1, 1, 0, 16), (1, 1, 16, 0), (0, 1, 16, 16)])
def test_empty_frames_fail_shape_propagation(shape):
    """A frame with a zero dimension is refused before anything is planned or
    launched; the smallest frame, 1x1, propagates."""
    e = Engine(0).build(models.r8f64())
    with pytest.raises(EngineError, match="shape propagation failed"):
        e.output_shape(shape)
    assert e.output_shape((1, 1, 1, 1)) == (1, 1, 2, 2)


def test_channel_mismatch_fails_shape_propagation(fixtures):
    e = Engine(0).build(fixtures.get("conv_c4m8").model)
    with pytest.raises(EngineError):
        e.output_shape((1, 3, 16, 16))


def test_r8f64_fuses_to_18_convs():
    ops = ops_of(Engine(0).build(models.r8f64()))
    assert len(ops) == 18
    assert all(" Conv " in o for o in ops)
    assert sum("+relu" in o for o in ops) == 8
    assert ops[-1].startswith("op17 Conv 64->4") and "+dts2" in ops[-1]
    skips = [len(re.findall(r"\+skip", o)) for o in ops]
    assert skips == [0] + [0, 1] * 7 + [0, 2] + [0]  # dual residual on the last block


def test_shipped_model_fuses_to_27_convs():
    e = Engine(0).build(SHIPPED)
    ops = ops_of(e)
    assert len(ops) == 27
    assert sum("+silu" in o for o in ops) == 16
    assert "+dts2" in ops[-1] and "+clip[0,1]" in ops[-1]
    assert e.output_shape((1, 1, 1080, 1920)) == (1, 1, 2160, 3840)
    assert e.io_info() == (False, False, 1, 4)


def test_shared_intermediates_block_fusion(fixtures):
    ops = ops_of(Engine(0).build(fixtures.get("silu_shared").model))
    assert [o.split()[1] for o in ops] == ["Conv", "Sigmoid", "Mul", "Add"]
    ops = ops_of(Engine(0).build(fixtures.get("add_shared_conv_out").model))
    assert [o.split()[1] for o in ops] == ["Conv", "Conv", "Add", "Mul"]


@pytest.mark.parametrize("b", [1, 2, 3])
def test_depth_to_space_shapes(fixtures, b):
    e = Engine(0).build(fixtures.get(f"dts_b{b}").model)
    assert e.output_shape((1, 1, 16, 20)) == (1, 1, 16 * b, 20 * b)
    assert e.io_info()[:2] == (False, True)


def test_batch_and_multichannel_shapes(fixtures):
    e = Engine(0).build(fixtures.get("multi_in_out").model)
    assert e.output_shape((3, 3, 7, 9)) == (3, 2, 7, 9)
    e = Engine(0).build(models.r8f64())
    assert e.output_shape((2, 1, 2160, 3840)) == (2, 1, 4320, 7680)


def test_fp32_io_is_detected(fixtures):
    e = Engine(0).build(fixtures.get("identity_fp32io").model)
    assert e.io_info() == (True, True, 1, 1)
    e = Engine(0).build(models.r8f64(io_fp32=True))
    assert e.io_info()[:2] == (True, True)
    assert len(ops_of(e)) == 18


@pytest.mark.parametrize("builder", [models.c4f32, models.r8f64, models.shipped_like])
def test_fp32_model_fuses_like_fp16(builder):
    """The all-fp32 form of a model (what the reference's plugin converts with
    fp16=1) builds with fp32 IO and lowers to the same fused ops."""
    spec = builder(seed=0)
    wide = models.widen_to_fp32(spec)
    e16, e32 = Engine(0).build(spec), Engine(0).build(wide)
    assert e32.io_info()[:2] == (True, True)
    assert e16.io_info()[2:] == e32.io_info()[2:]
    ops = lambda d: [l.split(":")[0].split(" ", 1)[1] for l in d.splitlines() if l.startswith("op")]
    assert ops(e16.describe()) == ops(e32.describe())
