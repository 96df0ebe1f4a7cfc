"""The VapourSynth filter core on the GPU: frames through arthip_vs_model_get_frame.

Mirrors the frame-level checks of the reference's plugin tests
(tests/correctness/test_plugin.py): the chroma model's flexible output planes
against an fp32 CPU run within CHROMA_TOL (153-244), fp16 multi-channel clips
coming back plane-major (P2-11, 250-331), an integer clip reaching an
fp32-input model as value / 255 (P2-12, 337-386). The oracle (oracle/) stands
in for ONNX Runtime's CPU EP, which is not installed. On top:
- sample packing and unpacking bit for bit: every 8-bit and 16-bit sample
  value through an identity model, fp32 clips, the integer output rule, strided
  planes in and out;
- the load-time fp16 conversion bit for bit against an engine built from the
  oracle's converted model;
- the engine pool: frames from several threads equal the one-stream results,
  and a variable-size clip;
- VSHIP_PROFILE=1 spans (P2-18, 483-512).
"""

from __future__ import annotations

import threading
from pathlib import Path

import numpy as np
import pytest

from arthip_amd import onnx_proto as op
from arthip_amd import vs

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
LUMA = GOLDEN / "ArtCNN_R8F64_fp16.onnx"
CHROMA = GOLDEN / "ArtCNN_R8F64_Chroma.onnx"
DEHALO = GOLDEN / "ArtCNN_R8F64_YCbCr_DEHALO.onnx"
CHROMA_TOL = 0.02  # the reference's tolerance against an fp32 CPU run


def identity_model(dtype: int) -> bytes:
    """1 -> 1 conv with a centre tap of 1: y = x exactly, in fp16 storage."""
    w = np.zeros((1, 1, 3, 3), np.float32)
    w[0, 0, 1, 1] = 1.0
    t = op.tensor("w", w.astype(np.float16 if dtype == op.FLOAT16 else np.float32))
    g = op.Graph(nodes=[op.node("Conv", ["x", "w"], ["y"], kernel_shape=[3, 3],
                                pads=[1, 1, 1, 1])],
                 initializers=[t],
                 inputs=[op.value_info("x", dtype, [1, 1, "h", "w"])],
                 outputs=[op.value_info("y", dtype, [1, 1, "h", "w"])])
    return op.encode_model(op.Model(graph=g))


def f16_bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16).view(np.uint16)


# ---------------------------------------------------------------------------
# Packing and unpacking, bit for bit
# ---------------------------------------------------------------------------

def test_gray8_every_value_packs_like_the_host_rule():
    x = np.arange(256, dtype=np.uint8).reshape(16, 16)
    with vs.Model("GRAY8", 16, 16, identity_model(op.FLOAT16)) as m:
        assert m.format.name == "GRAYH"
        (y,) = m.get_frame([x])
    want = (x.astype(np.float32) * np.float32(1.0 / 255.0)).astype(np.float16)
    np.testing.assert_array_equal(f16_bits(y), f16_bits(want))


def test_gray16_every_value_packs_like_the_host_rule():
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(256, 256)
    with vs.Model("GRAY16", 256, 256, identity_model(op.FLOAT16)) as m:
        (y,) = m.get_frame([x])
    want = (x.astype(np.float32) * np.float32(1.0 / 65535.0)).astype(np.float16)
    np.testing.assert_array_equal(f16_bits(y), f16_bits(want))


def test_integer_output_rule():
    """fp16=0 on an fp16 model: GRAY16 out, trunc(v * 65535 + 0.5) in fp32."""
    bits = np.arange(0, 0x3C01, dtype=np.uint16)  # every half in [0, 1]
    n = bits.size
    w = 128
    h = (n + w - 1) // w
    x = np.zeros(h * w, np.uint16)
    x[:n] = bits
    xh = x.view(np.float16).reshape(h, w)
    with vs.Model("GRAYH", w, h, identity_model(op.FLOAT16), fp16=0) as m:
        assert m.format.name == "GRAY16"
        (y,) = m.get_frame([xh])
    v = xh.astype(np.float32)
    want = np.floor((v * np.float32(65535.0)) + np.float32(0.5)).astype(np.uint16)
    np.testing.assert_array_equal(y, want)


@pytest.mark.parametrize("fmt,fp16", [("GRAYS", 1), ("GRAYS", 0), ("GRAYH", 0), ("GRAY8", 0)])
def test_fp32_io_model(fixtures, fmt, fp16):
    """fp32-IO identity: output = fp32(fp16(packed input)); an 8-bit 128 is 128/255
    (P2-12: the packed element type must follow the engine's input)."""
    rng = np.random.default_rng(3)
    f = vs.FORMATS[fmt]
    if f.sample_type == vs.INTEGER:
        x = np.full((16, 16), 128, np.uint8)
        packed = np.float32(128) * np.float32(1.0 / 255.0)
        want = np.full((16, 16), packed, np.float32)
    else:
        x = rng.uniform(0, 1, (16, 16)).astype(f.dtype)
        want = x.astype(np.float32)
    with vs.Model(fmt, 16, 16, fixtures.get("identity_fp32io").model, fp16=fp16) as m:
        (y,) = m.get_frame([x])
    assert y.dtype == np.float32
    np.testing.assert_array_equal(y, want.astype(np.float16).astype(np.float32))
    if fmt == "GRAY8":
        assert abs(float(y[8, 8]) - 128.0 / 255.0) < 1e-3


def test_strided_planes_in_and_out():
    rng = np.random.default_rng(4)
    wide = rng.integers(0, 256, (40, 80), dtype=np.uint8)
    x = wide[:, 5:5 + 61]  # 61 columns inside 80-sample rows
    with vs.Model("GRAY8", 61, 40, LUMA) as m:
        (a,) = m.get_frame([x])
        (b,) = m.get_frame([np.ascontiguousarray(x)], out_row_pad=7)
    assert b.strides[0] == (122 + 7) * 2
    np.testing.assert_array_equal(f16_bits(a), f16_bits(b))


# ---------------------------------------------------------------------------
# Shipped models against the oracle
# ---------------------------------------------------------------------------

def test_luma_frame_equals_the_engine():
    from arthip_amd.engine import Engine
    d = np.load(GOLDEN / "shipped_luma_48x64.npz")
    x = d["x"]
    with vs.Model("GRAYH", 64, 48, LUMA) as m:
        (y,) = m.get_frame([x[0, 0]])
    with Engine(0) as e:
        ref = e.build(op.load(LUMA)).run(x)[0, 0]
    np.testing.assert_array_equal(f16_bits(y), f16_bits(ref))
    assert np.abs(y.astype(np.float64) - d["y"][0, 0]).max() <= 2e-2


def _oracle(model_path, x32, *, cast_io: bool):
    from oracle.convert import to_fp16
    from oracle.model import run_model
    m = op.load(model_path)
    conv = to_fp16(m, cast_input=cast_io, cast_output=cast_io)
    xin = x32 if cast_io else x32.astype(np.float16)
    return run_model(conv, xin[None]), run_model(m, x32[None], round_fp16=False)


def test_chroma_flexible_planes_match_the_cpu_reference():
    rng = np.random.RandomState(1234)
    data = rng.uniform(0.0, 1.0, (3, 64, 64)).astype(np.float32)
    with vs.Model("YUV444PS", 64, 64, CHROMA, fp16=1, flexible_output_prop="MlrtFlexible") as m:
        assert (m.num_planes, m.planes_written, m.format.name) == (2, 2, "GRAYS")
        planes = m.get_frame(list(data))
    y16, y32 = _oracle(CHROMA, data, cast_io=True)
    for c in range(2):
        p = planes[c].astype(np.float64)
        assert np.isfinite(p).all()
        assert np.abs(p - y32[0, c]).max() < CHROMA_TOL
        assert np.abs(p - y16[0, c]).max() <= 1e-2
    assert planes[0].mean() != pytest.approx(planes[1].mean(), abs=1e-6)


@pytest.mark.parametrize("fmt", ["YUV444PH", "RGBH"])
def test_fp16_multichannel_planes_are_planar(fmt):
    rng = np.random.RandomState(4242)
    data = rng.uniform(0.0, 1.0, (3, 64, 64)).astype(np.float32)
    planes_in = [np.ascontiguousarray(data[p], dtype=np.float16) for p in range(3)]
    with vs.Model(fmt, 64, 64, DEHALO, fp16=1) as m:
        assert m.format.name == "RGBH" and m.planes_written == 3
        out = m.get_frame(planes_in)
    y16, y32 = _oracle(DEHALO, np.stack([p.astype(np.float32) for p in planes_in]), cast_io=False)
    for p in range(3):
        o = out[p].astype(np.float64)
        assert np.isfinite(o).all()
        assert np.abs(o - y32[0, p]).max() < CHROMA_TOL
        assert np.abs(o - y16[0, p]).max() <= 1e-2


def test_load_time_conversion_is_the_oracles_conversion():
    """fp16=1 on the fp32 chroma model gives the same bits as an engine built
    from the oracle's converted model (fp16 initializers, fp32 IO behind Casts)."""
    from oracle.convert import to_fp16
    rng = np.random.default_rng(9)
    data = rng.uniform(0.0, 1.0, (3, 40, 56)).astype(np.float32)
    conv = op.encode_model(to_fp16(op.load(CHROMA), cast_input=True, cast_output=True))
    with vs.Model("YUV444PS", 56, 40, CHROMA, fp16=1, flexible_output_prop="p") as a, \
            vs.Model("YUV444PS", 56, 40, conv, fp16=0, flexible_output_prop="p") as b:
        pa = a.get_frame(list(data))
        pb = b.get_frame(list(data))
    for u, v in zip(pa, pb):
        np.testing.assert_array_equal(u, v)


# ---------------------------------------------------------------------------
# Pool and frame-time checks
# ---------------------------------------------------------------------------

def test_pool_threads_match_one_stream():
    rng = np.random.default_rng(11)
    frames = [rng.uniform(0, 1, (72, 96)).astype(np.float16) for _ in range(12)]
    with vs.Model("GRAYH", 96, 72, LUMA, num_streams=1) as one:
        want = [one.get_frame([f])[0] for f in frames]
    got = [None] * len(frames)
    errors = []
    with vs.Model("GRAYH", 96, 72, LUMA, num_streams=3) as pool:
        def work(k):
            try:
                for i in range(k, len(frames), 4):
                    got[i] = pool.get_frame([frames[i]])[0]
            except Exception as e:  # reported below
                errors.append(e)
        threads = [threading.Thread(target=work, args=(k,)) for k in range(4)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
    assert not errors, errors
    for a, b in zip(got, want):
        np.testing.assert_array_equal(f16_bits(a), f16_bits(b))


def test_one_engine_threads_with_changing_frame_sizes():
    """One engine, two frames in flight, the frame shape changing between them:
    the engine re-plans only after the other frame's work has drained."""
    from arthip_amd.engine import Engine
    rng = np.random.default_rng(13)
    sizes = [(24, 40), (33, 18), (24, 40), (8, 8), (40, 64), (33, 18)]
    frames = [rng.uniform(0, 1, sizes[i % len(sizes)]).astype(np.float16) for i in range(24)]
    with Engine(0) as e:
        e.build(op.load(LUMA))
        want = [e.run(f[None, None])[0, 0] for f in frames]
    got = [None] * len(frames)
    errors = []
    with vs.Model("GRAYH", 0, 0, LUMA, num_streams=1) as m:
        def work(k):
            try:
                for i in range(k, len(frames), 4):
                    got[i] = m.get_frame([frames[i]])[0]
            except Exception as ex:  # reported below
                errors.append(ex)
        threads = [threading.Thread(target=work, args=(k,)) for k in range(4)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
    assert not errors, errors
    for a, b in zip(got, want):
        np.testing.assert_array_equal(f16_bits(a), f16_bits(b))


def test_variable_size_clip():
    from arthip_amd.engine import Engine
    rng = np.random.default_rng(12)
    with vs.Model("GRAYH", 0, 0, LUMA) as m, Engine(0) as e:
        e.build(op.load(LUMA))
        for h, w in ((24, 40), (33, 18), (24, 40)):
            x = rng.uniform(0, 1, (h, w)).astype(np.float16)
            (y,) = m.get_frame([x])
            assert y.shape == (2 * h, 2 * w)
            ref = e.run(x[None, None])[0, 0]
            np.testing.assert_array_equal(f16_bits(y), f16_bits(ref))


def test_frame_time_refusals():
    with vs.Model("GRAYH", 32, 32, LUMA) as m:
        x = np.zeros((32, 32), np.float16)
        with pytest.raises(vs.ModelError, match="plane count does not match"):
            m.get_frame([x, x, x], fmt="YUV444PH")
    with vs.Model("YUV444PS", 32, 32, CHROMA) as m:
        a = np.zeros((32, 32), np.float32)
        b = np.zeros((16, 16), np.float32)
        with pytest.raises(vs.ModelError, match="subsampled input frame"):
            m.get_frame([a, b, b])


def test_profiling_reports_ops_and_a_separate_transfer(capfd, monkeypatch):
    """VSHIP_PROFILE=1 (test_plugin.py P2-18): per-op GPU spans and the output
    conversion + download as its own span, not folded into the last op."""
    monkeypatch.setenv("VSHIP_PROFILE", "1")
    x = np.random.default_rng(13).uniform(0, 1, (48, 64)).astype(np.float16)
    with vs.Model("GRAYH", 64, 48, LUMA, fp16=0) as m:  # GRAY16 out: a conversion kernel too
        for _ in range(2):
            m.get_frame([x])
    err = capfd.readouterr().err
    assert "[vship-prof]" in err, err
    assert "output-convert+download" in err, err
    ops = [ln for ln in err.splitlines() if ln.startswith("[vship-prof] op")]
    # Both frames, every launch of the shipped model: 27 convs, of which each
    # block's second SiLU conv and its residual conv run as one fused launch.
    assert len(ops) >= 2 * 19, err
    for ln in ops:
        ms = float(ln.split()[-2])
        assert 0.0 <= ms < 1000.0, ln
