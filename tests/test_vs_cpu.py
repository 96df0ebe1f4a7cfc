"""The VapourSynth filter core (arthip_amd.vs over include/arthip.h's arthip_vs_*)
without a GPU.

Filter creation does no device work, so the reference's creation-time plugin
checks run here (tests/correctness/test_plugin.py): the accepted clip/model
pairs (90-103), subsampled clips (110-124), plane count against the model's
input channels (131-148), the fp16 default and the tiling arguments (P2-15,
362-416) and the flexible-output plane count (P2-16, 420-451). The shipped
chroma and dehalo models are the reference's own fixtures
(tests/fixtures/models/, copied into tests/golden/).

Also pins the load-time fp16 conversion: the oracle's rounding rule against
numpy's IEEE float16 cast and the rule's fixed points, the library's rule
against the oracle's, and the converted graph's structure.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest

from arthip_amd import _lib
from arthip_amd import onnx_proto as op
from arthip_amd import vs

GOLDEN = Path(__file__).resolve().parent / "golden"
SHIPPED = {
    "luma": GOLDEN / "ArtCNN_R8F64_fp16.onnx",
    "chroma": GOLDEN / "ArtCNN_R8F64_Chroma.onnx",
    "dehalo": GOLDEN / "ArtCNN_R8F64_YCbCr_DEHALO.onnx",
}


def make(fmt, model_key, *, width=64, height=64, **kw):
    return vs.Model(fmt, width, height, SHIPPED[model_key], **kw)


def expect_reject(match, fmt, model, *, width=64, height=64, **kw):
    with pytest.raises(vs.ModelError) as ei:
        vs.Model(fmt, width, height, model, **kw)
    msg = str(ei.value)
    assert msg.startswith("hip.Model: "), msg
    assert match in msg, msg
    return msg


# ---------------------------------------------------------------------------
# Accepted combinations and the output clip
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("fmt,key,flexible,out_fmt,planes,written", [
    ("GRAY8", "luma", False, "GRAYH", 1, 1),
    ("YUV444PS", "dehalo", False, "RGBS", 3, 3),
    ("RGBS", "dehalo", False, "RGBS", 3, 3),
    ("YUV444PS", "chroma", True, "GRAYS", 2, 2),
    ("YUV444PH", "dehalo", False, "RGBH", 3, 3),
    ("YUV444PS", "chroma", False, "GRAYS", 2, 1),
], ids=["gray8-luma", "yuv444ps-dehalo", "rgbs-dehalo", "yuv444ps-chroma-flex",
        "yuv444ph-dehalo", "yuv444ps-chroma"])
def test_clip_format_is_accepted(fmt, key, flexible, out_fmt, planes, written):
    m = make(fmt, key, flexible_output_prop="MlrtFlexible" if flexible else None)
    assert m.format.name == out_fmt
    assert (m.num_planes, m.planes_written, m.flexible) == (planes, written, flexible)
    scale = 2 if key == "luma" else 1
    assert (m.width, m.height) == (64 * scale, 64 * scale)


@pytest.mark.parametrize("key,fmt", [("dehalo", "YUV420P8"), ("dehalo", "YUV422P8"),
                                     ("chroma", "YUV420P8"), ("chroma", "YUV422P8")])
def test_subsampled_clip_is_rejected(key, fmt):
    expect_reject("subsampled", fmt, SHIPPED[key])


@pytest.mark.parametrize("key,fmt", [("dehalo", "GRAY8"), ("chroma", "GRAY8"),
                                     ("luma", "YUV444PS")])
def test_plane_count_mismatch_is_rejected(key, fmt):
    expect_reject("plane(s)", fmt, SHIPPED[key])


def test_more_channels_than_planes_is_rejected(fixtures):
    expect_reject("input channels", "YUV444PS", fixtures.get("conv_c4m4").model)


def test_format_checks():
    undefined = vs.VideoFormat("undefined", 0, vs.INTEGER, 8)
    expect_reject("expects a gray, YUV or RGB clip", undefined, SHIPPED["luma"])
    gray10 = vs.VideoFormat("GRAY10", vs.GRAY, vs.INTEGER, 10)
    expect_reject("expects 8/16-bit int or fp16/fp32 float input", gray10, SHIPPED["luma"])
    expect_reject("expects exactly 1 input clip", "GRAY8", SHIPPED["luma"], num_clips=2)


def test_loader_errors(tmp_path):
    missing = tmp_path / "missing.onnx"
    expect_reject(f"open {missing} failed", "GRAY8", missing)
    bad = tmp_path / "bad.onnx"
    bad.write_bytes(b"\x0a\xff\xff\xff\xff\xff")
    expect_reject(f"parse {bad} failed", "GRAY8", bad)
    expect_reject("parse onnx serialization failed", "GRAY8", b"\x0a\xff\xff\xff\xff\xff")


# ---------------------------------------------------------------------------
# P2-15: options and tiling; P2-16: flexible plane count
# ---------------------------------------------------------------------------

def test_fp16_default_is_true():
    omitted = make("GRAY8", "luma")
    explicit = make("GRAY8", "luma", fp16=1)
    assert omitted.format.name == explicit.format.name == "GRAYH"
    assert omitted.format.sample_type == vs.FLOAT
    assert (omitted.width, omitted.height) == (128, 128)
    assert make("GRAY8", "luma", fp16=0).format.name == "GRAY16"


def test_explicit_tiling_is_rejected():
    expect_reject("overlap", "GRAY8", SHIPPED["luma"], overlap=[1, 1])
    expect_reject("overlap", "GRAY8", SHIPPED["luma"], overlap=[0, 2])
    expect_reject("must be non-negative", "GRAY8", SHIPPED["luma"], overlap=[-1])
    expect_reject("tilesize", "GRAY8", SHIPPED["luma"], tilesize=[32, 32])
    # tilesize[1] defaults to tilesize[0]: a 64x48 clip is not one 64x64 tile
    expect_reject("tilesize", "GRAY8", SHIPPED["luma"], tilesize=[64], width=64, height=48)


def test_frame_sized_tiling_is_accepted():
    make("GRAY8", "luma", tilesize=[64, 64])
    make("GRAY8", "luma", tilesize=[64])
    make("GRAY8", "luma", overlap=[0])
    make("GRAY8", "luma", overlap=[0, 0], tilesize=[64, 48], height=48)


def test_flexible_plane_count_follows_the_final_output():
    m = make("GRAY8", "luma", fp16=1, flexible_output_prop="MlrtFlexible")
    assert m.num_planes == 1 and m.planes_written == 1


def test_num_streams():
    assert make("GRAY8", "luma").num_streams == 1
    assert make("GRAY8", "luma", num_streams=0).num_streams == 1
    assert make("GRAY8", "luma", num_streams=3).num_streams == 3


@pytest.mark.parametrize("fmt,fp16,in32,out32,out_fmt", [
    ("GRAY8", 1, False, False, "GRAYH"),     # converted: fp16 IO
    ("GRAYH", 1, False, False, "GRAYH"),
    ("GRAYS", 1, True, True, "GRAYS"),       # fp32 clip keeps fp32 IO behind Casts
    ("GRAY8", 0, True, True, "GRAYS"),       # native fp32 IO (P2-12's setting)
    ("GRAYS", 0, True, True, "GRAYS"),
])
def test_fp32_model_io_follows_the_clip(fixtures, fmt, fp16, in32, out32, out_fmt):
    m = vs.Model(fmt, 16, 16, fixtures.get("identity_fp32io").model, fp16=fp16)
    assert (m.in_fp32, m.out_fp32, m.format.name) == (in32, out32, out_fmt)


def test_fp16_model_with_fp32_clip_and_integer_output():
    # An fp16-IO model stays fp16 whatever the clip; fp16=0 makes the output GRAY16.
    m = vs.Model("GRAYS", 64, 64, SHIPPED["luma"], fp16=0)
    assert (m.in_fp32, m.out_fp32, m.format.name) == (False, False, "GRAY16")


def test_version_and_device_properties():
    version, count = vs.Model.version()
    assert version.startswith("arthip")
    assert isinstance(count, int)


# ---------------------------------------------------------------------------
# The load-time conversion's rounding and graph
# ---------------------------------------------------------------------------

def _bits(h) -> np.ndarray:
    return np.asarray(h, dtype=np.float16).view(np.uint16)


def test_oracle_half_no_subnormals_fixed_points():
    from oracle.convert import half_no_subnormals as h
    min_normal = np.float32(2.0 ** -14)
    cases = [
        (float(min_normal), 0x0400),
        (float(np.nextafter(min_normal, np.float32(0))), 0x0000),   # would round up in IEEE
        (float(-np.nextafter(min_normal, np.float32(0))), 0x8000),
        (2.0 ** -20, 0x0000),                                        # IEEE: subnormal 0x0010
        (65504.0, 0x7BFF),
        (65519.99, 0x7BFF),
        (65520.0, 0x7C00),                                           # tie -> even -> overflow
        (1e30, 0x7C00), (-1e30, 0xFC00),
        (float("inf"), 0x7C00), (float("-inf"), 0xFC00),
        (1.0 + 2.0 ** -11, 0x3C00),                                  # tie, even below
        (1.0 + 3 * 2.0 ** -11, 0x3C02),                              # tie, even above
        (0.0, 0x0000), (-0.0, 0x8000),
    ]
    for x, want in cases:
        got = int(_bits(h(np.float32(x))))
        assert got == want, (x, hex(got), hex(want))
    nan = np.array([np.nan, -np.nan], dtype=np.float32)
    nan[1] = np.float32(-np.nan)
    assert list(_bits(h(nan))) == [0x7C00, 0xFC00]


def test_oracle_half_no_subnormals_matches_ieee_in_the_normal_range():
    from oracle.convert import half_no_subnormals as h
    rng = np.random.default_rng(5)
    x = rng.standard_normal(200_000).astype(np.float32) * np.float32(
        2.0) ** rng.integers(-13, 15, 200_000).astype(np.float32)
    x = x[np.abs(x) >= 2.0 ** -14]
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(_bits(h(x)), _bits(x.astype(np.float16)))


def test_library_rounding_matches_the_oracle():
    from oracle.convert import half_no_subnormals as h
    lib = _lib.lib()
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 20_000, dtype=np.uint64).astype(np.uint32)
    special = np.array([0x38800000, 0x387FFFFF, 0xB87FFFFF, 0x477FE000, 0x477FEFFF, 0x477FF000,
                        0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x00000001, 0x33000000,
                        0x3F801000, 0x3F803000, 0x80000000], dtype=np.uint32)
    xs = np.concatenate([bits, special]).view(np.float32)
    want = _bits(h(xs))
    got = np.array([lib.arthip_f32_to_f16_no_subnormals(ctypes.c_float(float(x)))
                    for x in xs], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


def test_converted_graph_structure():
    from oracle.convert import to_fp16
    m = op.load(SHIPPED["chroma"])
    kept = to_fp16(m, cast_input=True, cast_output=True)
    g = kept.graph
    assert g.inputs[0].elem_type == op.FLOAT and g.outputs[0].elem_type == op.FLOAT
    assert g.nodes[0].op_type == "Cast" and g.nodes[0].outputs == ["graph_input_cast_0"]
    assert g.nodes[-1].op_type == "Cast" and g.nodes[-1].inputs == ["graph_output_cast_0"]
    assert all(t.data_type == op.FLOAT16 for t in g.initializers)
    assert not any(g.inputs[0].name in n.inputs for n in g.nodes[1:])
    plain = to_fp16(m, cast_input=False, cast_output=False)
    assert plain.graph.inputs[0].elem_type == op.FLOAT16
    assert plain.graph.outputs[0].elem_type == op.FLOAT16
    assert len(plain.graph.nodes) == len(m.graph.nodes)


def test_converted_model_builds_like_the_conversion_option():
    """The engine's load-time conversion and an engine built from the oracle's
    converted model agree on the boundary types."""
    from oracle.convert import to_fp16
    m = op.load(SHIPPED["chroma"])
    conv = op.encode_model(to_fp16(m, cast_input=True, cast_output=True))
    a = vs.Model("YUV444PS", 32, 32, SHIPPED["chroma"], fp16=1)
    b = vs.Model("YUV444PS", 32, 32, conv, fp16=0)
    assert (a.in_fp32, a.out_fp32, a.format) == (b.in_fp32, b.out_fp32, b.format)


# ---------------------------------------------------------------------------
# Frame-time refusals (validated before any device work)
# ---------------------------------------------------------------------------

def _frame_call(m, planes, fmt=None, n_dst=None, null_dst=False, out_stride=None):
    """Calls arthip_vs_model_get_frame directly with hand-made arguments."""
    lib = _lib.lib()
    fmt = m.clip_format if fmt is None else vs.FORMATS[fmt]
    n = len(planes)
    pw = (ctypes.c_int * n)(*[p.shape[1] for p in planes])
    ph = (ctypes.c_int * n)(*[p.shape[0] for p in planes])
    sp = (ctypes.c_void_p * n)(*[p.ctypes.data for p in planes])
    ss = (ctypes.c_ssize_t * n)(*[p.strides[0] for p in planes])
    k = m.planes_written if n_dst is None else n_dst
    out = np.zeros((planes[0].shape[0] * m.scale_h, planes[0].shape[1] * m.scale_w),
                   m.format.dtype)
    dp = (ctypes.c_void_p * max(k, 1))(*([None if null_dst else out.ctypes.data] * k))
    stride = out.strides[0] if out_stride is None else out_stride
    ds = (ctypes.c_ssize_t * max(k, 1))(*([stride] * k))
    err = ctypes.create_string_buffer(512)
    rc = lib.arthip_vs_model_get_frame(m._h, ctypes.byref(fmt._c()), pw, ph, sp, ss, dp, ds, k,
                                       err, len(err))
    return rc, err.value.decode()


def test_frame_refusals_before_device_work():
    with make("GRAYH", "luma", width=32, height=32) as m:
        x = np.zeros((32, 32), np.float16)
        rc, msg = _frame_call(m, [x, x, x], fmt="YUV444PH")
        assert rc == 2 and "plane count does not match" in msg
        rc, msg = _frame_call(m, [x], n_dst=0)
        assert rc == 2 and "destination plane" in msg
        rc, msg = _frame_call(m, [x], null_dst=True)
        assert rc == 2 and "null destination" in msg
        short = np.zeros((32, 8), np.float16)
        lib = _lib.lib()
        # A source stride shorter than a row.
        pw = (ctypes.c_int * 1)(32)
        ph = (ctypes.c_int * 1)(32)
        sp = (ctypes.c_void_p * 1)(short.ctypes.data)
        ss = (ctypes.c_ssize_t * 1)(16)
        out = np.zeros((64, 64), np.float16)
        dp = (ctypes.c_void_p * 1)(out.ctypes.data)
        ds = (ctypes.c_ssize_t * 1)(out.strides[0])
        err = ctypes.create_string_buffer(512)
        rc = lib.arthip_vs_model_get_frame(m._h, ctypes.byref(vs.FORMATS["GRAYH"]._c()), pw, ph,
                                           sp, ss, dp, ds, 1, err, len(err))
        assert rc == 2 and "stride shorter than a row" in err.value.decode()
    with make("YUV444PS", "chroma", width=32, height=32) as m:
        a = np.zeros((32, 32), np.float32)
        b = np.zeros((16, 16), np.float32)
        rc, msg = _frame_call(m, [a, b, b])
        assert rc == 2 and "subsampled input frame" in msg
        gray10 = vs.VideoFormat("YUV444P10", vs.YUV, vs.INTEGER, 10)
        lib = _lib.lib()
        pw = (ctypes.c_int * 3)(32, 32, 32)
        ph = (ctypes.c_int * 3)(32, 32, 32)
        sp = (ctypes.c_void_p * 3)(a.ctypes.data, a.ctypes.data, a.ctypes.data)
        ss = (ctypes.c_ssize_t * 3)(128, 128, 128)
        out = np.zeros((32, 32), np.float32)
        dp = (ctypes.c_void_p * 1)(out.ctypes.data)
        ds = (ctypes.c_ssize_t * 1)(128)
        err = ctypes.create_string_buffer(512)
        rc = lib.arthip_vs_model_get_frame(m._h, ctypes.byref(gray10._c()), pw, ph, sp, ss, dp,
                                           ds, 1, err, len(err))
        assert rc == 2 and "8/16-bit int or fp16/fp32" in err.value.decode()


def test_null_arguments_are_refused():
    lib = _lib.lib()
    err = ctypes.create_string_buffer(256)
    out = ctypes.c_void_p()
    rc = lib.arthip_vs_model_create(None, 1, None, 64, 64, ctypes.byref(out), None, err, 256)
    assert rc == 1 and "null argument" in err.value.decode() and not out.value
    rc = lib.arthip_vs_model_get_frame(None, None, None, None, None, None, None, None, 0, err, 256)
    assert rc == 2 and "null model" in err.value.decode()
