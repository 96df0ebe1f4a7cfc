"""End-to-end parity of the benchmark model family on the GPU vs the graph oracle.

The oracle (oracle/model.py) evaluates the same ONNX model node by node in fp32
with fp16 tensors between nodes -- ONNX Runtime CPU EP semantics for an fp16
model. Whether ONNX Runtime keeps fp32 between nodes instead is not pinned
(no ONNX Runtime here), so the literal gates are checked against both oracle
modes: fp16 storage per node and fp32 throughout.

Gates:
- max-abs <= 2e-2 and PSNR >= 50 dB (peak 1) where the configuration's output
  range allows it (C4F32, the single layer, the shipped luma model); the
  shipped model is also held to max-abs <= 1.34e-3, the reference's accuracy
  against ONNX Runtime CPU at 1920x1080 (NOTES.md:78-79), with at most four of
  the 1920x1080 frame's 8.3 M samples one fp16 ulp past it;
- for the deep He-normal models the fp16-storage floor of the model itself is
  far above that (outputs span ~+-200), so those are gated on relative RMS
  error <= 3x the floor measured in the same test (the engine measures ~2x).
"""

from __future__ import annotations

import numpy as np
import pytest

from arthip_amd import models
from arthip_amd.engine import Engine
from oracle.model import run_model
from tests import reference_math as ref

pytestmark = pytest.mark.gpu


#: Deep models: engine relative RMS error against the oracle, as a multiple of
#: the model's own fp16-storage floor (oracle fp16 storage vs fp32 throughout).
FLOOR_RATIO = 3.0


def _compare(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = got - want
    rms = float(np.sqrt(np.mean(want ** 2))) + 1e-30
    return {"max_abs": float(np.abs(err).max()), "psnr": ref.psnr(got, want, 1.0),
            "rel_rms": float(np.sqrt(np.mean(err ** 2))) / rms}


def _literal_gate(got, model, x, label, max_abs=2e-2):
    """max-abs and PSNR (peak 1) against the oracle in both modes."""
    for mode in (True, False):
        want = run_model(model, x, round_fp16=mode)
        s = _compare(got, want)
        print(label, "fp16 storage" if mode else "fp32 throughout", s)
        assert s["max_abs"] <= max_abs and s["psnr"] >= 50.0, (mode, s)


def test_c4f32_full_size_meets_gate():
    spec = models.c4f32(seed=0)
    x = models.synthetic_input((1, 1, 540, 960), seed=1)
    with Engine(0) as e:
        got = e.build(spec).run(x).astype(np.float32)
    assert got.shape == (1, 1, 1080, 1920)
    _literal_gate(got, spec.model, x, "c4f32 540x960")


def test_single_layer_meets_gate():
    spec = models.single64(seed=0)
    x = models.synthetic_input((1, 64, 270, 480), seed=1, kind="normal")
    with Engine(0) as e:
        got = e.build(spec).run(x).astype(np.float32)
    _literal_gate(got, spec.model, x, "single64 270x480")


def test_single_layer_full_size():
    """The single-layer config at its stated size, 1x64x1080x1920 N(0, 0.5): the
    whole frame against the oracle in both modes (one conv, so the oracle is
    cheap enough for the full frame)."""
    spec = models.single64(seed=0)
    x = models.synthetic_input((1, 64, 1080, 1920), seed=1, kind="normal")
    with Engine(0) as e:
        got = e.build(spec).run(x).astype(np.float32)
    assert got.shape == (1, 64, 1080, 1920) and np.isfinite(got).all()
    _literal_gate(got, spec.model, x, "single64 1080x1920")


@pytest.mark.parametrize("builder,hw", [(models.r8f64, (48, 80)), (models.shipped_like, (40, 72)),
                                        (models.r16f96, (32, 48))])
def test_deep_models_within_fp16_floor(builder, hw):
    spec = builder(seed=0)
    x = models.synthetic_input((1, 1) + hw, seed=1)
    with Engine(0) as e:
        got = e.build(spec).run(x).astype(np.float32)
    want = run_model(spec.model, x)  # fp16 tensors between nodes
    exact = run_model(spec.model, x, round_fp16=False)  # fp32 throughout
    s = _compare(got, want)
    floor = _compare(want, exact)
    print(spec.name, "engine vs oracle", s, "| oracle fp16 vs fp32 floor", floor,
          "| ratio", s["rel_rms"] / floor["rel_rms"])
    assert np.isfinite(got).all()
    assert s["rel_rms"] <= max(FLOOR_RATIO * floor["rel_rms"], 2e-3), (s, floor)


def test_r8f64_batch_two():
    spec = models.r8f64(seed=0)
    x = models.synthetic_input((2, 1, 36, 52), seed=3)
    with Engine(0) as e:
        e.build(spec)
        both = e.run(x)
        one = e.run(np.ascontiguousarray(x[1:2]))
    np.testing.assert_array_equal(both[1:2], one)


def test_fresh_engines_bit_identical():
    """Fresh engines on the same input must agree bit for bit (the reference
    allows 1e-4, test_engine.py:288-326; nothing here is order-dependent)."""
    spec = models.r8f64(seed=0)
    x = models.synthetic_input((1, 1, 270, 480), seed=2)
    first = None
    for _ in range(4):
        with Engine(0) as e:
            out = e.build(spec).run(x)
        if first is None:
            first = out
        else:
            np.testing.assert_array_equal(out, first)


def _window_oracle(model, x, r0, r1, c0, c1, margin, scale, round_fp16=True):
    """Oracle output for input rows [r0, r1) and columns [c0, c1), run on the window
    grown by `margin` pixels (at least one per 3x3 conv) and clipped to the image,
    so the kept outputs never see the window's artificial edges."""
    H, W = x.shape[2:]
    a0, a1 = max(r0 - margin, 0), min(r1 + margin, H)
    b0, b1 = max(c0 - margin, 0), min(c1 + margin, W)
    win = np.ascontiguousarray(x[:, :, a0:a1, b0:b1])
    y = run_model(model, win, round_fp16=round_fp16)
    return y[:, :, (r0 - a0) * scale:(r1 - a0) * scale, (c0 - b0) * scale:(c1 - b0) * scale]


def _band_check(got_full, spec, x, r0, r1, margin, c0=0, c1=None):
    """Engine full-frame output for input rows [r0, r1) (and columns [c0, c1))
    against the oracle on that window; returns (engine vs oracle, oracle floor)."""
    c1 = x.shape[3] if c1 is None else c1
    s = spec.scale
    want = _window_oracle(spec.model, x, r0, r1, c0, c1, margin, s)
    exact = _window_oracle(spec.model, x, r0, r1, c0, c1, margin, s, round_fp16=False)
    got = got_full[:, :, r0 * s:r1 * s, c0 * s:c1 * s]
    return _compare(got, want), _compare(want, exact)


#: Full-frame oracle outputs, computed once per (workload, mode) and shared by
#: the tests of both modes (each full 1080p oracle run takes tens of seconds).
_ORACLE_FULL: dict = {}
_GPU_FULL: dict = {}


def _oracle_full(key, model, x, round_fp16):
    k = (key, round_fp16)
    if k not in _ORACLE_FULL:
        _ORACLE_FULL[k] = run_model(model, x, round_fp16=round_fp16).astype(np.float32)
    return _ORACLE_FULL[k]


def _r8f64_1080p():
    """R8F64 on one 1920x1080 frame through the engine, twice (bit-stability)."""
    if not _GPU_FULL.get("r8f64"):
        spec = models.r8f64(seed=0)
        x = models.synthetic_input((1, 1, 1080, 1920), seed=1)
        with Engine(0) as e:
            got = e.build(spec).run(x)
            again = e.run(x)
        _GPU_FULL["r8f64"] = (spec, x, got, again)
    return _GPU_FULL["r8f64"]


#: R8F64 at 1080p, whole frame: largest per-element error against the oracle
#: (outputs up to ~370 in magnitude). The engine measures 0.81 against the
#: fp16-storage oracle and 0.68 against fp32 throughout (the two oracle modes
#: differ by up to 0.46); the bounds sit 1.5x above. A wrong tile, strip edge or
#: run boundary gives errors of the order of the outputs themselves.
R8F64_FULL_MAX_ABS = {True: 1.25, False: 1.05}


@pytest.mark.parametrize("round_fp16", [True, False], ids=["fp16_storage", "fp32_throughout"])
def test_r8f64_full_1080p_every_pixel(round_fp16):
    """Full-size frame on the GPU, every output pixel against the oracle in the
    given mode: relative RMS within 3x the model's fp16-storage floor (the
    oracle in one mode against the other, over the whole frame) and a
    per-element max-abs bound."""
    spec, x, got, again = _r8f64_1080p()
    assert got.shape == (1, 1, 2160, 3840)
    np.testing.assert_array_equal(got.view(np.uint16), again.view(np.uint16))
    got = got.astype(np.float32)
    assert np.isfinite(got).all()
    want = _oracle_full("r8f64", spec.model, x, round_fp16)
    floor = _compare(_oracle_full("r8f64", spec.model, x, True),
                     _oracle_full("r8f64", spec.model, x, False))
    s = _compare(got, want)
    err = np.abs(got.astype(np.float64) - want)
    # Error per 60x64-pixel output block (one 30-pixel strip x 16 tile rows of
    # the input): a defect confined to one workgroup's run shows up here.
    blocks = err[0, 0, :2160 // 64 * 64, :3840 // 60 * 60].reshape(2160 // 64, 64, 3840 // 60, 60)
    block_rms = np.sqrt((blocks ** 2).mean(axis=(1, 3)))
    print("r8f64 1080p full frame", "fp16 storage" if round_fp16 else "fp32 throughout", s,
          "floor", floor, "ratio %.3f" % (s["rel_rms"] / floor["rel_rms"]),
          "block RMS max %.4f median %.4f" % (block_rms.max(), np.median(block_rms)))
    assert s["rel_rms"] <= FLOOR_RATIO * floor["rel_rms"], (s, floor)
    assert s["max_abs"] <= R8F64_FULL_MAX_ABS[round_fp16], s


def test_r16f96_full_1080p_window_parity():
    """R16F96 at full 1920x1080 (intermediates near 2e4, where fp16 overflow would
    show first): finite everywhere, bit-stable across runs, and three windows (two
    image corners and the middle) against the oracle with a 34-pixel margin (the
    receptive field of 34 convs)."""
    spec = models.r16f96(seed=0)
    x = models.synthetic_input((1, 1, 1080, 1920), seed=1)
    with Engine(0) as e:
        got = e.build(spec).run(x)
        again = e.run(x)
    assert got.shape == (1, 1, 2160, 3840) and np.isfinite(got).all()
    np.testing.assert_array_equal(got.view(np.uint16), again.view(np.uint16))
    got = got.astype(np.float32)
    print("r16f96 1080p output range", float(got.min()), float(got.max()))
    for r0, r1, c0, c1 in ((0, 24, 0, 96), (528, 552, 928, 1024), (1056, 1080, 1824, 1920)):
        s, floor = _band_check(got, spec, x, r0, r1, 34, c0, c1)
        print("r16f96 1080p window", (r0, r1, c0, c1), s, "floor", floor,
              "ratio", s["rel_rms"] / floor["rel_rms"])
        assert s["rel_rms"] <= max(FLOOR_RATIO * floor["rel_rms"], 2e-3), (s, floor)


def test_r8f64_4k_batch2_full_size():
    """R8F64 on a batch of two 3840x2160 frames at full size: finite, each image equal to its own
    single-image run, and band parity against the oracle."""
    spec = models.r8f64(seed=0)
    x = models.synthetic_input((2, 1, 2160, 3840), seed=5)
    with Engine(0) as e:
        e.build(spec)
        got = e.run(x)
        one = e.run(np.ascontiguousarray(x[1:2]))
    assert got.shape == (2, 1, 4320, 7680) and np.isfinite(got).all()
    np.testing.assert_array_equal(got[1:2], one)
    s, floor = _band_check(got[1:2].astype(np.float32), spec, x[1:2], 1000, 1016, 18)
    print("r8f64 4k band", s, "floor", floor)
    assert s["rel_rms"] <= max(FLOOR_RATIO * floor["rel_rms"], 2e-3), (s, floor)


def _gray8(name):
    """The reference's test image as its accuracy tool feeds it
    (tests/tools/multires.py:84-92: cv2.imread(..., IMREAD_GRAYSCALE) / 255 as
    fp16 NCHW): 8-bit BT.601 gray with OpenCV's fixed-point rounding,
    (4899 R + 9617 G + 1868 B + 2^13) >> 14."""
    from pathlib import Path

    from PIL import Image
    here = Path(__file__).resolve().parent / "golden"
    rgb = np.asarray(Image.open(here / name).convert("RGB")).astype(np.int64)
    g = (4899 * rgb[..., 0] + 9617 * rgb[..., 1] + 1868 * rgb[..., 2] + 8192) >> 14
    x = np.clip(g.astype(np.float32) / 255.0, 0.0, 1.0)
    return x[None, None].astype(np.float16)


def _shipped_model():
    from pathlib import Path

    from arthip_amd import onnx_proto as op
    return op.load(Path(__file__).resolve().parent / "golden" / "ArtCNN_R8F64_fp16.onnx")


#: The shipped model against the oracle, held to the reference's own accuracy
#: against ONNX Runtime CPU at 1920x1080 (0.00134; 0.00098 at 256;
#: NOTES.md:78-79,294). The engine measures 0.00049 on the 256-1024 test images.
SHIPPED_MAX_ABS = 1.34e-3

#: One fp16 ulp of an output in [0.5, 1): the differences between two fp16
#: outputs are multiples of it there, and 0.00134 lies between two and three.
OUT_ULP = 2.0 ** -11

#: The 1920x1080 frame (8.3 M outputs): at most this many samples may exceed
#: SHIPPED_MAX_ABS, by one ulp at most (three ulps). A CPU emulation of the
#: engine's fp16 arithmetic (row-Winograd transforms rounded to fp16, fp32
#: accumulation) puts one sample of this frame at three ulps and five at two;
#: a direct conv puts seven at two ulps and none at three, the 2-D Winograd
#: tile ten at two, so the third ulp is one sample's rounding, not a trend.
#: A wrong tile, strip edge or run boundary moves thousands of samples.
SHIPPED_1920_OVER = 4


def _code_mismatch(got, want):
    """Fraction of output samples whose 8-bit codes differ, the reference's
    accuracy tool's second gate (tests/tools/multires.py:62-73,202-208):
    round(v * 255) half to even, clipped to [0, 255]."""
    def code(v):
        return np.clip(np.round(np.asarray(v, np.float32) * 255), 0, 255).astype(np.uint8)
    return float((code(got) != code(want)).mean())


#: Fraction of 8-bit codes allowed to differ (multires.py:67-73: the reference
#: measures 1.0-2.0 % against ONNX Runtime CPU).
SHIPPED_MISMATCH = 0.025


def _shipped_gates(got, model, x, key, label):
    """Literal gates of the shipped model against the oracle in both modes:
    max-abs <= SHIPPED_MAX_ABS, PSNR >= 50 dB and <= 2.5 % 8-bit code
    mismatches, every pixel."""
    for mode in (True, False):
        want = _oracle_full(key, model, x, mode)
        s = _compare(got, want)
        s["mismatch"] = _code_mismatch(got, want)
        print(label, "fp16 storage" if mode else "fp32 throughout", s)
        assert s["max_abs"] <= SHIPPED_MAX_ABS and s["psnr"] >= 50.0, (mode, s)
        assert s["mismatch"] <= SHIPPED_MISMATCH, (mode, s)


@pytest.mark.parametrize("image", ["test_256.png", "test_512.png", "test_1024.png"])
def test_shipped_model_on_real_images(image):
    """The reference's shipped luma model on its own test images at the sizes its
    accuracy sweep feeds (multires.py:73: 256, 512, 1024), whole frames: bounded
    [0,1] output, so the literal gates apply, and the reference's 1e-3 class."""
    x = _gray8(image)
    model = _shipped_model()
    with Engine(0) as e:
        got = e.build(model).run(x)
        again = e.run(x)
    n = x.shape[2]
    assert got.shape == (1, 1, 2 * n, 2 * n) and np.isfinite(got.astype(np.float32)).all()
    np.testing.assert_array_equal(got.view(np.uint16), again.view(np.uint16))
    _shipped_gates(got.astype(np.float32), model, x, image, "shipped luma %s" % image)


def _shipped_1920():
    if not _GPU_FULL.get("shipped"):
        x = _gray8("test_1920.png")
        assert x.shape == (1, 1, 1080, 1920)
        model = _shipped_model()
        with Engine(0) as e:
            got = e.build(model).run(x)
            again = e.run(x)
        _GPU_FULL["shipped"] = (model, x, got, again)
    return _GPU_FULL["shipped"]


@pytest.mark.parametrize("round_fp16", [True, False], ids=["fp16_storage", "fp32_throughout"])
def test_shipped_model_full_1920_real_image(round_fp16):
    """The product's real workload: the shipped luma model on the reference's
    1920x1080 test photo, the whole frame against the oracle in the given mode
    (the reference's accuracy gate, NOTES.md:78-79, with at most
    SHIPPED_1920_OVER samples one output ulp past it, and its 8-bit code
    mismatch gate); bit-stable across runs."""
    model, x, got, again = _shipped_1920()
    assert got.shape == (1, 1, 2160, 3840)
    np.testing.assert_array_equal(got.view(np.uint16), again.view(np.uint16))
    got = got.astype(np.float32)
    assert np.isfinite(got).all()
    want = _oracle_full("test_1920.png", model, x, round_fp16)
    s = _compare(got, want)
    s["mismatch"] = _code_mismatch(got, want)
    s["over"] = int((np.abs(got - want) > SHIPPED_MAX_ABS).sum())
    print("shipped luma 1920x1080 full frame", "fp16 storage" if round_fp16 else "fp32 throughout",
          s, "(reference vs ONNX Runtime CPU: max-abs 0.00134)")
    assert s["max_abs"] <= 3 * OUT_ULP and s["over"] <= SHIPPED_1920_OVER, s
    assert s["psnr"] >= 50.0 and s["mismatch"] <= SHIPPED_MISMATCH, s


def test_r8f64_8k_frame_past_2gib_activations():
    """One 7680x4320 frame: each padded 64-channel activation is 4.25 GB, past the
    32-bit buffer-resource range of the fused block and the row-packed tail, so
    the engine runs every conv unfused (winograd_pipe / winograd_strip, the
    general tail). Finite, bit-stable, and four windows (two corners, the middle,
    the right edge) against the oracle with an 18-pixel margin."""
    spec = models.r8f64(seed=0)
    x = models.synthetic_input((1, 1, 4320, 7680), seed=3)
    with Engine(0) as e:
        e.build(spec)
        e.set_profiling(True)
        got = e.run(x)
        steps = [name for name, _, _ in e.profile_read()]
        e.set_profiling(False)
        again = e.run(x)
        plan = e.describe()
    assert steps and not any("block" in s for s in steps), steps
    assert "18 launches" in plan, plan
    assert got.shape == (1, 1, 8640, 15360) and np.isfinite(got).all()
    np.testing.assert_array_equal(got.view(np.uint16), again.view(np.uint16))
    got = got.astype(np.float32)
    for r0, r1, c0, c1 in ((0, 24, 0, 96), (2144, 2168, 3808, 3904), (4296, 4320, 7584, 7680),
                           (1200, 1224, 7632, 7680)):
        s, floor = _band_check(got, spec, x, r0, r1, 18, c0, c1)
        print("r8f64 8k window", (r0, r1, c0, c1), s, "floor", floor)
        assert s["rel_rms"] <= max(FLOOR_RATIO * floor["rel_rms"], 2e-3), (s, floor)


@pytest.mark.parametrize("builder,hw", [(models.c4f32, (36, 52)), (models.r8f64, (24, 40)),
                                        (models.shipped_like, (20, 36))])
def test_fp32_model_runs_the_fp16_network(builder, hw):
    """An all-fp32 model (fp32 initializers and IO, no Casts) runs exactly the
    fp16 network: against the fp16 model on the same (fp16-representable)
    input, the fp32 output is the fp16 output before its final rounding, so the
    two differ by at most half an fp16 ulp; and it is within the same bound of
    the oracle on the fp16 model as the fp16 engine output is."""
    spec = builder(seed=0)
    wide = models.widen_to_fp32(spec)
    h, w = hw
    x16 = models.synthetic_input((1, spec.in_channels, h, w), seed=3)
    with Engine(0) as e16, Engine(0) as e32:
        e16.build(spec)
        e32.build(wide)
        assert e32.io_info()[:2] == (True, True)
        y16 = e16.run(x16).astype(np.float64)
        y32 = e32.run(x16.astype(np.float32)).astype(np.float64)
    assert y32.shape == y16.shape
    half_ulp = np.spacing(np.abs(y16).astype(np.float16)).astype(np.float64) / 2
    assert np.all(np.abs(y32 - y16) <= half_ulp), float(np.abs(y32 - y16).max())
    want = run_model(spec.model, x16)
    s16, s32 = _compare(y16, want), _compare(y32, want)
    print(spec.name, "fp16 model", s16, "fp32 model", s32)
    assert s32["rel_rms"] <= s16["rel_rms"] * 1.05 + 1e-6


@pytest.mark.parametrize("builder,hw", [(models.r8f64, (1, 1)), (models.r8f64, (3, 5)),
                                        (models.r8f64, (2, 65)), (models.c4f32, (1, 3)),
                                        (models.c4f32, (7, 130)), (models.shipped_like, (5, 2))])
def test_tiny_frames(builder, hw):
    """Whole models (head, strip body, narrow tail with DepthToSpace) on frames
    of a few pixels: every kernel's edge handling at once."""
    spec = builder(seed=0)
    h, w = hw
    x = models.synthetic_input((1, spec.in_channels, h, w), seed=4)
    with Engine(0) as e:
        got = e.build(spec).run(x).astype(np.float32)
    want = run_model(spec.model, x)
    floor = run_model(spec.model, x, round_fp16=False)
    s, f = _compare(got, want), _compare(floor, want)
    print(spec.name, hw, s, "floor", f)
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    # 4 to 1000 outputs: the error ratio of so few samples is noisy (a 5x2 frame
    # measures 3.5x its floor), so these frames get 4x and an absolute 4e-3; a
    # wrong edge index costs an error of the order of the output itself.
    assert s["rel_rms"] <= max(4 * f["rel_rms"], 4e-3), (s, f)


@pytest.mark.parametrize("filters,out_ch,scale,clip,io32", [
    (64, 1, 2, None, False),      # R8F64's tail: M = 4, DepthToSpace(2)
    (32, 1, 2, (0.0, 1.0), False),
    (96, 1, 2, None, True),
    (64, 5, 1, None, False),      # M = 5, plain NCHW output
    (64, 1, 1, None, True),       # M = 1
    (96, 3, 2, (0.0, 1.0), False),  # M = 12: one MFMA operand per tap
    (32, 1, 3, None, False),      # M = 9
    (64, 1, 4, None, True),       # M = 16
])
def test_boundary_tail_convs(filters, out_ch, scale, clip, io32):
    """Head conv 1 -> F, then the boundary conv F -> out_ch * scale^2 with the
    fused DepthToSpace, Clip and fp32 output: the row-packed tail kernel for
    M <= 5 and the per-tap kernel above, on frames whose width is not a multiple
    of the 64-pixel segment."""
    spec = models.artcnn(0, filters, out_ch=out_ch, scale=scale, clip=clip, io_fp32=io32,
                         global_skip=False, bias="uniform", seed=3, name="tail")
    for h, w in [(37, 70), (9, 200)]:
        x = models.synthetic_input((1, 1, h, w), seed=5)
        if io32:
            x = x.astype(np.float32)
        with Engine(0) as e:
            got = e.build(spec).run(x).astype(np.float32)
        want = run_model(spec.model, x)
        floor = run_model(spec.model, x, round_fp16=False)
        s, f = _compare(got, want), _compare(floor, want)
        print(filters, out_ch, scale, (h, w), s, "floor", f)
        assert got.shape == want.shape == (1, out_ch, h * scale, w * scale)
        assert np.isfinite(got).all()
        assert s["rel_rms"] <= max(FLOOR_RATIO * f["rel_rms"], 2e-3), (s, f)
        assert s["max_abs"] <= 2e-2, s


@pytest.mark.parametrize("io32", [False, True])
@pytest.mark.parametrize("cin,cout", [(8, 24), (12, 20), (24, 64), (64, 64), (64, 128)])
def test_multichannel_boundary_conversions(cin, cout, io32):
    """Multi-channel NCHW boundaries: the input goes through the tiled input
    conversion (vector form when C and W are multiples of 8, scalar form
    otherwise) and a final conv with more than 16 outputs through the tiled
    output conversion. Widths cover a whole number of 128-pixel segments, a
    partial last segment and widths that are not a multiple of 8."""
    b = models._Builder(11, "uniform", io32)
    xin = "xh" if io32 else "x"
    y = b.conv(xin, cin, cout)
    m = b.finish(xin, y, cin, cout)
    for h, w in [(5, 256), (6, 200), (3, 70), (4, 13)]:
        x = models.synthetic_input((1, cin, h, w), seed=h * w, kind="normal")
        if io32:
            x = x.astype(np.float32)
        with Engine(0) as e:
            got, names = _steps(e.build(m), x)
        got = got.astype(np.float32)
        # A lone fp16 64 -> 64 conv reads the boundary input and writes the
        # boundary output itself when W % 8 == 0 (test_pipe_nchw_boundary
        # covers that path).
        pipe = cin == cout == 64 and not io32
        assert any(n.startswith("input_convert") for n in names) == (not pipe or w % 8 != 0), names
        assert any(n.startswith("output_convert") for n in names) == (not pipe or w % 8 != 0), names
        want = run_model(m, x)
        floor = run_model(m, x, round_fp16=False)
        s, f = _compare(got, want), _compare(floor, want)
        assert got.shape == want.shape == (1, cout, h, w), (got.shape, want.shape)
        assert np.isfinite(got).all()
        assert s["rel_rms"] <= max(FLOOR_RATIO * f["rel_rms"], 2e-3), ((h, w), s, f)
        assert s["max_abs"] <= 2e-2 * max(1.0, float(np.abs(want).max())), ((h, w), s)


def _steps(engine, x):
    engine.set_profiling(True)
    engine.profile_read()
    got = engine.run(x)
    names = [n for n, _, _ in engine.profile_read()]
    engine.set_profiling(False)
    return got, names


@pytest.mark.parametrize("io32", [False, True])
def test_head_reads_boundary_input(io32):
    """A one-channel input read only by the head conv goes straight into the
    head kernel (no input conversion step); an input that is also a residual
    operand keeps its padded copy. Both match the oracle."""
    spec = models.artcnn(1, 32, io_fp32=io32, bias="uniform", seed=7, name="head_in")
    x = models.synthetic_input((1, 1, 23, 70), seed=8)
    if io32:
        x = x.astype(np.float32)
    with Engine(0) as e:
        got, names = _steps(e.build(spec), x)
    assert not any(n.startswith("input_convert") for n in names), names
    want = run_model(spec.model, x)
    floor = run_model(spec.model, x, round_fp16=False)
    s, f = _compare(got.astype(np.float32), want), _compare(floor, want)
    assert s["rel_rms"] <= max(FLOOR_RATIO * f["rel_rms"], 2e-3), (s, f)

    # Same model with the graph input added to the tail's output: the input
    # is now also a residual operand.
    b = models._Builder(7, "uniform", io32)
    xin = "xh" if io32 else "x"
    h = b.conv(xin, 1, 8, "relu")
    t = b.conv(h, 8, 1)
    y = b.add(t, xin, "res")
    m = b.finish(xin, y, 1, 1)
    with Engine(0) as e:
        got2, names2 = _steps(e.build(m), x)
    assert any(n.startswith("input_convert") for n in names2), names2
    want2 = run_model(m, x)
    floor2 = run_model(m, x, round_fp16=False)
    s2, f2 = _compare(got2.astype(np.float32), want2), _compare(floor2, want2)
    assert s2["rel_rms"] <= max(FLOOR_RATIO * f2["rel_rms"], 2e-3), (s2, f2)


@pytest.mark.parametrize("builder", [models.r8f64, models.shipped_like, models.r16f96],
                         ids=["r8f64", "shipped_like", "r16f96"])
def test_full_frame_equals_cropped_runs(builder):
    """Size-independent parity at 1920x1080: every output pixel is a function of
    its receptive field only (one pixel per 3x3 conv), computed by the same
    instructions wherever it sits as long as the 2x2 Winograd tile alignment is
    kept (even offsets). So the full frame, cropped to a window with a margin of
    at least one pixel per conv, equals a run on that window bit for bit over
    the window's interior. Windows: the top-left and bottom-right corners (real
    image edges) and one in the middle. Small runs are pinned to the oracle by
    test_deep_models_within_fp16_floor; this carries that to full size."""
    spec = builder(seed=0)
    n_conv = len(spec.convs)
    m = n_conv + (n_conv & 1)  # margin, even
    H, W = 1080, 1920
    x = models.synthetic_input((1, 1, H, W), seed=7)
    s = spec.scale
    with Engine(0) as e:
        e.build(spec)
        full = e.run(x)
        assert np.isfinite(full).all(), f"{spec.name}: non-finite output at 1080p"
        for r0, r1, c0, c1 in ((0, 48, 0, 64), (520, 552, 928, 1000), (H - 40, H, W - 64, W)):
            a0, a1 = max(r0 - m, 0), min(r1 + m, H)
            b0, b1 = max(c0 - m, 0), min(c1 + m, W)
            assert a0 % 2 == 0 and b0 % 2 == 0
            win = e.run(np.ascontiguousarray(x[:, :, a0:a1, b0:b1]))
            got = win[:, :, (r0 - a0) * s:(r1 - a0) * s, (c0 - b0) * s:(c1 - b0) * s]
            want = full[:, :, r0 * s:r1 * s, c0 * s:c1 * s]
            np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16),
                                          err_msg=f"{spec.name} window {r0}:{r1},{c0}:{c1}")


def _conv64(act):
    b = models._Builder(11, "uniform")
    y = b.conv("x", 64, 64, act)
    m = b.finish("x", y, 64, 64)
    init = {t.name: t.to_numpy() for t in m.graph.initializers}
    return m, init["w0"], init["b0"]


@pytest.mark.parametrize("act", [None, "relu", "silu"])
@pytest.mark.parametrize("hw", [(1080, 1920), (37, 64), (36, 70), (35, 33), (2, 8), (1, 2),
                                (9, 1000)])
def test_pipe_nchw_boundary(act, hw):
    """A lone fp16 64 -> 64 conv reads the NCHW boundary input in the pipe's
    producers and stores the NCHW boundary output from its consumers (both for
    W % 8 == 0), with no layout pass; the output equals, bit for bit, the same
    conv on padded NHWC buffers through the kernel-level entry point (the same
    arithmetic, other layouts), and meets the literal gate against the oracle
    (small frames; the full 1080p single-layer frame is checked against the
    oracle by test_single_layer_full_size)."""
    from tests.test_conv_kernel_gpu import run_conv
    model, w16, b16 = _conv64(act)
    h, w = hw
    x = models.synthetic_input((1, 64, h, w), seed=h + 7 * w, kind="normal")
    with Engine(0) as e:
        got, names = _steps(e.build(model), x)
    assert any(n.startswith("input_convert") for n in names) == (w % 8 != 0), names
    assert any(n.startswith("output_convert") for n in names) == (w % 8 != 0), names
    code = {None: 0, "relu": 1, "silu": 2}[act]
    ref = run_conv(x, w16, b16, act=code)
    np.testing.assert_array_equal(got.view(np.uint16), ref.astype(np.float16).view(np.uint16))
    if h * w <= 40000:
        want = run_model(model, x)
        s = _compare(got.astype(np.float32), want)
        assert s["max_abs"] <= 2e-2 and s["psnr"] >= 50.0, s


@pytest.mark.parametrize("act", [None, "silu"])
def test_pipe_nchw_boundary_batch(act):
    """The NCHW boundary conv on a batch of two (each image's planes at its own
    offset, workgroup runs crossing strips and images): bit for bit the padded
    path, and the literal gate against the oracle."""
    from tests.test_conv_kernel_gpu import run_conv
    model, w16, b16 = _conv64(act)
    x = models.synthetic_input((2, 64, 37, 136), seed=5, kind="normal")
    with Engine(0) as e:
        got, names = _steps(e.build(model), x)
    assert not any(n.startswith(("input_convert", "output_convert")) for n in names), names
    code = {None: 0, "silu": 2}[act]
    ref = run_conv(x, w16, b16, act=code)
    np.testing.assert_array_equal(got.view(np.uint16), ref.astype(np.float16).view(np.uint16))
    s = _compare(got.astype(np.float32), run_model(model, x))
    assert s["max_abs"] <= 2e-2 and s["psnr"] >= 50.0, s
