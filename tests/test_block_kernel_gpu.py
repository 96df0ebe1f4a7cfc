"""The fused residual block (two 64 -> 64 convs in one launch,
arthip_conv3x3_block_f16_nhwc) against the CPU oracle and against the same two
convs as separate arthip_conv3x3_f16_nhwc launches, across the reference's
geometry sweep (tests/correctness/test_engine.py:18-31), strip-width edge cases
(the kernel walks 30-pixel strips), batches, activations and 0-2 residual
inputs.

The fused kernel computes the intermediate tensor with Winograd tiles at odd
offsets (so one 16-tile block covers the 32 columns a 30-pixel output strip
reads) while a separate launch tiles at even offsets; F(2x2,3x3) rounds a
tile's two outputs differently, so the two results agree to fp16 rounding, not
bit for bit. Both are held to the per-element error model of the conv kernel
tests against the oracle, and the fused error may not exceed the two-launch
error by more than the rounding noise between them. Engine level: models with
block fusion against the oracle and against the same models with every conv
launched alone."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from arthip_amd import _lib, models
from arthip_amd.engine import Engine
from tests.test_conv_kernel_gpu import check, oracle_conv, pack, to_padded

pytestmark = pytest.mark.gpu

GEOMETRY = [(8, 8), (8, 17), (8, 24), (8, 25), (17, 16), (17, 17), (33, 17), (16, 33),
            (33, 33), (64, 64), (1082, 64), (54, 1920)]
EDGES = [(1, 1), (2, 1), (1, 2), (3, 29), (4, 30), (5, 31), (6, 32), (7, 59), (9, 60),
         (11, 61), (2, 91), (13, 3)]


def _torch():
    import torch
    return torch


def _case(seed, n, h, w, nskip):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, 64, h, w)) * 0.5).astype(np.float16)
    ws, bs = [], []
    for _ in range(2):
        ws.append((rng.standard_normal((64, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float16))
        bs.append(rng.uniform(-0.1, 0.1, 64).astype(np.float16))
    skips = [(rng.standard_normal((n, 64, h, w)) * 0.5).astype(np.float16) for _ in range(nskip)]
    return x, ws, bs, skips


def _run(x, ws, bs, skips, act1):
    """(fused output, two-launch output) as padded NHWC fp16 numpy arrays."""
    torch = _torch()
    lib = _lib.lib()
    n, c, h, w = x.shape
    dev = torch.device("cuda")
    xin = torch.from_numpy(to_padded(x)).to(dev)
    packed = [pack(wi, bi) for wi, bi in zip(ws, bs)]
    us = [torch.from_numpy(u.view(np.float16)).to(dev) for u, _ in packed]
    bb = [torch.from_numpy(b).to(dev) for _, b in packed]
    sk = [torch.from_numpy(to_padded(s)).to(dev) for s in skips]
    # Zero border (the kernels never write it), NaN interior: every interior
    # element must be written.
    fused = torch.zeros_like(xin)
    fused[:, 1:h + 1, 1:w + 1, :] = float("nan")
    mid = torch.zeros_like(xin)
    two = torch.zeros_like(xin)
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    s0 = sk[0] if len(sk) > 0 else None
    s1 = sk[1] if len(sk) > 1 else None
    rc = lib.arthip_conv3x3_block_f16_nhwc(p(xin), p(us[0]), p(bb[0]), act1, p(us[1]), p(bb[1]),
                                           p(s0), p(s1), p(fused), n, h, w, 64, None)
    assert rc == 0, _lib.last_error()
    rc = lib.arthip_conv3x3_f16_nhwc(p(xin), p(us[0]), p(bb[0]), act1, None, None, p(mid),
                                     n, h, w, 64, 64, None)
    assert rc == 0, _lib.last_error()
    rc = lib.arthip_conv3x3_f16_nhwc(p(mid), p(us[1]), p(bb[1]), 0, p(s0), p(s1), p(two),
                                     n, h, w, 64, 64, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return fused.cpu().numpy(), two.cpu().numpy()


def _interior(a, h, w):
    return a[:, 1:h + 1, 1:w + 1, :].astype(np.float32).transpose(0, 3, 1, 2)


def _rel_rms(got, want):
    want = want.astype(np.float64)
    return float(np.sqrt(np.mean((got.astype(np.float64) - want) ** 2))) / (
        float(np.sqrt(np.mean(want ** 2))) + 1e-30)


def _check_block(x, ws, bs, skips, act1, label):
    n, c, h, w = x.shape
    fused, two = _run(x, ws, bs, skips, act1)
    border = fused.copy()
    border[:, 1:h + 1, 1:w + 1, :] = 0
    assert not border.view(np.uint16).any(), f"{label}: fused block wrote outside the interior"
    assert np.isfinite(fused).all(), f"{label}: an interior element was not written"
    again, _ = _run(x, ws, bs, skips, act1)
    assert np.array_equal(again.view(np.uint16), fused.view(np.uint16)), f"{label}: not bit-stable"
    t = oracle_conv(x, ws[0], bs[0], act=act1)
    want = oracle_conv(t.astype(np.float16), ws[1], bs[1], act=0, skips=skips)
    gf, g2 = _interior(fused, h, w), _interior(two, h, w)
    check(gf, want, f"{label} fused vs oracle")
    check(g2, want, f"{label} two launches vs oracle")
    ef, e2, d = _rel_rms(gf, want), _rel_rms(g2, want), _rel_rms(gf, g2)
    print(label, "rel RMS vs oracle: fused %.3g, two launches %.3g; between them %.3g" % (ef, e2, d))
    assert ef <= e2 + d, (ef, e2, d)


@pytest.mark.parametrize("h,w", GEOMETRY + EDGES)
def test_block_geometry(h, w):
    x, ws, bs, skips = _case(h * 1000 + w, 1, h, w, 1)
    _check_block(x, ws, bs, skips, 1, f"{h}x{w}")


@pytest.mark.parametrize("h,w", EDGES + [(33, 33), (54, 1920)])
@pytest.mark.parametrize("act1,nskip", [(0, 2), (1, 2), (2, 1), (1, 0)])
def test_block_geometry_other_epilogues(h, w, act1, nskip):
    """The strip-width edge cases and two larger frames for the kernel's other
    store arrangements: with two residual inputs each output row pair's store is
    split between the two wave groups, with ReLU / no activation and one input
    the residual loads follow the conv1 fold, with SiLU they precede it."""
    x, ws, bs, skips = _case(h * 1000 + w + 97 * nskip + act1, 1, h, w, nskip)
    _check_block(x, ws, bs, skips, act1, f"{h}x{w} act1={act1} nskip={nskip}")


@pytest.mark.parametrize("act1", [0, 1, 2])
@pytest.mark.parametrize("nskip", [0, 1, 2])
def test_block_epilogues(act1, nskip):
    h, w = 37, 70
    x, ws, bs, skips = _case(7 + act1 + 10 * nskip, 2, h, w, nskip)
    _check_block(x, ws, bs, skips, act1, f"act1={act1} nskip={nskip}")


def test_block_refusals():
    lib = _lib.lib()
    torch = _torch()
    buf = torch.zeros(1024, dtype=torch.float16, device="cuda")
    out = torch.zeros(1024, dtype=torch.float16, device="cuda")
    b = torch.zeros(64, dtype=torch.float32, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    # 32 channels: not a fused block
    assert lib.arthip_conv3x3_block_f16_nhwc(p(buf), p(buf), p(b), 1, p(buf), p(b), None, None,
                                             p(out), 1, 2, 2, 32, None) == 1
    assert "C = 64" in _lib.last_error()
    # out aliasing the input, skip1 without skip0
    assert lib.arthip_conv3x3_block_f16_nhwc(p(buf), p(buf), p(b), 1, p(buf), p(b), None, None,
                                             p(buf), 1, 2, 2, 64, None) == 1
    assert "alias" in _lib.last_error()
    assert lib.arthip_conv3x3_block_f16_nhwc(p(buf), p(buf), p(b), 1, p(buf), p(b), None, p(buf),
                                             p(out), 1, 2, 2, 64, None) == 1
    assert not out.any()


def _fused_and_plain(spec, x):
    with Engine(0) as e:
        e.build(spec)
        e.set_profiling(True)
        e.profile_read()
        fused = e.run(x)
        names = [nm for nm, _, _ in e.profile_read()]
        assert any(nm.startswith("winograd_block") for nm in names), names
        e.set_debug(Engine.DEBUG_UNFUSED)
        e.profile_read()
        plain = e.run(x)
        names2 = [nm for nm, _, _ in e.profile_read()]
        assert not any(nm.startswith("winograd_block") for nm in names2), names2
    assert np.isfinite(fused).all() and np.isfinite(plain).all()
    return fused.astype(np.float32), plain.astype(np.float32)


@pytest.mark.parametrize("builder,shape", [
    (models.r8f64, (2, 1, 61, 93)), (models.r8f64, (1, 1, 1, 1)), (models.r8f64, (1, 1, 3, 31)),
    (models.r8f64, (1, 1, 48, 80)), (models.shipped_like, (1, 1, 45, 59)),
], ids=["r8f64-b2", "r8f64-1x1", "r8f64-3x31", "r8f64-48x80", "shipped_like-45x59"])
def test_engine_fused_blocks_vs_oracle(builder, shape):
    """Whole models with fused blocks against the oracle, at the deep-model gate
    (relative RMS within 3x the model's fp16-storage floor), and no worse than
    the same model with every conv launched alone."""
    from oracle.model import run_model
    spec = builder(seed=1)
    x = models.synthetic_input(shape, seed=9)
    fused, plain = _fused_and_plain(spec, x)
    want = run_model(spec.model, x)
    floor = _rel_rms(run_model(spec.model, x, round_fp16=False), want)
    ef, ep = _rel_rms(fused, want), _rel_rms(plain, want)
    print(spec.name, shape, "rel RMS vs oracle: fused %.3g, unfused %.3g, floor %.3g" % (ef, ep, floor))
    bound = 4 if shape[2] * shape[3] < 1000 else 3  # few outputs: a noisy ratio
    assert ef <= max(bound * floor, 2e-3), (ef, floor)
    assert ef <= 1.25 * ep + 1e-4, (ef, ep)


#: Per-element difference between the fused and unfused 1080p frames. R8F64
#: (outputs up to ~370): the largest measures 1.125, bound 1.7. The shipped
#: architecture's outputs are clipped to [0, 1] from pre-clip values in the
#: hundreds, so near the clip edges a rounding difference can move an output
#: by the whole range (max-abs 1 is measured): there the bound is on the share
#: of elements that differ by more than 0.05, which measures 0.30 % (0.11 % by
#: more than 0.25); bound 0.45 %.
FUSED_VS_UNFUSED_MAX_ABS = {"r8f64": 1.7}
FUSED_VS_UNFUSED_FAR = {"shipped_like": (0.05, 0.0045)}  # (threshold, largest share)


@pytest.mark.parametrize("builder", [models.r8f64, models.shipped_like],
                         ids=["r8f64", "shipped_like"])
def test_engine_fused_blocks_1080p(builder):
    """At 1920x1080 fused and unfused frames differ only by fp16 rounding: their
    relative RMS difference stays within about 3x the model's own fp16-storage
    floor (R8F64 ~1.3e-3, the shipped architecture ~8.5e-3; each engine path
    alone measures ~2x against the oracle, a wrong index would give an error of
    the order of the output)."""
    spec = builder(seed=1)
    x = models.synthetic_input((1, 1, 1080, 1920), seed=9)
    fused, plain = _fused_and_plain(spec, x)
    d = _rel_rms(fused, plain)
    diff = np.abs(np.asarray(fused, np.float64) - np.asarray(plain, np.float64))
    shares = {t: float((diff > t).mean()) for t in (1 / 255, 0.05, 0.25)}
    print(spec.name, "1080p fused vs unfused rel RMS %.3g, max-abs %.4g (output max %.4g), "
          "share of elements differing by more than" % (d, diff.max(),
                                                      np.abs(np.asarray(plain, np.float64)).max()),
          shares)
    assert d <= (4e-3 if spec.name == "r8f64" else 3e-2), d
    if spec.name in FUSED_VS_UNFUSED_MAX_ABS:
        assert diff.max() <= FUSED_VS_UNFUSED_MAX_ABS[spec.name], diff.max()
    else:
        t, share = FUSED_VS_UNFUSED_FAR[spec.name]
        assert float((diff > t).mean()) <= share, shares


@pytest.mark.parametrize("builder,want", [
    (models.r8f64, [False] * 7 + [True]),      # the last block feeds the tail
    (models.shipped_like, [False] * 7 + [True]),  # the last block feeds the residual conv
], ids=["r8f64", "shipped_like"])
def test_plain_stores_only_before_hbm_bound_steps(builder, want):
    """A fused block stores with plain stores only where the next launch is
    HBM-bound (the tail, a conv with residual inputs); blocks followed by
    another block or by a conv without residual inputs keep non-temporal
    stores. The store policy does not change a value: the output still matches
    the same model with every conv launched alone."""
    spec = builder(seed=1)
    x = models.synthetic_input((1, 1, 40, 72), seed=9)
    with Engine(0) as e:
        e.build(spec)
        e.set_profiling(True)
        e.profile_read()
        fused = e.run(x)
        steps = [nm for nm, _, _ in e.profile_read()]
    blocks = [nm for nm in steps if nm.startswith("winograd_block")]
    assert [("+cached_out" in nm) for nm in blocks] == want, steps
    assert not any("+cached_out" in nm for nm in steps if not nm.startswith("winograd_block"))
    from oracle.model import run_model
    want_y = run_model(spec.model, x)
    floor = _rel_rms(run_model(spec.model, x, round_fp16=False), want_y)
    assert _rel_rms(fused.astype(np.float32), want_y) <= max(4 * floor, 2e-3)


@pytest.mark.parametrize("shape,cached", [((1, 1, 1080, 1920), True), ((1, 1, 2160, 3840), False)],
                         ids=["1080p", "4k"])
def test_plain_stores_only_for_outputs_that_fit_the_cache(shape, cached):
    """The last R8F64 block stores plainly at 1080p (a 266 MB output) but not at
    4K (1.06 GB), where the last-level cache cannot hold the output for the
    tail."""
    spec = models.r8f64(seed=1)
    x = models.synthetic_input(shape, seed=9)
    with Engine(0) as e:
        e.build(spec)
        e.set_profiling(True)
        e.profile_read()
        y = e.run(x)
        steps = [nm for nm, _, _ in e.profile_read()]
    blocks = [nm for nm in steps if nm.startswith("winograd_block")]
    assert len(blocks) == 8, steps
    assert [("+cached_out" in nm) for nm in blocks] == [False] * 7 + [cached], steps
    assert np.isfinite(y).all()
