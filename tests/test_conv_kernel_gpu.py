"""Kernel-level parity: one fused 3x3 conv through the C ABI vs the CPU oracle.

Covers the Winograd path (C > 1) and the direct head-conv path (C == 1) across
the reference's geometry sweep (tests/correctness/test_engine.py:18-31) and
the channel counts of the benchmark configs, with each epilogue option.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from arthip_amd import _lib
from oracle import ops as orc

pytestmark = pytest.mark.gpu

GEOMETRY = [(8, 8), (8, 17), (8, 24), (8, 25), (17, 16), (17, 17), (33, 17), (16, 33),
            (33, 33), (64, 64), (1082, 64), (54, 1920)]


def _torch():
    import torch
    return torch


def _u16p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def _f32p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def pack(w16: np.ndarray, b16: np.ndarray | None):
    lib = _lib.lib()
    m, c = w16.shape[:2]
    n_u = lib.arthip_conv3x3_packed_halfs(m, c)
    n_b = lib.arthip_conv3x3_bias_len(m)
    u = np.zeros(n_u, np.uint16)
    b = np.zeros(n_b, np.float32)
    wb = np.ascontiguousarray(w16.view(np.uint16))
    bb = None if b16 is None else np.ascontiguousarray(b16.view(np.uint16))
    rc = lib.arthip_conv3x3_pack(_u16p(wb), None if bb is None else _u16p(bb), m, c,
                                 _u16p(u), n_u, _f32p(b), n_b)
    assert rc == 0, _lib.last_error()
    return u, b


def to_padded(x_nchw: np.ndarray) -> np.ndarray:
    """NCHW -> padded NHWC with a zero border (the kernels' internal layout)."""
    lib = _lib.lib()
    n, c, h, w = x_nchw.shape
    hp, wp = ctypes.c_int(), ctypes.c_int()
    assert lib.arthip_padded_dims(h, w, ctypes.byref(hp), ctypes.byref(wp)) == 0
    out = np.zeros((n, hp.value, wp.value, c), dtype=x_nchw.dtype)
    out[:, 1:h + 1, 1:w + 1, :] = x_nchw.transpose(0, 2, 3, 1)
    return out


def run_conv(x16_nchw, w16, b16, act=0, skips=()):
    """Runs the HIP conv on NCHW fp16 numpy input; returns NCHW fp32."""
    torch = _torch()
    lib = _lib.lib()
    n, c, h, w = x16_nchw.shape
    m = w16.shape[0]
    u, b = pack(w16, b16)
    dev = torch.device("cuda")
    xin = torch.from_numpy(to_padded(x16_nchw)).to(dev)
    ut = torch.from_numpy(u.view(np.float16)).to(dev)
    bt = torch.from_numpy(b).to(dev)
    sk = [torch.from_numpy(to_padded(s)).to(dev) for s in skips]
    out = torch.zeros((n, xin.shape[1], xin.shape[2], m), dtype=torch.float16, device=dev)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = lib.arthip_conv3x3_f16_nhwc(ptr(xin), ptr(ut), ptr(bt), act,
                                     ptr(sk[0]) if len(sk) > 0 else None,
                                     ptr(sk[1]) if len(sk) > 1 else None,
                                     ptr(out), n, h, w, c, m, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    # The zero border must survive the launch untouched.
    border = o.copy()
    border[:, 1:h + 1, 1:w + 1, :] = 0
    assert not border.any(), "conv wrote outside the interior of the padded output"
    return o[:, 1:h + 1, 1:w + 1, :].astype(np.float32).transpose(0, 3, 1, 2)


def oracle_conv(x16, w16, b16, act=0, skips=()):
    """Per-node fp16 storage (Conv -> act -> Add, each output rounded to fp16)."""
    y = orc.round_f16(orc.conv3x3(x16.astype(np.float32), w16.astype(np.float32),
                                  None if b16 is None else b16.astype(np.float32), acc64=True))
    if act == 1:
        y = orc.relu(y)
    elif act == 2:
        y = orc.round_f16(orc.silu(y))
    for s in skips:
        y = orc.round_f16(orc.add(y, s.astype(np.float32)))
    return y


def make_case(seed, n, c, m, h, w, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, c, h, w)) * scale).astype(np.float16)
    wt = (rng.standard_normal((m, c, 3, 3)) * np.sqrt(2.0 / (9 * c))).astype(np.float16)
    b = rng.uniform(-0.1, 0.1, m).astype(np.float16)
    return x, wt, b


def check(got, ref, label):
    assert np.isfinite(got).all(), f"{label}: non-finite output"
    err = np.abs(got - ref)
    # Error model: fp16 rounding of the conv output and of each later node costs
    # up to 2^-11 |ref| each (two ulps in all: the engine and the oracle may round
    # a conv value to neighbouring fp16 values); fp16 U and V (F(2x2,3x3)
    # Winograd) add roundings of the per-position partial products, which scale
    # with the typical term size, not with each output: an fp16 emulation of the
    # transform arithmetic on 64 channels puts the 0.99999 quantile of
    # |err| / rms(ref) at 3.9e-3, so over the 15M outputs of the largest case the
    # tail reaches about 5e-3. A wrong index or a dropped term produces errors of
    # the order of rms(ref).
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) + 1e-30
    tol = 2.0 ** -9 * np.abs(ref) + 6e-3 * rms
    bad = err > tol
    rel_rms = float(np.sqrt(np.mean((got - ref).astype(np.float64) ** 2))) / rms
    assert not bad.any(), (f"{label}: {bad.sum()} elements off, max err {err.max():.4g} "
                           f"at ref {ref.flat[err.argmax()]:.4g} (rms {rms:.3g})")
    assert rel_rms < 1e-3, f"{label}: relative RMS error {rel_rms:.3g}"
    return float(err.max())


@pytest.mark.parametrize("h,w", GEOMETRY)
def test_winograd_geometry(h, w):
    x, wt, b = make_case(1, 1, 4, 4, h, w)
    check(run_conv(x, wt, b), oracle_conv(x, wt, b), f"c4m4 {h}x{w}")


@pytest.mark.parametrize("h,w", GEOMETRY)
def test_direct_geometry(h, w):
    x, wt, b = make_case(2, 1, 1, 8, h, w)
    check(run_conv(x, wt, b), oracle_conv(x, wt, b), f"c1m8 {h}x{w}")


@pytest.mark.parametrize("c,m", [(4, 8), (4, 64), (32, 32), (64, 64), (64, 4), (96, 96),
                                 (4, 128), (3, 5), (48, 24), (1, 64), (1, 4), (1, 96)])
def test_channel_counts(c, m):
    x, wt, b = make_case(3, 1, c, m, 37, 45)
    check(run_conv(x, wt, b), oracle_conv(x, wt, b), f"c{c}m{m}")


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("nskip", [0, 1, 2])
def test_epilogue(act, nskip):
    x, wt, b = make_case(4, 1, 64, 64, 18, 34)
    rng = np.random.default_rng(5)
    skips = [rng.standard_normal((1, 64, 18, 34)).astype(np.float16) for _ in range(nskip)]
    check(run_conv(x, wt, b, act, skips), oracle_conv(x, wt, b, act, skips),
          f"act{act} skip{nskip}")


def test_batch():
    x, wt, b = make_case(6, 3, 64, 64, 20, 30)
    check(run_conv(x, wt, b, 1), oracle_conv(x, wt, b, 1), "batch3")


def test_deterministic():
    x, wt, b = make_case(7, 1, 64, 64, 96, 160)
    a = run_conv(x, wt, b, 1)
    for _ in range(3):
        np.testing.assert_array_equal(a, run_conv(x, wt, b, 1))


# C == M in {32, 64} with the fast epilogue runs the sliding-window kernel
# (winograd_strip): work items slide down 16-tile-wide strips, so these cases
# vary the strip count, partial right-edge strips, odd heights (the last tile
# row stores one output row), batches and runs that cross strip boundaries.
@pytest.mark.parametrize("h,w", GEOMETRY)
def test_strip_geometry(h, w):
    x, wt, b = make_case(8, 1, 64, 64, h, w)
    rng = np.random.default_rng(9)
    skips = [rng.standard_normal((1, 64, h, w)).astype(np.float16)]
    check(run_conv(x, wt, b, 1, skips), oracle_conv(x, wt, b, 1, skips), f"strip64 {h}x{w}")


@pytest.mark.parametrize("h,w", [(8, 8), (17, 33), (33, 17), (1082, 64), (54, 1920)])
def test_strip_c32(h, w):
    x, wt, b = make_case(10, 1, 32, 32, h, w)
    rng = np.random.default_rng(11)
    skips = [rng.standard_normal((1, 32, h, w)).astype(np.float16) for _ in range(2)]
    check(run_conv(x, wt, b, 0, skips), oracle_conv(x, wt, b, 0, skips), f"strip32 {h}x{w}")


@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("nskip", [0, 1, 2])
def test_strip_epilogue_c32(act, nskip):
    x, wt, b = make_case(12, 1, 32, 32, 19, 35)
    rng = np.random.default_rng(13)
    skips = [rng.standard_normal((1, 32, 19, 35)).astype(np.float16) for _ in range(nskip)]
    check(run_conv(x, wt, b, act, skips), oracle_conv(x, wt, b, act, skips),
          f"strip32 act{act} skip{nskip}")


def test_strip_batch_odd():
    x, wt, b = make_case(14, 3, 64, 64, 17, 45)
    rng = np.random.default_rng(15)
    skips = [rng.standard_normal((3, 64, 17, 45)).astype(np.float16) for _ in range(2)]
    check(run_conv(x, wt, b, 2, skips), oracle_conv(x, wt, b, 2, skips), "strip batch3 17x45")


def test_strip_long_runs():
    # 180 tile rows x 20 strips: every workgroup walks several items of a strip
    # and most ranges cross a strip boundary.
    x, wt, b = make_case(16, 1, 64, 64, 360, 640)
    check(run_conv(x, wt, b, 1), oracle_conv(x, wt, b, 1), "strip 360x640")


# Degenerate sizes: one tile row / column, a single pixel, widths below one
# strip (32 px) or one head-conv segment (128 px at M = 64).
TINY = [(1, 1), (1, 5), (2, 2), (3, 1), (1, 64), (5, 3), (2, 33)]


@pytest.mark.parametrize("h,w", TINY)
def test_strip_tiny(h, w):
    x, wt, b = make_case(20, 1, 64, 64, h, w)
    rng = np.random.default_rng(21)
    skips = [rng.standard_normal((1, 64, h, w)).astype(np.float16)]
    check(run_conv(x, wt, b, 1, skips), oracle_conv(x, wt, b, 1, skips), f"strip64 {h}x{w}")


@pytest.mark.parametrize("h,w", TINY)
def test_head_tiny(h, w):
    x, wt, b = make_case(22, 2, 1, 64, h, w)
    check(run_conv(x, wt, b, 1), oracle_conv(x, wt, b, 1), f"head {h}x{w}")


# The MFMA head (C = 1, M = 32, 64 or 96 without residual inputs; 64-pixel row
# segments, 16 per wave): every geometry, each activation, a batch of two.
@pytest.mark.parametrize("m", [32, 64, 96])
@pytest.mark.parametrize("h,w", GEOMETRY)
def test_head_mfma_geometry(m, h, w):
    x, wt, b = make_case(23, 1, 1, m, h, w)
    check(run_conv(x, wt, b), oracle_conv(x, wt, b), f"head{m} {h}x{w}")


@pytest.mark.parametrize("act", [0, 1, 2])
def test_head_mfma_epilogue_batch(act):
    x, wt, b = make_case(24, 2, 1, 64, 19, 70)
    check(run_conv(x, wt, b, act), oracle_conv(x, wt, b, act), f"head act{act}")


# C == M in {64, 96} without residual inputs runs a row-Winograd pipe
# (winograd_rowpipe on 64-pixel strips at 64 channels, winograd_rowpipe96 on
# 32-pixel strips at 96), its load waves' rows restarting at every strip
# boundary of a workgroup's item range.
@pytest.mark.parametrize("c", [64, 96])
@pytest.mark.parametrize("h,w", GEOMETRY)
def test_pipe_geometry(c, h, w):
    x, wt, b = make_case(30, 1, c, c, h, w)
    check(run_conv(x, wt, b, 1), oracle_conv(x, wt, b, 1), f"pipe{c} {h}x{w}")


@pytest.mark.parametrize("c", [64, 96])
@pytest.mark.parametrize("h,w", TINY)
def test_pipe_tiny(c, h, w):
    x, wt, b = make_case(31, 1, c, c, h, w)
    check(run_conv(x, wt, b, 1), oracle_conv(x, wt, b, 1), f"pipe{c} {h}x{w}")


@pytest.mark.parametrize("act", [0, 1, 2])
def test_pipe_epilogue_c64(act):
    x, wt, b = make_case(39, 1, 64, 64, 21, 70)
    check(run_conv(x, wt, b, act), oracle_conv(x, wt, b, act), f"pipe64 act{act}")


# SiLU at 64 channels: the consumers apply it in the fold (exp and reciprocal
# on the critical path), across geometries and a 360x640 frame.
@pytest.mark.parametrize("h,w", GEOMETRY + TINY + [(360, 640)])
def test_pipe_silu_c64(h, w):
    x, wt, b = make_case(40, 1, 64, 64, h, w)
    check(run_conv(x, wt, b, 2), oracle_conv(x, wt, b, 2), f"pipe64 silu {h}x{w}")


# A lone 64 -> 64 conv runs the row-Winograd pipe (64-pixel strips): a batch
# of two with a partial last strip and an odd height, so that workgroup runs
# cross strip and image boundaries, each activation.
@pytest.mark.parametrize("act", [0, 1, 2])
def test_rowpipe_batch_runs(act):
    x, wt, b = make_case(41, 2, 64, 64, 271, 200)
    check(run_conv(x, wt, b, act), oracle_conv(x, wt, b, act), f"rowpipe batch2 271x200 act{act}")


# A lone 96 -> 96 conv without residual inputs runs winograd_rowpipe96
# (32-pixel strips, the row filters split by position pairs over two waves):
# a batch of two with a partial last strip and an odd height, so that
# workgroup runs cross strip and image boundaries, each activation.
@pytest.mark.parametrize("act", [0, 1, 2])
def test_rowpipe96_batch_runs(act):
    x, wt, b = make_case(42, 2, 96, 96, 137, 100)
    check(run_conv(x, wt, b, act), oracle_conv(x, wt, b, act), f"rowpipe96 batch2 137x100 act{act}")


# winograd_rowpipe96 with one residual input, each activation (applied before
# the residual add, which the load waves do in fp16 as they store).
@pytest.mark.parametrize("act", [0, 1, 2])
def test_rowpipe96_residual_epilogues(act):
    x, wt, b = make_case(43, 1, 96, 96, 35, 70)
    skip = [np.random.default_rng(44).standard_normal((1, 96, 35, 70)).astype(np.float16)]
    check(run_conv(x, wt, b, act, skip), oracle_conv(x, wt, b, act, skip),
          f"rowpipe96 skip1 act{act} 35x70")


@pytest.mark.parametrize("act", [0, 1, 2])
def test_pipe_epilogue_c96(act):
    x, wt, b = make_case(32, 1, 96, 96, 21, 70)
    check(run_conv(x, wt, b, act), oracle_conv(x, wt, b, act), f"pipe96 act{act}")


def test_pipe_batch_odd_c96():
    x, wt, b = make_case(33, 3, 96, 96, 17, 45)
    check(run_conv(x, wt, b, 1), oracle_conv(x, wt, b, 1), "pipe96 batch3 17x45")


def test_pipe_long_runs_c96():
    # 135 tile rows x 10 strips over 256 workgroups: ranges cross strips.
    x, wt, b = make_case(34, 1, 96, 96, 270, 320)
    check(run_conv(x, wt, b, 1), oracle_conv(x, wt, b, 1), "pipe96 270x320")


@pytest.mark.parametrize("nskip", [1, 2])
@pytest.mark.parametrize("h,w", [(8, 17), (17, 33), (33, 17), (1082, 64), (54, 1920)])
def test_pipe_residual_c96(nskip, h, w):
    """96 channels with residual inputs (one: winograd_rowpipe96; two:
    winograd_pipe): the load waves fetch the residual chunks into registers a
    phase ahead and add them, in graph order, as they store."""
    x, wt, b = make_case(35, 1, 96, 96, h, w)
    rng = np.random.default_rng(36)
    skips = [rng.standard_normal((1, 96, h, w)).astype(np.float16) for _ in range(nskip)]
    check(run_conv(x, wt, b, 1, skips), oracle_conv(x, wt, b, 1, skips),
          f"pipe96 skip{nskip} {h}x{w}")


def test_pipe_residual_c96_batch_tiny():
    for n, h, w in [(3, 17, 45), (1, 1, 1), (2, 3, 5), (1, 2, 33)]:
        x, wt, b = make_case(37, n, 96, 96, h, w)
        rng = np.random.default_rng(38)
        skips = [rng.standard_normal((n, 96, h, w)).astype(np.float16) for _ in range(2)]
        check(run_conv(x, wt, b, 2, skips), oracle_conv(x, wt, b, 2, skips),
              f"pipe96 skip2 {n}x{h}x{w}")
