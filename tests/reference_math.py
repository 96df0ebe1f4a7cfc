"""Float64 reference math and comparison helpers for the engine tests.

Mirrors the reference suite's helpers (tests/correctness/harness/reference.py):
the shared deterministic ramp input (16-30), the float64 3x3 SAME conv
(67-81), DepthToSpace DCR (84-93), and NaN-aware closeness (96-112). The
float64 conv here is numpy, independent of the C oracle it also checks.
"""

from __future__ import annotations

import numpy as np

#: Tolerance of one fp16 conv chain (reference.py:22).
FP16_CONV_TOL = 2e-2


def ramp(numel: int) -> np.ndarray:
    i = np.arange(numel, dtype=np.int64)
    return ((i * 37 + 11) % 251).astype(np.float32) / 251


def raw_input(c: int, h: int, w: int, in_fp32: bool, n: int = 1) -> np.ndarray:
    flat = ramp(n * c * h * w).reshape(n, c, h, w)
    return flat.astype(np.float32) if in_fp32 else flat.astype(np.float16)


def logical_input(c: int, h: int, w: int, in_fp32: bool, n: int = 1) -> np.ndarray:
    return raw_input(c, h, w, in_fp32, n).astype(np.float64)


def conv3x3(x: np.ndarray, weight: np.ndarray, bias=None) -> np.ndarray:
    m, c, kh, kw = weight.shape
    n, _, h, w = x.shape
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (1, 1), (1, 1)))
    wt = weight.astype(np.float64)
    out = np.zeros((n, m, h, w), np.float64)
    for r in range(kh):
        for s in range(kw):
            out += np.einsum("mc,nchw->nmhw", wt[:, :, r, s], xp[:, :, r:r + h, s:s + w])
    if bias is not None:
        out += np.asarray(bias, np.float64)[None, :, None, None]
    return out


def depth_to_space_dcr(x: np.ndarray, b: int) -> np.ndarray:
    n, c, h, w = x.shape
    return (x.reshape(n, b, b, c // (b * b), h, w).transpose(0, 3, 4, 1, 5, 2)
            .reshape(n, c // (b * b), h * b, w * b))


def max_abs_diff(got, ref) -> float:
    if not np.isfinite(got).all():
        return float("inf")
    return float(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64)).max())


def assert_close(got, ref, tol: float, label: str) -> float:
    assert np.isfinite(got).all(), f"{label}: output contains non-finite values"
    d = max_abs_diff(got, ref)
    assert d < tol, f"{label}: max abs diff {d:.6g} >= tolerance {tol:g}"
    return d


def psnr(got, ref, peak: float = 1.0) -> float:
    mse = float(np.mean((np.asarray(got, np.float64) - np.asarray(ref, np.float64)) ** 2))
    return float("inf") if mse == 0 else 10.0 * np.log10(peak * peak / mse)
