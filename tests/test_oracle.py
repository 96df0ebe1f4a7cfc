"""Pins every function of the CPU oracle (oracle/) against independent checks.

Each oracle function is compared with at least one of: a library routine
(numpy's IEEE float16 casts, torch conv2d / pixel_shuffle / silu in float64,
scipy's correlate2d and expit), brute force on tiny inputs written here as
plain loops, or a closed-form invariant (the Winograd F(2x2,3x3) identity).
The checks are chosen so that a plausible mistake (transposed kernel, CRD
instead of DCR, round-toward-zero instead of round-to-nearest-even, a dropped
bias or a wrong Winograd matrix entry) fails at least one of them; the
planted-mistake tests at the end show that for the conv and DepthToSpace
checks.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import scipy.signal
import scipy.special
import torch

from oracle import ops as orc

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# fp16 conversions (hip_engine.cc:1190-1276) vs numpy's IEEE casts
# ---------------------------------------------------------------------------

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _f32_cases() -> np.ndarray:
    # every fp16 value, the midpoints between neighbours (ties), nudges either
    # side, subnormal range, overflow boundary, specials and random values
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    h = h[np.isfinite(h)].astype(np.float64)
    h = np.unique(h)
    mids = (h[:-1] + h[1:]) / 2
    cases = [h, mids, np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
             np.nextafter(mids.astype(np.float32), np.float32(-np.inf)),
             np.array([65504, 65519.99, 65520, 65536, 1e6, -65520, 2.0 ** -24, 2.0 ** -25,
                       2.0 ** -25 * 1.0000001, 2.0 ** -26, 0.0, -0.0, 3e-8, 6e-8, 5.96e-8]),
             RNG.standard_normal(100000) * 10.0 ** RNG.integers(-8, 5, 100000)]
    return np.concatenate([np.asarray(c, np.float32) for c in cases])


def test_f32_to_f16_matches_numpy_rne():
    x = _f32_cases()
    got = orc.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f32_to_f16_specials():
    x = np.array([np.inf, -np.inf, np.nan, -np.nan], np.float32)
    got = orc.f32_to_f16_bits(x)
    assert got[0] == 0x7C00 and got[1] == 0xFC00
    assert (got[2] & 0x7C00) == 0x7C00 and (got[2] & 0x3FF) and (got[2] & 0x200)


def test_round_f16_is_cast_roundtrip():
    x = _f32_cases()
    assert np.array_equal(orc.round_f16(x), x.astype(np.float16).astype(np.float32),
                          equal_nan=True)


# ---------------------------------------------------------------------------
# conv3x3 (reference.py:67-81)
# ---------------------------------------------------------------------------

def _brute_conv(x, w, b):
    """Plain-loop ONNX Conv 3x3, pads 1, stride 1 (cross-correlation)."""
    n, c, h, wd = x.shape
    m = w.shape[0]
    y = np.zeros((n, m, h, wd))
    for ni, mi, oh, ow in itertools.product(range(n), range(m), range(h), range(wd)):
        s = 0.0 if b is None else float(b[mi])
        for ci, r, q in itertools.product(range(c), range(3), range(3)):
            ih, iw = oh + r - 1, ow + q - 1
            if 0 <= ih < h and 0 <= iw < wd:
                s += float(w[mi, ci, r, q]) * float(x[ni, ci, ih, iw])
        y[ni, mi, oh, ow] = s
    return y


@pytest.mark.parametrize("acc64", [False, True])
def test_conv3x3_brute_force(acc64):
    x = RNG.standard_normal((2, 3, 4, 5)).astype(np.float32)
    w = RNG.standard_normal((4, 3, 3, 3)).astype(np.float32)
    b = RNG.standard_normal(4).astype(np.float32)
    got = orc.conv3x3(x, w, b, acc64=acc64)
    np.testing.assert_allclose(got, _brute_conv(x, w, b), rtol=1e-5, atol=1e-5)
    got0 = orc.conv3x3(x, w, None, acc64=acc64)
    np.testing.assert_allclose(got0, _brute_conv(x, w, None), rtol=1e-5, atol=1e-5)


def test_conv3x3_matches_torch_conv2d():
    x = RNG.standard_normal((2, 7, 19, 23)).astype(np.float32)
    w = RNG.standard_normal((5, 7, 3, 3)).astype(np.float32)
    b = RNG.standard_normal(5).astype(np.float32)
    want = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                      torch.from_numpy(b).double(), padding=1).numpy()
    np.testing.assert_allclose(orc.conv3x3(x, w, b, acc64=True), want, rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(orc.conv3x3(x, w, b, acc64=False), want, rtol=1e-4, atol=1e-4)


def test_conv3x3_matches_scipy_correlate():
    x = RNG.standard_normal((1, 2, 11, 9)).astype(np.float32)
    w = RNG.standard_normal((3, 2, 3, 3)).astype(np.float32)
    want = np.zeros((1, 3, 11, 9))
    for m in range(3):
        for c in range(2):
            want[0, m] += scipy.signal.correlate2d(x[0, c].astype(np.float64),
                                                   w[m, c].astype(np.float64), mode="same")
    np.testing.assert_allclose(orc.conv3x3(x, w, acc64=True), want, rtol=1e-6, atol=1e-5)


def test_conv3x3_edge_sizes():
    for h, wd in [(1, 1), (1, 7), (6, 1), (2, 2)]:
        x = RNG.standard_normal((1, 2, h, wd)).astype(np.float32)
        w = RNG.standard_normal((3, 2, 3, 3)).astype(np.float32)
        np.testing.assert_allclose(orc.conv3x3(x, w, acc64=True), _brute_conv(x, w, None),
                                   rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# elementwise ops
# ---------------------------------------------------------------------------

def test_relu_sigmoid_silu_vs_libraries():
    x = np.concatenate([RNG.standard_normal(5000) * 8, [0.0, -0.0, 40.0, -40.0, 100.0, -100.0]])
    x = x.astype(np.float32)
    t = torch.from_numpy(x).double()
    np.testing.assert_array_equal(orc.relu(x), torch.relu(t).numpy().astype(np.float32))
    np.testing.assert_allclose(orc.sigmoid(x), scipy.special.expit(x.astype(np.float64)),
                               rtol=2e-7, atol=1e-30)
    np.testing.assert_allclose(orc.silu(x), torch.nn.functional.silu(t).numpy(), rtol=2e-7,
                               atol=1e-30)


def test_add_mul():
    a = RNG.standard_normal(1000).astype(np.float32)
    b = RNG.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(orc.add(a, b), a + b)
    np.testing.assert_array_equal(orc.mul(a, b), a * b)


def test_clip_onnx_semantics():
    x = np.array([-3.0, -0.5, 0.0, 0.5, 2.0, np.nan, np.inf, -np.inf], np.float32)
    got = orc.clip(x, 0.0, 1.0)
    np.testing.assert_array_equal(got[:5], [0.0, 0.0, 0.0, 0.5, 1.0])
    assert np.isnan(got[5]) and got[6] == 1.0 and got[7] == 0.0
    np.testing.assert_array_equal(orc.clip(x), x)  # omitted bounds are +/-inf


# ---------------------------------------------------------------------------
# DepthToSpace DCR (hip_kernels.h:521-546; reference.py:84-93)
# ---------------------------------------------------------------------------

def _brute_dcr(x, b):
    """ONNX spec: y[n, c, h*b + r, w*b + q] = x[n, (r*b + q)*Cout + c, h, w]."""
    n, c, h, w = x.shape
    co = c // (b * b)
    y = np.zeros((n, co, h * b, w * b), x.dtype)
    for ni, ci, hi, wi, r, q in itertools.product(range(n), range(co), range(h), range(w),
                                                  range(b), range(b)):
        y[ni, ci, hi * b + r, wi * b + q] = x[ni, (r * b + q) * co + ci, hi, wi]
    return y


@pytest.mark.parametrize("b,co", [(1, 3), (2, 1), (2, 2), (3, 2)])
def test_depth_to_space_brute_force(b, co):
    x = RNG.standard_normal((2, co * b * b, 3, 4)).astype(np.float32)
    np.testing.assert_array_equal(orc.depth_to_space_dcr(x, b), _brute_dcr(x, b))


def test_depth_to_space_vs_pixel_shuffle():
    # One output channel: DCR and CRD coincide, so torch's pixel_shuffle (CRD)
    # must match exactly.
    x = RNG.standard_normal((1, 4, 5, 6)).astype(np.float32)
    ps = torch.nn.functional.pixel_shuffle(torch.from_numpy(x), 2).numpy()
    np.testing.assert_array_equal(orc.depth_to_space_dcr(x, 2), ps)
    # Several output channels: DCR equals pixel_shuffle of the channel
    # permutation (r, q, c) -> (c, r, q), and differs from plain pixel_shuffle.
    b, co = 2, 3
    x = RNG.standard_normal((1, co * b * b, 4, 4)).astype(np.float32)
    perm = [(r * b + q) * co + c for c in range(co) for r in range(b) for q in range(b)]
    ps = torch.nn.functional.pixel_shuffle(torch.from_numpy(x[:, perm]), b).numpy()
    got = orc.depth_to_space_dcr(x, b)
    np.testing.assert_array_equal(got, ps)
    assert not np.array_equal(got, torch.nn.functional.pixel_shuffle(torch.from_numpy(x), b).numpy())


# ---------------------------------------------------------------------------
# Winograd F(2x2,3x3) transforms
# ---------------------------------------------------------------------------

def _valid_corr(d, g):
    return np.array([[np.sum(d[i:i + 3, j:j + 3] * g) for j in range(2)] for i in range(2)])


def test_winograd_identity_matches_direct_correlation():
    """A^T [(G g G^T) . (B^T d B)] A equals the 2x2 valid correlation exactly
    in real arithmetic; checked in fp64 on random tiles."""
    for _ in range(500):
        d = RNG.standard_normal((4, 4))
        g = RNG.standard_normal((3, 3))
        y = orc.winograd_output(orc.winograd_filter(g) * orc.winograd_input(d))
        np.testing.assert_allclose(y, _valid_corr(d, g), rtol=1e-12, atol=1e-12)


def test_winograd_known_values():
    g = np.zeros((3, 3))
    g[1, 1] = 1.0  # identity kernel: U = outer(G[:,1], G[:,1]) = [0,.5,-.5,0]^T [0,.5,-.5,0]
    u = orc.winograd_filter(g)
    v = np.array([0, 0.5, -0.5, 0])
    np.testing.assert_array_equal(u, np.outer(v, v))
    d = np.arange(16, dtype=np.float64).reshape(4, 4)
    bt = np.array([[1, 0, -1, 0], [0, 1, 1, 0], [0, -1, 1, 0], [0, 1, 0, -1]], np.float64)
    np.testing.assert_array_equal(orc.winograd_input(d), bt @ d @ bt.T)
    at = np.array([[1, 1, 1, 0], [0, 1, -1, -1]], np.float64)
    m = RNG.standard_normal((4, 4))
    np.testing.assert_allclose(orc.winograd_output(m), at @ m @ at.T, rtol=0, atol=1e-14)


# ---------------------------------------------------------------------------
# graph oracle (oracle/model.py) vs an independent torch composition
# ---------------------------------------------------------------------------

def test_graph_oracle_matches_torch_composition():
    from arthip_amd import models
    from oracle.model import run_model

    spec = models.artcnn(2, 8, seed=3, name="tiny")
    x = models.synthetic_input((1, 1, 9, 13), seed=4)
    got = run_model(spec.model, x)

    consts = {t.name: t.to_numpy() for t in spec.model.graph.initializers}

    def h(t):  # fp16 tensor storage between nodes
        return t.half().double()

    def conv(t, i):
        w = torch.from_numpy(consts[f"w{i}"].astype(np.float64))
        b = torch.from_numpy(consts[f"b{i}"].astype(np.float64))
        return h(torch.nn.functional.conv2d(t, w, b, padding=1))

    t = torch.from_numpy(x.astype(np.float64))
    head = conv(t, 0)
    y = head
    k = 1
    for _ in range(2):
        r = h(torch.relu(conv(y, k)))
        y = h(conv(r, k + 1) + y)
        k += 2
    y = h(y + head)
    y = conv(y, k)
    want = torch.nn.functional.pixel_shuffle(y, 2).numpy()
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3)


def test_ramp_matches_reference_formula():
    r = orc.ramp(300)
    assert r[0] == np.float32(11 / 251) and r[1] == np.float32(48 / 251)
    assert r[6] == np.float32(((6 * 37 + 11) % 251) / 251)
    assert r.min() >= 0 and r.max() < 1


# ---------------------------------------------------------------------------
# planted mistakes must be caught by the checks above
# ---------------------------------------------------------------------------

def test_planted_transposed_kernel_is_caught():
    x = RNG.standard_normal((1, 2, 6, 7)).astype(np.float32)
    w = RNG.standard_normal((3, 2, 3, 3)).astype(np.float32)
    wrong = orc.conv3x3(x, np.ascontiguousarray(w.transpose(0, 1, 3, 2)), acc64=True)
    assert not np.allclose(wrong, _brute_conv(x, w, None), atol=1e-3)


def test_planted_crd_order_is_caught():
    b, co = 2, 2
    x = RNG.standard_normal((1, co * b * b, 3, 3)).astype(np.float32)
    crd = torch.nn.functional.pixel_shuffle(torch.from_numpy(x), b).numpy()
    assert not np.array_equal(crd, _brute_dcr(x, b))


def test_planted_winograd_sign_error_is_caught():
    d = RNG.standard_normal((4, 4))
    g = RNG.standard_normal((3, 3))
    u = orc.winograd_filter(g)
    u[1, 2] = -u[1, 2]
    y = orc.winograd_output(u * orc.winograd_input(d))
    assert not np.allclose(y, _valid_corr(d, g), atol=1e-6)


def test_planted_truncation_is_caught():
    x = _f32_cases()
    trunc = (x.view(np.uint32) & 0xFFFFE000).view(np.float32)  # round toward zero
    assert not np.array_equal(orc.f32_to_f16_bits(trunc), x.astype(np.float16).view(np.uint16))
