"""ctypes bindings to oracle.c plus NumPy restatements (test infrastructure only).

Every function names the reference code it restates. Arrays are NCHW float32
unless stated otherwise.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "liboracle.so"

_lib = None


def build(force: bool = False) -> Path:
    """Compile oracle.c with gcc (oracle/Makefile); force: even when up to date."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)] + (["-B"] if force else []), check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = ctypes.CDLL(str(LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        f64p = ctypes.POINTER(ctypes.c_double)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        i64 = ctypes.c_int64
        h.or_f32_to_f16.restype = ctypes.c_uint16
        h.or_f32_to_f16.argtypes = [ctypes.c_float]
        h.or_f16_to_f32.restype = ctypes.c_float
        h.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        h.or_f32_to_f16_array.argtypes = [f32p, u16p, i64]
        h.or_f16_to_f32_array.argtypes = [u16p, f32p, i64]
        h.or_round_f16.argtypes = [f32p, i64]
        h.or_conv3x3.argtypes = [f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 f32p, f32p, ctypes.c_int, f32p, ctypes.c_int]
        for name in ("or_relu", "or_sigmoid", "or_silu"):
            getattr(h, name).argtypes = [f32p, i64]
        h.or_add.argtypes = [f32p, f32p, f32p, i64]
        h.or_mul.argtypes = [f32p, f32p, f32p, i64]
        h.or_clip.argtypes = [f32p, i64, ctypes.c_float, ctypes.c_float]
        h.or_depth_to_space_dcr.argtypes = [f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, f32p]
        for name in ("or_winograd_filter", "or_winograd_input", "or_winograd_output"):
            getattr(h, name).argtypes = [f64p, f64p]
        h.or_num_threads.restype = ctypes.c_int
        h.or_set_num_threads.argtypes = [ctypes.c_int]
        _lib = h
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray, ctype=ctypes.c_float):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# -- fp16 ----------------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    """IEEE RNE fp32 -> fp16 bit patterns (hip_engine.cc:1190-1232)."""
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_f16_array(_p(x), _p(out, ctypes.c_uint16), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    """Exact fp16 -> fp32 widening (hip_engine.cc:1251-1276)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().or_f16_to_f32_array(_p(h, ctypes.c_uint16), _p(out), h.size)
    return out


def round_f16(x) -> np.ndarray:
    """Round every element to the nearest fp16 value (fp16 tensor storage)."""
    x = _f32(x).copy()
    lib().or_round_f16(_p(x), x.size)
    return x


# -- ops -----------------------------------------------------------------------

def conv3x3(x, w, b=None, acc64: bool = False) -> np.ndarray:
    """ONNX Conv 3x3, stride 1, pads 1/1/1/1, NCHW; fp32 (or fp64) accumulation.

    Restates tests/correctness/harness/reference.py:67-81 and the geometry the
    reference engine accepts (src/vapoursynth/hip_engine.cc:397-433).
    """
    x = _f32(x)
    w = _f32(w)
    n, c, h, wd = x.shape
    m = w.shape[0]
    assert w.shape == (m, c, 3, 3), w.shape
    y = np.empty((n, m, h, wd), dtype=np.float32)
    bp = None
    if b is not None:
        bb = _f32(b)
        assert bb.shape == (m,)
        bp = _p(bb)
    lib().or_conv3x3(_p(x), n, c, h, wd, _p(w), bp, m, _p(y), 1 if acc64 else 0)
    return y


def relu(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_relu(_p(x), x.size)
    return x


def sigmoid(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_sigmoid(_p(x), x.size)
    return x


def silu(x) -> np.ndarray:
    """x * sigmoid(x): the Sigmoid+Mul pair the reference fuses (hip_engine.cc:493-522)."""
    x = _f32(x).copy()
    lib().or_silu(_p(x), x.size)
    return x


def add(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    assert a.shape == b.shape
    y = np.empty_like(a)
    lib().or_add(_p(a), _p(b), _p(y), a.size)
    return y


def mul(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    assert a.shape == b.shape
    y = np.empty_like(a)
    lib().or_mul(_p(a), _p(b), _p(y), a.size)
    return y


def clip(x, lo: float = -np.inf, hi: float = np.inf) -> np.ndarray:
    """ONNX Clip; omitted bounds are +/-inf (hip_engine.h:47-52)."""
    x = _f32(x).copy()
    lib().or_clip(_p(x), x.size, float(lo), float(hi))
    return x


def depth_to_space_dcr(x, b: int) -> np.ndarray:
    """ONNX DepthToSpace, DCR mode (hip_kernels.h:521-546; reference.py:84-93)."""
    x = _f32(x)
    n, c, h, w = x.shape
    assert c % (b * b) == 0
    y = np.empty((n, c // (b * b), h * b, w * b), dtype=np.float32)
    lib().or_depth_to_space_dcr(_p(x), n, c, h, w, b, _p(y))
    return y


# -- Winograd F(2x2,3x3) pieces (fp64) ------------------------------------------

def winograd_filter(g) -> np.ndarray:
    """U = G g G^T (hip_engine.cc:995-1016)."""
    g = np.ascontiguousarray(g, dtype=np.float64).reshape(3, 3)
    u = np.empty((4, 4), dtype=np.float64)
    lib().or_winograd_filter(_p(g, ctypes.c_double), _p(u, ctypes.c_double))
    return u


def winograd_input(d) -> np.ndarray:
    """V = B^T d B (hip_kernels.h:86-96)."""
    d = np.ascontiguousarray(d, dtype=np.float64).reshape(4, 4)
    v = np.empty((4, 4), dtype=np.float64)
    lib().or_winograd_input(_p(d, ctypes.c_double), _p(v, ctypes.c_double))
    return v


def winograd_output(m) -> np.ndarray:
    """Y = A^T M A (hip_kernels.h:133-141)."""
    m = np.ascontiguousarray(m, dtype=np.float64).reshape(4, 4)
    y = np.empty((2, 2), dtype=np.float64)
    lib().or_winograd_output(_p(m, ctypes.c_double), _p(y, ctypes.c_double))
    return y


def set_threads(n: int) -> None:
    lib().or_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().or_num_threads())


# -- shared deterministic inputs (tests/correctness/harness/reference.py:16-30) --

RAMP_MODULUS, RAMP_MULT, RAMP_ADD = 251, 37, 11


def ramp(numel: int) -> np.ndarray:
    """The reference suite's deterministic input ramp ((i*37 + 11) % 251) / 251."""
    i = np.arange(numel, dtype=np.int64)
    return ((i * RAMP_MULT + RAMP_ADD) % RAMP_MODULUS).astype(np.float32) / RAMP_MODULUS
