"""Loader for libarthip.so, the native engine (C ABI declared in include/arthip.h).

The library is built in-tree (``arthip_amd/_build/libarthip.so``) by
``arthip_amd.build.build()``. There is no Python fallback for any compute: if
the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "_build" / "libarthip.so"

_lib = None


class LibraryMissing(RuntimeError):
    """libarthip.so has not been built (run arthip_amd.build.build())."""


class VsFormat(ctypes.Structure):
    """arthip_vs_format (VSVideoFormat's fields the filter reads)."""
    _fields_ = [("color_family", ctypes.c_int), ("sample_type", ctypes.c_int),
                ("bits_per_sample", ctypes.c_int), ("sub_sampling_w", ctypes.c_int),
                ("sub_sampling_h", ctypes.c_int), ("num_planes", ctypes.c_int)]


class VsModelArgs(ctypes.Structure):
    """arthip_vs_model_args (hip.Model's arguments)."""
    _fields_ = [("network_path", ctypes.c_char_p), ("network_data", ctypes.c_void_p),
                ("network_size", ctypes.c_size_t),
                ("has_device_id", ctypes.c_int), ("device_id", ctypes.c_int64),
                ("has_num_streams", ctypes.c_int), ("num_streams", ctypes.c_int64),
                ("has_fp16", ctypes.c_int), ("fp16", ctypes.c_int64),
                ("overlap", ctypes.POINTER(ctypes.c_int64)), ("overlap_len", ctypes.c_int),
                ("tilesize", ctypes.POINTER(ctypes.c_int64)), ("tilesize_len", ctypes.c_int),
                ("flexible_output_prop", ctypes.c_char_p)]


class VsModelInfo(ctypes.Structure):
    """arthip_vs_model_info (the output clip)."""
    _fields_ = [("format", VsFormat), ("width", ctypes.c_int), ("height", ctypes.c_int),
                ("num_planes", ctypes.c_int), ("planes_written", ctypes.c_int),
                ("flexible", ctypes.c_int), ("in_fp32", ctypes.c_int), ("out_fp32", ctypes.c_int),
                ("num_streams", ctypes.c_int), ("scale_w", ctypes.c_int),
                ("scale_h", ctypes.c_int)]


def _declare(lib: ctypes.CDLL) -> None:
    c_int, c_size, c_void, c_char = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
    i32p = ctypes.POINTER(ctypes.c_int)
    i64p = ctypes.POINTER(ctypes.c_int64)
    sizep = ctypes.POINTER(ctypes.c_size_t)
    u16p = ctypes.POINTER(ctypes.c_uint16)
    f32p = ctypes.POINTER(ctypes.c_float)
    eng = c_void

    def sig(name, res, *args):
        try:
            fn = getattr(lib, name)
        except AttributeError:  # reported by tests/test_capi_exports.py
            return
        fn.restype = res
        fn.argtypes = list(args)

    sig("arthip_engine_create", c_int, c_int, ctypes.POINTER(c_void), c_char, c_int)
    sig("arthip_engine_destroy", None, eng)
    sig("arthip_engine_build_file", c_int, eng, c_char, c_char, c_int)
    sig("arthip_engine_build_bytes", c_int, eng, c_void, c_size, c_char, c_int)
    sig("arthip_engine_output_shape", c_int, eng, i64p, i64p)
    sig("arthip_engine_io_info", c_int, eng, i32p, i32p, i32p, i32p)
    sig("arthip_engine_run", c_int, eng, c_void, i64p, c_void, c_size, c_char, c_int)
    sig("arthip_engine_run_device", c_int, eng, c_void, i64p, c_void, c_void, c_char, c_int)
    sig("arthip_engine_run_device_noalloc", c_int, eng, c_void, i64p, c_void, c_void, c_char,
        c_int)
    sig("arthip_engine_describe", c_int, eng, c_char, c_int)
    sig("arthip_engine_set_profiling", c_int, eng, c_int)
    sig("arthip_engine_profile_read", c_int, eng, c_int, ctypes.POINTER(ctypes.c_double), i64p,
        c_char, c_int, c_char, c_int)
    sig("arthip_engine_set_debug", c_int, eng, c_int, c_char)
    sig("arthip_engine_get_debug", c_int, eng, i32p)
    sig("arthip_engine_set_log", c_int, eng, c_char, c_char, c_int)

    sig("engine_device_count", c_int, i32p)
    sig("engine_probe", c_int, c_char, c_int, c_int, c_int, c_int, c_int, c_char, c_int,
        i32p, i32p, i32p, i32p, i64p, i32p)
    sig("engine_run", c_int, c_char, c_int, c_int, c_int, c_int, c_int, c_void, c_size,
        c_void, c_size, sizep, i32p, i64p, i32p, c_char, c_int)
    sig("engine_alloc_failure_then_run", c_int, c_char, c_int, c_int, c_int, c_int, c_int,
        c_void, c_size, c_void, c_size, sizep, i32p, i64p, i32p, c_char, c_int, c_char, c_int)

    sig("arthip_ep_get_capability", c_int, c_void, c_size, c_int, i32p, i32p, c_int, i32p, i32p,
        c_int, c_char, c_int)
    sig("arthip_engine_build_subgraph", c_int, eng, c_void, c_size, i32p, c_int, c_char, c_int)
    sig("arthip_ep_run_boundary", c_int, c_void, c_size, i32p, c_int, c_char, c_int, i32p, c_char,
        c_int, i32p, c_char, c_int, i32p, c_char, c_int)
    sig("arthip_ep_node_keys", c_int, c_void, c_size, i32p, c_int, c_char, c_int, c_char, c_int)

    fmtp = ctypes.POINTER(VsFormat)
    ptrs = ctypes.POINTER(c_void)
    pdp = ctypes.POINTER(ctypes.c_ssize_t)
    sig("arthip_vs_model_create", c_int, ctypes.POINTER(VsModelArgs), c_int, fmtp, c_int, c_int,
        ctypes.POINTER(c_void), ctypes.POINTER(VsModelInfo), c_char, c_int)
    sig("arthip_vs_model_get_frame", c_int, c_void, fmtp, i32p, i32p, ptrs, pdp, ptrs, pdp, c_int,
        c_char, c_int)
    sig("arthip_vs_model_destroy", None, c_void)
    sig("arthip_vs_version", c_int, c_char, c_int, i32p)
    sig("arthip_vs_device_properties", c_int, c_int, c_char, c_int, i64p, i64p, i64p, c_char,
        c_int)

    sig("arthip_conv3x3_packed_halfs", c_size, c_int, c_int)
    sig("arthip_conv3x3_bias_len", c_size, c_int)
    sig("arthip_conv3x3_pack", c_int, u16p, u16p, c_int, c_int, u16p, c_size, f32p, c_size)
    sig("arthip_conv3x3_f16_nhwc", c_int, c_void, c_void, c_void, c_int, c_void, c_void, c_void,
        c_int, c_int, c_int, c_int, c_int, c_void)
    sig("arthip_conv3x3_block_f16_nhwc", c_int, c_void, c_void, c_void, c_int, c_void, c_void,
        c_void, c_void, c_void, c_int, c_int, c_int, c_int, c_void)
    sig("arthip_conv3x3_limits", c_int, i32p, i32p)
    sig("arthip_padded_dims", c_int, c_int, c_int, i32p, i32p)
    sig("arthip_f32_to_f16", ctypes.c_uint16, ctypes.c_float)
    sig("arthip_f16_to_f32", ctypes.c_float, ctypes.c_uint16)
    sig("arthip_f32_to_f16_no_subnormals", ctypes.c_uint16, ctypes.c_float)
    sig("arthip_last_error", c_char)
    sig("arthip_version", c_char)


#: Every symbol include/arthip.h declares (checked by tests/test_capi_exports.py).
EXPORTED_SYMBOLS = (
    "arthip_engine_create", "arthip_engine_destroy", "arthip_engine_build_file",
    "arthip_engine_build_bytes", "arthip_engine_output_shape", "arthip_engine_io_info",
    "arthip_engine_run", "arthip_engine_run_device", "arthip_engine_run_device_noalloc",
    "arthip_engine_describe",
    "arthip_engine_set_profiling", "arthip_engine_profile_read", "arthip_engine_set_debug",
    "arthip_engine_get_debug", "arthip_engine_set_log",
    "engine_device_count", "engine_probe", "engine_run", "engine_alloc_failure_then_run",
    "arthip_ep_get_capability", "arthip_ep_run_boundary", "arthip_ep_node_keys",
    "arthip_engine_build_subgraph",
    "arthip_vs_model_create", "arthip_vs_model_get_frame", "arthip_vs_model_destroy",
    "arthip_vs_version", "arthip_vs_device_properties",
    "arthip_conv3x3_packed_halfs", "arthip_conv3x3_bias_len", "arthip_conv3x3_pack",
    "arthip_conv3x3_f16_nhwc", "arthip_conv3x3_block_f16_nhwc", "arthip_conv3x3_limits", "arthip_padded_dims", "arthip_f32_to_f16",
    "arthip_f16_to_f32", "arthip_f32_to_f16_no_subnormals", "arthip_last_error", "arthip_version",
)


def lib() -> ctypes.CDLL:
    """The loaded native library; raises LibraryMissing if it is not built."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("ARTHIP_LIB", LIB_PATH))
        if not path.exists():
            raise LibraryMissing(
                f"{path} not found: the HIP engine is not built (python -c "
                "'import arthip_amd.build as b; b.build()'). There is no CPU fallback.")
        handle = ctypes.CDLL(str(path))
        _declare(handle)
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().arthip_last_error().decode(errors="replace")
