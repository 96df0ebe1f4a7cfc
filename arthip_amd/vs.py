"""hip.Model, the VapourSynth filter, over the native filter core (include/arthip.h,
``arthip_vs_*``), with numpy planes in place of VapourSynth frames.

Mirrors src/vapoursynth/vs_hip.cpp: ``Model(...)`` takes the filter's arguments
(network_path, overlap, tilesize, device_id, num_streams, fp16,
flexible_output_prop) and the clip's format and size, refuses what hipCreate
refuses with the same "hip.Model: ..." texts, and describes the output clip;
``get_frame`` runs one frame (hipGetFrame). Formats use VapourSynth's names and
numbering (``GRAY8``, ``YUV444PS``, ``RGBH``, ...).

All compute runs in libarthip.so on the GPU; there is no Python fallback.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path
from typing import Sequence

import numpy as np

from . import _lib

GRAY, RGB, YUV = 1, 2, 3
INTEGER, FLOAT = 0, 1


@dataclass(frozen=True)
class VideoFormat:
    name: str
    color_family: int
    sample_type: int
    bits_per_sample: int
    sub_sampling_w: int = 0
    sub_sampling_h: int = 0

    @property
    def num_planes(self) -> int:
        return 1 if self.color_family == GRAY else 3

    @property
    def dtype(self) -> np.dtype:
        if self.sample_type == INTEGER:
            return np.dtype(np.uint8 if self.bits_per_sample == 8 else np.uint16)
        return np.dtype(np.float16 if self.bits_per_sample == 16 else np.float32)

    def plane_shape(self, p: int, width: int, height: int) -> tuple[int, int]:
        if p == 0:
            return height, width
        return height >> self.sub_sampling_h, width >> self.sub_sampling_w

    def _c(self) -> _lib.VsFormat:
        return _lib.VsFormat(self.color_family, self.sample_type, self.bits_per_sample,
                             self.sub_sampling_w, self.sub_sampling_h, self.num_planes)


def _fmt(name, cf, st, bits, ssw=0, ssh=0):
    return VideoFormat(name, cf, st, bits, ssw, ssh)


#: VapourSynth preset formats the filter's tests use.
FORMATS = {f.name: f for f in (
    _fmt("GRAY8", GRAY, INTEGER, 8), _fmt("GRAY16", GRAY, INTEGER, 16),
    _fmt("GRAYH", GRAY, FLOAT, 16), _fmt("GRAYS", GRAY, FLOAT, 32),
    _fmt("YUV444P8", YUV, INTEGER, 8), _fmt("YUV444P16", YUV, INTEGER, 16),
    _fmt("YUV444PH", YUV, FLOAT, 16), _fmt("YUV444PS", YUV, FLOAT, 32),
    _fmt("YUV420P8", YUV, INTEGER, 8, 1, 1), _fmt("YUV422P8", YUV, INTEGER, 8, 1, 0),
    _fmt("YUV420PS", YUV, FLOAT, 32, 1, 1),
    _fmt("RGB24", RGB, INTEGER, 8), _fmt("RGB48", RGB, INTEGER, 16),
    _fmt("RGBH", RGB, FLOAT, 16), _fmt("RGBS", RGB, FLOAT, 32),
)}


def format_from(cf: int, st: int, bits: int, ssw: int = 0, ssh: int = 0) -> VideoFormat:
    for f in FORMATS.values():
        if (f.color_family, f.sample_type, f.bits_per_sample, f.sub_sampling_w,
                f.sub_sampling_h) == (cf, st, bits, ssw, ssh):
            return f
    return VideoFormat(f"cf{cf}st{st}b{bits}", cf, st, bits, ssw, ssh)


class ModelError(RuntimeError):
    """A refusal or failure reported by the filter ("hip.Model: ...")."""


def _err() -> ctypes.Array:
    return ctypes.create_string_buffer(1024)


class Model:
    """One hip.Model filter instance (an engine pool of num_streams engines)."""

    def __init__(self, clip_format: VideoFormat | str, width: int, height: int,
                 network: str | Path | bytes, *, overlap: Sequence[int] | None = None,
                 tilesize: Sequence[int] | None = None, device_id: int | None = None,
                 num_streams: int | None = None, fp16: int | None = None,
                 flexible_output_prop: str | None = None, num_clips: int = 1):
        self._lib = _lib.lib()
        self._h = ctypes.c_void_p()
        fmt = FORMATS[clip_format] if isinstance(clip_format, str) else clip_format
        self.clip_format = fmt
        a = _lib.VsModelArgs()
        self._keep = []
        if isinstance(network, (bytes, bytearray)):
            buf = ctypes.create_string_buffer(bytes(network), len(network))
            self._keep.append(buf)
            a.network_data = ctypes.cast(buf, ctypes.c_void_p)
            a.network_size = len(network)
        else:
            a.network_path = str(network).encode()
        if device_id is not None:
            a.has_device_id, a.device_id = 1, device_id
        if num_streams is not None:
            a.has_num_streams, a.num_streams = 1, num_streams
        if fp16 is not None:
            a.has_fp16, a.fp16 = 1, fp16
        for name, vals in (("overlap", overlap), ("tilesize", tilesize)):
            if vals is not None and len(vals):
                arr = (ctypes.c_int64 * len(vals))(*vals)
                self._keep.append(arr)
                setattr(a, name, ctypes.cast(arr, ctypes.POINTER(ctypes.c_int64)))
                setattr(a, name + "_len", len(vals))
        if flexible_output_prop is not None:
            a.flexible_output_prop = flexible_output_prop.encode()
        info = _lib.VsModelInfo()
        err = _err()
        rc = self._lib.arthip_vs_model_create(ctypes.byref(a), num_clips, ctypes.byref(fmt._c()),
                                              width, height, ctypes.byref(self._h),
                                              ctypes.byref(info), err, len(err))
        if rc != 0:
            self._h = None
            raise ModelError(err.value.decode(errors="replace"))
        f = info.format
        self.format = format_from(f.color_family, f.sample_type, f.bits_per_sample)
        self.width, self.height = info.width, info.height
        self.num_planes = info.num_planes
        self.planes_written = info.planes_written
        self.flexible = bool(info.flexible)
        self.in_fp32, self.out_fp32 = bool(info.in_fp32), bool(info.out_fp32)
        self.num_streams = info.num_streams
        self.scale_w, self.scale_h = info.scale_w, info.scale_h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.arthip_vs_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def get_frame(self, planes: Sequence[np.ndarray], fmt: VideoFormat | str | None = None,
                  *, out_row_pad: int = 0) -> list[np.ndarray]:
        """One frame: ``planes`` are 2-D arrays (rows may be strided) of the
        format's sample type. Returns planes_written output planes; with
        out_row_pad > 0 they are views into buffers whose rows carry that many
        extra samples (a strided destination)."""
        fmt = self.clip_format if fmt is None else (FORMATS[fmt] if isinstance(fmt, str) else fmt)
        n = fmt.num_planes
        if len(planes) != n:
            raise ValueError(f"{fmt.name} has {n} planes, got {len(planes)}")
        src = []
        for p in planes:
            if p.dtype != fmt.dtype or p.ndim != 2 or p.strides[1] != p.itemsize:
                raise ValueError(f"plane must be 2-D {fmt.dtype} with unit column stride")
            src.append(p)
        pw = (ctypes.c_int * n)(*[p.shape[1] for p in src])
        ph = (ctypes.c_int * n)(*[p.shape[0] for p in src])
        sp = (ctypes.c_void_p * n)(*[p.ctypes.data for p in src])
        ss = (ctypes.c_ssize_t * n)(*[p.strides[0] for p in src])
        # The output size follows this frame (a variable-size clip has no fixed one).
        ow, oh = src[0].shape[1] * self.scale_w, src[0].shape[0] * self.scale_h
        od = self.format.dtype
        outs = [np.zeros((oh, ow + out_row_pad), dtype=od)[:, :ow] for _ in range(self.planes_written)]
        m = len(outs)
        dp = (ctypes.c_void_p * m)(*[o.ctypes.data for o in outs])
        ds = (ctypes.c_ssize_t * m)(*[o.strides[0] for o in outs])
        err = _err()
        rc = self._lib.arthip_vs_model_get_frame(self._h, ctypes.byref(fmt._c()), pw, ph, sp, ss,
                                                 dp, ds, m, err, len(err))
        if rc != 0:
            raise ModelError(err.value.decode(errors="replace"))
        return outs

    @staticmethod
    def version() -> tuple[str, int]:
        lib = _lib.lib()
        buf = ctypes.create_string_buffer(256)
        n = ctypes.c_int()
        lib.arthip_vs_version(buf, len(buf), ctypes.byref(n))
        return buf.value.decode(), n.value

    @staticmethod
    def device_properties(device_id: int = 0) -> dict:
        lib = _lib.lib()
        name = ctypes.create_string_buffer(256)
        pci, clk, mem = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        err = _err()
        rc = lib.arthip_vs_device_properties(device_id, name, len(name), ctypes.byref(pci),
                                             ctypes.byref(clk), ctypes.byref(mem), err, len(err))
        if rc != 0:
            raise ModelError(err.value.decode(errors="replace"))
        return {"name": name.value.decode(errors="replace"), "pci_device_id": pci.value,
                "clock_rate": clk.value, "global_memory": mem.value}
