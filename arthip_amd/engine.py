"""Host-side mirror of the reference engine interface over libarthip.so.

``Engine`` follows vship::HipEngine (src/vapoursynth/hip_engine.h:88-188):
``build`` (Build), ``output_shape`` (GetOutputShape), ``run`` (Run),
``input_is_fp32`` / ``output_is_fp32`` / ``input_channels`` /
``output_channels``. Failures raise :class:`EngineError` with the engine's own
message. ``run_device`` takes device-resident torch tensors (torch is used only
as device-memory plumbing).

``EngineHarness`` mirrors the reference's ctypes test driver
(tests/correctness/harness/engine.py) over the same-named C entry points, so
the parity tests read like the reference's own.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import _lib

_ERR_LEN = 1024


class EngineError(RuntimeError):
    """The engine rejected the model, the shape, or the run."""


def model_bytes(model) -> bytes:
    """Serialized ONNX bytes of a path, bytes, onnx_proto.Model or models.ModelSpec."""
    if isinstance(model, (str, Path)):
        return Path(model).read_bytes()
    if hasattr(model, "bytes") and callable(model.bytes):
        return model.bytes()
    if hasattr(model, "graph"):
        from .onnx_proto import encode_model
        return encode_model(model)
    return bytes(model)


def get_capability(model, device_id: int = -1) -> list[list[int]]:
    """The ONNX Runtime EP's GetCapability: node indices of each claimed run.
    device_id >= 0 claims nothing when that device cannot be initialized."""
    lib = _lib.lib()
    data = model_bytes(model)
    buf = ctypes.create_string_buffer(data, len(data))
    n_runs, n_nodes = ctypes.c_int(), ctypes.c_int()
    cap_r, cap_n = 64, 4096
    for _ in range(2):
        starts = (ctypes.c_int * (cap_r + 1))()
        nodes = (ctypes.c_int * cap_n)()
        e = _err()
        rc = lib.arthip_ep_get_capability(buf, len(data), device_id, ctypes.byref(n_runs), starts,
                                          cap_r + 1, ctypes.byref(n_nodes), nodes, cap_n, e,
                                          _ERR_LEN)
        if rc == 0:
            return [list(nodes[starts[r]:starts[r + 1]]) for r in range(n_runs.value)]
        if n_runs.value + 1 <= cap_r + 1 and n_nodes.value <= cap_n:
            raise EngineError(_msg(e, f"get_capability failed (rc={rc})"))
        cap_r, cap_n = n_runs.value, max(n_nodes.value, 1)
    raise EngineError(_msg(e, "get_capability failed"))


def run_boundary(model, nodes) -> tuple[list[str], list[str], list[str]]:
    """The fused node's MetaDef for a node run: (activations, constants, outputs)."""
    lib = _lib.lib()
    data = model_bytes(model)
    buf = ctypes.create_string_buffer(data, len(data))
    idx = (ctypes.c_int * max(len(nodes), 1))(*nodes)
    size = 1 << 16
    bufs = [ctypes.create_string_buffer(size) for _ in range(3)]
    counts = [ctypes.c_int() for _ in range(3)]
    e = _err()
    rc = lib.arthip_ep_run_boundary(buf, len(data), idx, len(nodes), bufs[0], size,
                                    ctypes.byref(counts[0]), bufs[1], size, ctypes.byref(counts[1]),
                                    bufs[2], size, ctypes.byref(counts[2]), e, _ERR_LEN)
    if rc != 0:
        raise EngineError(_msg(e, f"run_boundary failed (rc={rc})"))

    def names(b, n):
        return b.raw.split(b"\0")[:n.value] if n.value else []
    return tuple([x.decode() for x in names(b, n)] for b, n in zip(bufs, counts))


def node_keys(model, nodes) -> list[str]:
    """Each listed node's key (its first non-empty output name), which names
    the node in any node order of the same graph."""
    lib = _lib.lib()
    data = model_bytes(model)
    buf = ctypes.create_string_buffer(data, len(data))
    idx = (ctypes.c_int * max(len(nodes), 1))(*nodes)
    out = ctypes.create_string_buffer(1 << 16)
    e = _err()
    rc = lib.arthip_ep_node_keys(buf, len(data), idx, len(nodes), out, len(out), e, _ERR_LEN)
    if rc != 0:
        raise EngineError(_msg(e, f"node_keys failed (rc={rc})"))
    return [x.decode() for x in out.raw.split(b"\0")[:len(nodes)]] if nodes else []


def _err() -> ctypes.Array:
    return ctypes.create_string_buffer(_ERR_LEN)


def _msg(buf, fallback: str) -> str:
    text = bytes(buf.value).decode(errors="replace").strip()
    return text or fallback


def _shape(s) -> ctypes.Array:
    return (ctypes.c_int64 * 4)(*[int(v) for v in s])


class Engine:
    def __init__(self, device: int = 0):
        self._lib = _lib.lib()
        self._h = ctypes.c_void_p()
        e = _err()
        rc = self._lib.arthip_engine_create(device, ctypes.byref(self._h), e, _ERR_LEN)
        if rc != 0:
            raise EngineError(_msg(e, f"engine create failed (rc={rc})"))
        self.device = device

    def close(self) -> None:
        if self._h:
            self._lib.arthip_engine_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- Build ------------------------------------------------------------------
    def build(self, model) -> "Engine":
        """model: path, raw ONNX bytes, or an onnx_proto.Model / models.ModelSpec."""
        e = _err()
        if isinstance(model, (str, Path)):
            rc = self._lib.arthip_engine_build_file(self._h, str(model).encode(), e, _ERR_LEN)
        else:
            data = model_bytes(model)
            buf = ctypes.create_string_buffer(data, len(data))
            rc = self._lib.arthip_engine_build_bytes(self._h, buf, len(data), e, _ERR_LEN)
        if rc != 0:
            raise EngineError(_msg(e, f"build failed (rc={rc})"))
        return self

    def build_subgraph(self, model, nodes) -> "Engine":
        """The ONNX Runtime EP's Compile for one claimed run: the engine runs the
        given nodes (indices in graph order) of the model."""
        data = model_bytes(model)
        buf = ctypes.create_string_buffer(data, len(data))
        idx = (ctypes.c_int * max(len(nodes), 1))(*nodes)
        e = _err()
        rc = self._lib.arthip_engine_build_subgraph(self._h, buf, len(data), idx, len(nodes), e,
                                                    _ERR_LEN)
        if rc != 0:
            raise EngineError(_msg(e, f"build failed (rc={rc})"))
        return self

    # -- introspection -----------------------------------------------------------
    def io_info(self) -> tuple[bool, bool, int, int]:
        a, b, c, d = (ctypes.c_int() for _ in range(4))
        self._lib.arthip_engine_io_info(self._h, ctypes.byref(a), ctypes.byref(b),
                                        ctypes.byref(c), ctypes.byref(d))
        return bool(a.value), bool(b.value), c.value, d.value

    @property
    def input_is_fp32(self) -> bool:
        return self.io_info()[0]

    @property
    def output_is_fp32(self) -> bool:
        return self.io_info()[1]

    @property
    def input_channels(self) -> int:
        return self.io_info()[2]

    @property
    def output_channels(self) -> int:
        return self.io_info()[3]

    def output_shape(self, in_shape) -> tuple[int, int, int, int]:
        out = (ctypes.c_int64 * 4)()
        if self._lib.arthip_engine_output_shape(self._h, _shape(in_shape), out) != 0:
            raise EngineError("shape propagation failed")
        return tuple(int(v) for v in out)

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(1 << 16)
        self._lib.arthip_engine_describe(self._h, buf, len(buf))
        return buf.value.decode()

    # -- profiling ----------------------------------------------------------------
    def set_profiling(self, on: bool) -> None:
        self._lib.arthip_engine_set_profiling(self._h, 1 if on else 0)

    def profile_read(self) -> list[tuple[str, float, int]]:
        """(step name, summed ms, launches) per plan step since the last read."""
        cap = 256
        ms = (ctypes.c_double * cap)()
        cnt = (ctypes.c_int64 * cap)()
        names = ctypes.create_string_buffer(1 << 16)
        e = _err()
        n = self._lib.arthip_engine_profile_read(self._h, cap, ms, cnt, names, len(names), e,
                                                  _ERR_LEN)
        if n < 0:
            raise EngineError(_msg(e, "profile_read failed"))
        labels = names.value.decode().split("\n")
        return [(labels[i], ms[i], cnt[i]) for i in range(min(n, cap))]

    # -- diagnostics --------------------------------------------------------------
    DEBUG_POISON, DEBUG_SYNC_EACH, DEBUG_DUMP, DEBUG_UNFUSED = 1, 2, 4, 8
    DEBUG_TRACE, DEBUG_HOST_PROFILE, DEBUG_DUMPOPS, DEBUG_PLAN = 16, 32, 64, 128

    def set_debug(self, flags: int = 0, dump_dir=None) -> None:
        """The reference's VSHIP_POISON / VSHIP_SYNC_EACH / VSHIP_DUMP switches
        (hip_engine.cc:1310-1349): POISON fills every activation interior with
        fp16 NaN before each run, SYNC_EACH synchronizes after every launch, DUMP
        writes each launch's inputs and output under dump_dir (first two runs),
        UNFUSED runs every conv as its own launch (no residual-block fusion).
        Host-side lines to the engine's log (set_log): TRACE (VSHIP_TRACE),
        HOST_PROFILE (HIP_PROFILE), DUMPOPS (HIP_DUMPOPS), PLAN (VSHIP_DEBUG)."""
        d = str(dump_dir).encode() if dump_dir is not None else None
        if self._lib.arthip_engine_set_debug(self._h, int(flags), d) != 0:
            raise EngineError(_lib.last_error() or "set_debug failed")

    def set_log(self, path=None) -> None:
        """Append the TRACE / HOST_PROFILE / DUMPOPS / PLAN lines to the file at
        path (None: stderr, the default)."""
        e = _err()
        p = str(path).encode() if path is not None else None
        if self._lib.arthip_engine_set_log(self._h, p, e, len(e)) != 0:
            raise EngineError(_msg(e, "set_log failed"))

    def debug_flags(self) -> int:
        f = ctypes.c_int()
        if self._lib.arthip_engine_get_debug(self._h, ctypes.byref(f)) != 0:
            raise EngineError(_lib.last_error() or "get_debug failed")
        return f.value

    # -- Run ----------------------------------------------------------------------
    def run(self, x: np.ndarray) -> np.ndarray:
        """One batch host-to-host: x is NCHW in the model's input dtype."""
        in_fp32, out_fp32, _, _ = self.io_info()
        x = np.ascontiguousarray(x, dtype=np.float32 if in_fp32 else np.float16)
        oshape = self.output_shape(x.shape)
        out = np.empty(oshape, dtype=np.float32 if out_fp32 else np.float16)
        e = _err()
        rc = self._lib.arthip_engine_run(self._h, x.ctypes.data_as(ctypes.c_void_p),
                                         _shape(x.shape), out.ctypes.data_as(ctypes.c_void_p),
                                         out.nbytes, e, _ERR_LEN)
        if rc != 0:
            raise EngineError(_msg(e, f"run failed (rc={rc})"))
        return out

    def run_device(self, x, out, stream=None) -> None:
        """Device-resident run on torch tensors (NCHW, contiguous); no sync."""
        e = _err()
        s = ctypes.c_void_p(stream) if stream is not None else None
        rc = self._lib.arthip_engine_run_device(self._h, ctypes.c_void_p(x.data_ptr()),
                                                _shape(tuple(x.shape)),
                                                ctypes.c_void_p(out.data_ptr()), s, e, _ERR_LEN)
        if rc != 0:
            raise EngineError(_msg(e, f"run_device failed (rc={rc})"))


    def run_device_noalloc(self, x, out, stream=None) -> None:
        """run_device with the activations in the library's scratch array: no
        device allocation (for callers that cannot allocate). Needs one earlier
        run or run_device on this engine; inputs whose activations exceed the
        scratch are refused."""
        e = _err()
        s = ctypes.c_void_p(stream) if stream is not None else None
        rc = self._lib.arthip_engine_run_device_noalloc(
            self._h, ctypes.c_void_p(x.data_ptr()), _shape(tuple(x.shape)),
            ctypes.c_void_p(out.data_ptr()), s, e, _ERR_LEN)
        if rc != 0:
            raise EngineError(_msg(e, f"run_device_noalloc failed (rc={rc})"))


# ---------------------------------------------------------------------------
# Reference-style test driver
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class Probe:
    in_fp32: bool
    out_fp32: bool
    in_channels: int
    out_channels: int
    shape: tuple


@dataclass(frozen=True)
class RunResult:
    output: np.ndarray  # logical NCHW float64
    shape: tuple


class EngineHarness:
    """engine_probe / engine_run / engine_alloc_failure_then_run over the C ABI
    (tests/correctness/harness/engine_harness.cc:56-210)."""

    def __init__(self):
        self._lib = _lib.lib()

    def device_count(self) -> int:
        n = ctypes.c_int(-1)
        return n.value if self._lib.engine_device_count(ctypes.byref(n)) == 0 else -1

    def probe(self, model, *, n=1, h=16, w=16, c=1, device=0) -> Probe:
        e = _err()
        a, b, ci, co = (ctypes.c_int() for _ in range(4))
        shape = (ctypes.c_int64 * 8)()
        rank = ctypes.c_int()
        rc = self._lib.engine_probe(str(model).encode(), n, h, w, c, device, e, _ERR_LEN,
                                    ctypes.byref(a), ctypes.byref(b), ctypes.byref(ci),
                                    ctypes.byref(co), shape, ctypes.byref(rank))
        if rc != 0:
            raise EngineError(_msg(e, f"engine_probe failed (rc={rc})"))
        return Probe(bool(a.value), bool(b.value), ci.value, co.value,
                     tuple(int(shape[i]) for i in range(rank.value)))

    def run(self, model, raw_input: np.ndarray, *, n=1, h=16, w=16, c=1, device=0) -> RunResult:
        p = self.probe(model, n=n, h=h, w=w, c=c, device=device)
        raw_input = np.ascontiguousarray(raw_input)
        numel = int(np.prod(p.shape))
        cap = numel * (4 if p.out_fp32 else 2)
        out = ctypes.create_string_buffer(cap)
        ob = ctypes.c_size_t()
        of = ctypes.c_int()
        shape = (ctypes.c_int64 * 8)()
        rank = ctypes.c_int()
        e = _err()
        rc = self._lib.engine_run(str(model).encode(), n, h, w, c, device,
                                  raw_input.ctypes.data_as(ctypes.c_void_p), raw_input.nbytes,
                                  ctypes.cast(out, ctypes.c_void_p), cap, ctypes.byref(ob),
                                  ctypes.byref(of), shape, ctypes.byref(rank), e, _ERR_LEN)
        if rc != 0:
            raise EngineError(_msg(e, f"engine_run failed (rc={rc})"))
        rshape = tuple(int(shape[i]) for i in range(rank.value))
        dt = np.float32 if of.value else np.float16
        arr = np.frombuffer(out.raw[:ob.value], dtype=dt).reshape(rshape).astype(np.float64)
        return RunResult(arr, rshape)

    def alloc_failure_then_run(self, model, recovery_input: np.ndarray, *, big_h=200_000,
                               big_w=200_000, n=1, c=1, device=0) -> tuple[str, RunResult]:
        p = self.probe(model, n=n, h=16, w=16, c=c, device=device)
        recovery_input = np.ascontiguousarray(recovery_input)
        numel = int(np.prod(p.shape))
        cap = numel * (4 if p.out_fp32 else 2)
        out = ctypes.create_string_buffer(cap)
        ob = ctypes.c_size_t()
        of = ctypes.c_int()
        shape = (ctypes.c_int64 * 8)()
        rank = ctypes.c_int()
        fe, re_ = _err(), _err()
        rc = self._lib.engine_alloc_failure_then_run(
            str(model).encode(), n, big_h, big_w, c, device,
            recovery_input.ctypes.data_as(ctypes.c_void_p), recovery_input.nbytes,
            ctypes.cast(out, ctypes.c_void_p), cap, ctypes.byref(ob), ctypes.byref(of), shape,
            ctypes.byref(rank), fe, _ERR_LEN, re_, _ERR_LEN)
        fmsg = _msg(fe, "")
        if rc != 0:
            raise EngineError(f"driver rc={rc}; reported failure={fmsg!r}; "
                              f"recovery={_msg(re_, '')!r}")
        rshape = tuple(int(shape[i]) for i in range(rank.value))
        dt = np.float32 if of.value else np.float16
        arr = np.frombuffer(out.raw[:ob.value], dtype=dt).reshape(rshape).astype(np.float64)
        return fmsg, RunResult(arr, rshape)
