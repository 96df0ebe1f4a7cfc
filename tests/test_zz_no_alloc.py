"""The no-allocation entry point (arthip_engine_run_device_noalloc) through the
C ABI, against arthip_engine_run_device on the same engine and inputs: bit for
bit, on two calls in a row, the second with a smaller input (a new scratch
layout over what the first call left). Also: the device's free memory does not
change across noalloc calls, inputs beyond the scratch are refused before
anything runs, and a handle that never ran is refused."""

from __future__ import annotations

import numpy as np
import pytest

from arthip_amd import models
from arthip_amd.engine import Engine, EngineError

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 256 << 20


def _torch():
    import torch
    return torch


def _dev(x):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _bits(t):
    return t.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("builder", [models.r8f64, models.shipped_like, models.c4f32],
                         ids=["r8f64", "shipped_like", "c4f32"])
def test_noalloc_matches_run_device(builder):
    torch = _torch()
    spec = builder(seed=3)
    big = models.synthetic_input((1, spec.in_channels, 270, 480), seed=21)
    small = models.synthetic_input((1, spec.in_channels, 135, 242), seed=22)
    with Engine(0) as e:
        e.build(spec)
        ins = [_dev(big), _dev(small)]
        want = []
        for xi in ins:
            o = torch.empty(e.output_shape(tuple(xi.shape)), dtype=torch.float16, device="cuda")
            e.run_device(xi, o)
            want.append(o)
        torch.cuda.synchronize()
        outs = [torch.full_like(w, float("nan")) for w in want]
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        for xi, o in zip(ins, outs):  # the second call is the smaller input
            e.run_device_noalloc(xi, o)
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0, (free0, free1)
        for o, w in zip(outs, want):
            assert np.array_equal(_bits(o), _bits(w))
        # The same two calls again, now over the scratch contents they left.
        for xi, o in zip(ins, outs):
            o.fill_(float("nan"))
            e.run_device_noalloc(xi, o)
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert np.array_equal(_bits(o), _bits(w))


def test_noalloc_refusals():
    torch = _torch()
    spec = models.r8f64(seed=3)
    x = _dev(models.synthetic_input((1, 1, 16, 16), seed=1))
    out = torch.empty((1, 1, 32, 32), dtype=torch.float16, device="cuda")
    with Engine(0) as e:
        e.build(spec)
        with pytest.raises(EngineError, match="weights"):
            e.run_device_noalloc(x, out)  # never ran: no stream, no weights on the device
        e.run_device(x, out)
        torch.cuda.synchronize()
        # R8F64 at 1920x1080 needs four 266 MB activations: refused, nothing enqueued.
        big = torch.zeros((1, 1, 1080, 1920), dtype=torch.float16, device="cuda")
        big_out = torch.zeros((1, 1, 2160, 3840), dtype=torch.float16, device="cuda")
        with pytest.raises(EngineError, match="no-allocation scratch holds %d" % SCRATCH_BYTES):
            e.run_device_noalloc(big, big_out)
        torch.cuda.synchronize()
        assert not big_out.any()
        # The engine still works after the refusal.
        want = torch.empty_like(out)
        e.run_device(x, want)
        e.run_device_noalloc(x, out)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), _bits(want))


def test_noalloc_graph_capture_replays():
    """One noalloc run captured into a HIP graph on a side stream (after a
    warm-up run_device and a device synchronize), replayed several times with
    the program's own eager runs and synchronizations between the replays:
    every replay equals run_device bit for bit."""
    torch = _torch()
    spec = models.r8f64(seed=4)
    x = _dev(models.synthetic_input((1, 1, 135, 242), seed=31))
    x2 = _dev(models.synthetic_input((1, 1, 135, 242), seed=32))
    with Engine(0) as e:
        e.build(spec)
        shape = e.output_shape(tuple(x.shape))
        want = torch.empty(shape, dtype=torch.float16, device="cuda")
        want2 = torch.empty_like(want)
        e.run_device(x, want)
        e.run_device(x2, want2)
        torch.cuda.synchronize()
        out = torch.full(shape, float("nan"), dtype=torch.float16, device="cuda")
        side = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            e.run_device_noalloc(x, out, stream=side.cuda_stream)
        torch.cuda.synchronize()
        assert np.isnan(_bits(out).view(np.float16).astype(np.float32)).all()  # captured, not run
        other = torch.empty_like(want)
        for rep in range(4):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(_bits(out), _bits(want)), f"replay {rep}"
            # Eager work between replays: the same handle on another input,
            # through the allocated plan and through the scratch.
            e.run_device(x2, other)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(other), _bits(want2))
            e.run_device_noalloc(x2, other)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(other), _bits(want2))


def test_noalloc_capture_refuses_sync_each():
    torch = _torch()
    spec = models.c4f32(seed=2)
    x = _dev(models.synthetic_input((1, 1, 24, 40), seed=3))
    with Engine(0) as e:
        e.build(spec)
        out = torch.empty(e.output_shape(tuple(x.shape)), dtype=torch.float16, device="cuda")
        e.run_device(x, out)
        torch.cuda.synchronize()
        e.set_debug(2)  # VSHIP_SYNC_EACH
        side = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with pytest.raises(EngineError, match="SYNC_EACH"):
            with torch.cuda.graph(g, stream=side):
                e.run_device_noalloc(x, out, stream=side.cuda_stream)
        torch.cuda.synchronize()
        e.set_debug(0)
        e.run_device_noalloc(x, out)  # the handle still works
        torch.cuda.synchronize()


def test_noalloc_two_handles_two_streams():
    """Two handles share the device's scratch; their noalloc calls on two
    streams, issued back to back without host synchronization, are ordered by
    the scratch's own event: both outputs equal run_device bit for bit."""
    torch = _torch()
    specs = [models.r8f64(seed=5), models.shipped_like(seed=6)]
    xs = [_dev(models.synthetic_input((1, 1, 270, 480), seed=41)),
          _dev(models.synthetic_input((1, 1, 270, 480), seed=42))]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    with Engine(0) as a, Engine(0) as b:
        engines = [a.build(specs[0]), b.build(specs[1])]
        want, outs = [], []
        for e, x in zip(engines, xs):
            w = torch.empty(e.output_shape(tuple(x.shape)), dtype=torch.float16, device="cuda")
            e.run_device(x, w)
            want.append(w)
            outs.append(torch.full_like(w, float("nan")))
        torch.cuda.synchronize()
        for rep in range(3):
            for o in outs:
                o.fill_(float("nan"))
            torch.cuda.synchronize()
            for e, x, o, s in zip(engines, xs, outs, streams):
                e.run_device_noalloc(x, o, stream=s.cuda_stream)
            torch.cuda.synchronize()
            for o, w in zip(outs, want):
                assert np.array_equal(_bits(o), _bits(w)), f"round {rep}"
