"""Run ordering across streams on one engine handle.

Runs on one handle share its intermediate activation buffers. The reference
serializes every frame on its one stream under a lock (hip_engine.cc:1282);
here run_device takes the caller's stream, so the engine orders each run after
the previous one on the GPU whatever streams they were given. These tests drive
one engine from two streams (and from two threads with a stream each), with
host runs in between, and require every output to equal the sequential result
bit for bit.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

from arthip_amd import models
from arthip_amd.engine import Engine

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _frames(n, shape, seed):
    return [models.synthetic_input(shape, seed=seed + i) for i in range(n)]


def test_run_device_alternating_streams_with_host_runs():
    """Frames alternate between two streams, with a host-path run (the engine's
    own stream) after every third frame; 540x960 frames take long enough
    (~0.6 ms) that unordered runs would overlap on the GPU."""
    torch = _torch()
    spec = models.r8f64(seed=2)
    shape = (1, 1, 540, 960)
    xs = _frames(9, shape, 100)
    with Engine(0) as e:
        e.build(spec)
        want = [e.run(x) for x in xs]
        oshape = want[0].shape
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        cur = torch.cuda.current_stream()
        dev_in = [torch.from_numpy(x).cuda() for x in xs]
        dev_out = [torch.empty(oshape, dtype=torch.float16, device="cuda") for _ in xs]
        for s in streams:
            s.wait_stream(cur)  # inputs and outputs were made on the current stream
        host = {}
        for i, (xi, yo) in enumerate(zip(dev_in, dev_out)):
            s = streams[i % 2]
            e.run_device(xi, yo, stream=s.cuda_stream)
            if i % 3 == 2:
                host[i] = e.run(xs[i])
        torch.cuda.synchronize()
        got = [y.cpu().numpy() for y in dev_out]
    for i in range(len(xs)):
        assert np.array_equal(got[i].view(np.uint16), want[i].view(np.uint16)), f"frame {i}"
        if i in host:
            assert np.array_equal(host[i].view(np.uint16), want[i].view(np.uint16)), f"host {i}"


def test_run_device_from_two_threads_two_streams():
    """Two threads, each with its own stream, submit frames to one engine."""
    torch = _torch()
    spec = models.r8f64(seed=3)
    shape = (1, 1, 540, 960)
    xs = _frames(8, shape, 200)
    with Engine(0) as e:
        e.build(spec)
        want = [e.run(x) for x in xs]
        oshape = want[0].shape
        dev_in = [torch.from_numpy(x).cuda() for x in xs]
        dev_out = [torch.empty(oshape, dtype=torch.float16, device="cuda") for _ in xs]
        torch.cuda.synchronize()
        errors = []

        def work(k):
            try:
                s = torch.cuda.Stream()
                for i in range(k, len(xs), 2):
                    e.run_device(dev_in[i], dev_out[i], stream=s.cuda_stream)
                s.synchronize()
            except Exception as ex:  # reported below
                errors.append(ex)

        threads = [threading.Thread(target=work, args=(k,)) for k in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        torch.cuda.synchronize()
        got = [y.cpu().numpy() for y in dev_out]
    assert not errors, errors
    for i in range(len(xs)):
        assert np.array_equal(got[i].view(np.uint16), want[i].view(np.uint16)), f"frame {i}"


def test_shape_change_between_streams():
    """A new input shape re-plans (frees and reallocates the activation buffers)
    while the previous frame may still run on another stream."""
    torch = _torch()
    spec = models.r8f64(seed=5)
    a = models.synthetic_input((1, 1, 540, 960), seed=7)
    b = models.synthetic_input((1, 1, 270, 480), seed=8)
    with Engine(0) as e:
        e.build(spec)
        want_a, want_b = e.run(a), e.run(b)
        s0, s1 = torch.cuda.Stream(), torch.cuda.Stream()
        ia, ib = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        oa = torch.empty(want_a.shape, dtype=torch.float16, device="cuda")
        ob = torch.empty(want_b.shape, dtype=torch.float16, device="cuda")
        torch.cuda.synchronize()
        e.run_device(ia, oa, stream=s0.cuda_stream)
        e.run_device(ib, ob, stream=s1.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(oa.cpu().numpy().view(np.uint16), want_a.view(np.uint16))
        assert np.array_equal(ob.cpu().numpy().view(np.uint16), want_b.view(np.uint16))
