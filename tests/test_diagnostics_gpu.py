"""The reference's run diagnostics on the GPU (VSHIP_POISON, VSHIP_SYNC_EACH,
VSHIP_DUMP; hip_engine.cc:1310-1349, hip_graph.cc:1231-1248,1356-1365).

Poison fills every activation buffer's interior with fp16 NaN before each run;
the outputs must not change by a single bit. That pins the liveness allocator
(no launch reads a recycled buffer before this run wrote it) and the rule that
kernels write only interiors (the zero border, which poison leaves alone, is
what the convs read as padding)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from arthip_amd import models
from arthip_amd import onnx_proto as op
from arthip_amd.engine import Engine

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _case(name):
    if name == "shipped":
        model = op.load(GOLDEN / "ArtCNN_R8F64_fp16.onnx")
        x = models.synthetic_input((1, 1, 270, 480), seed=11)
        return model, x
    if name == "r8f64_1080p":
        return models.r8f64(seed=0), models.synthetic_input((1, 1, 1080, 1920), seed=1)
    if name == "r16f96":
        return models.r16f96(seed=0), models.synthetic_input((1, 1, 270, 480), seed=1)
    if name == "c4f32_fp32io":
        return models.widen_to_fp32(models.c4f32(seed=0)), \
            models.synthetic_input((1, 1, 37, 70), seed=2).astype(np.float32)
    if name == "r8f64_batch2":
        return models.r8f64(seed=1), models.synthetic_input((2, 1, 60, 90), seed=3)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["r8f64_1080p", "r16f96", "shipped", "c4f32_fp32io",
                                  "r8f64_batch2"])
def test_poison_leaves_outputs_bit_identical(name):
    model, x = _case(name)
    with Engine(0) as e:
        e.build(model)
        plain = e.run(x)
        e.set_debug(Engine.DEBUG_POISON)
        assert e.debug_flags() == Engine.DEBUG_POISON
        first = e.run(x)
        second = e.run(x)  # buffers now hold the last run's tensors, then poison
    assert np.isfinite(plain).all()
    for got in (first, second):
        assert np.array_equal(got.view(np.uint16), plain.view(np.uint16)), name


def test_poison_across_plan_changes():
    """Alternating input shapes re-plan; with poison on, each plan's first run
    and the runs after it equal unpoisoned runs."""
    spec = models.shipped_like(seed=2)
    xa = models.synthetic_input((1, 1, 64, 96), seed=4)
    xb = models.synthetic_input((1, 1, 33, 50), seed=5)
    with Engine(0) as e:
        e.build(spec)
        want_a, want_b = e.run(xa), e.run(xb)
        e.set_debug(Engine.DEBUG_POISON)
        for x, want in ((xa, want_a), (xb, want_b), (xa, want_a), (xa, want_a)):
            got = e.run(x)
            assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_sync_each_matches():
    model, x = _case("r8f64_batch2")
    with Engine(0) as e:
        e.build(model)
        plain = e.run(x)
        e.set_debug(Engine.DEBUG_SYNC_EACH | Engine.DEBUG_POISON)
        got = e.run(x)
    assert np.array_equal(got.view(np.uint16), plain.view(np.uint16))


def _padded(h, w):
    return 2 * ((h + 1) // 2) + 2, 2 * ((w + 1) // 2) + 2


@pytest.mark.parametrize("fused", [False, True], ids=["unfused", "fused"])
def test_dump_writes_every_launch_of_the_first_two_runs(tmp_path, fused):
    """R8F64 at 20x28: 18 launches with every conv alone (head conv on the NCHW
    input, 16 body convs, tail conv with DepthToSpace into the NCHW output), 10
    with the residual blocks fused. Each launch's output buffer is the padded
    NHWC activation with a zero border and a finite interior; consecutive
    launches see the same bytes; the head's input dump is the boundary input and
    the tail's output dump the returned output. Only the first two runs are
    dumped."""
    spec = models.r8f64(seed=0)
    x = models.synthetic_input((1, 1, 20, 28), seed=1)
    hp, wp = _padded(20, 28)
    n_launch = 10 if fused else 18
    flags = Engine.DEBUG_DUMP | Engine.DEBUG_POISON | (0 if fused else Engine.DEBUG_UNFUSED)
    with Engine(0) as e:
        e.build(spec)
        e.set_debug(flags, tmp_path)
        outs = [e.run(x) for _ in range(3)]
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    files = sorted(p.name for p in tmp_path.iterdir())
    assert not any(f.startswith("run3_") for f in files), files
    for run in (1, 2):
        outs_run = sorted(f for f in files if f.startswith(f"run{run}_") and f.endswith("_out.bin"))
        assert len(outs_run) == n_launch, outs_run
        head_in = (tmp_path / f"run{run}_op00_in0.bin").read_bytes()
        assert head_in == x.tobytes()
        tail_out = (tmp_path / f"run{run}_op{n_launch - 1:02d}_out.bin").read_bytes()
        assert tail_out == outs[0].tobytes()
        for k in range(n_launch - 1):
            a = np.frombuffer((tmp_path / f"run{run}_op{k:02d}_out.bin").read_bytes(),
                              np.float16).reshape(1, hp, wp, 64)
            border = a.copy()
            border[:, 1:21, 1:29, :] = 0
            assert not border.view(np.uint16).any(), f"op{k}: nonzero border"
            assert np.isfinite(a[:, 1:21, 1:29, :]).all(), f"op{k}: non-finite interior"
            nxt = (tmp_path / f"run{run}_op{k + 1:02d}_in0.bin").read_bytes()
            assert nxt == a.tobytes(), f"op{k + 1} input differs from op{k} output"


def test_host_log_lines(tmp_path):
    """TRACE, HOST_PROFILE, DUMPOPS and PLAN (the reference's VSHIP_TRACE,
    HIP_PROFILE, HIP_DUMPOPS and VSHIP_DEBUG) write their lines to the engine's
    log: the plan once per new shape, per run an enter / built / one line per
    launch / done sequence, one op-dump line per launch naming its buffers, and
    the host time spans; the output does not change."""
    import re

    spec = models.r8f64(seed=0)
    x = models.synthetic_input((1, 1, 60, 90), seed=2)
    log = tmp_path / "engine.log"
    with Engine(0) as e:
        e.build(spec)
        want = e.run(x)
        e.set_debug(Engine.DEBUG_TRACE | Engine.DEBUG_HOST_PROFILE | Engine.DEBUG_DUMPOPS
                    | Engine.DEBUG_PLAN)
        e.set_log(log)
        y1 = e.run(x)  # same shape: planned already, no plan lines
        y2 = e.run(np.ascontiguousarray(x[:, :, :40, :70]))  # a new plan
        e.set_debug(0)
        e.set_log(None)
    np.testing.assert_array_equal(y1.view(np.uint16), want.view(np.uint16))
    lines = log.read_text().splitlines()
    steps = [l for l in lines if l.startswith("[vship] step")]
    assert len(steps) == 10, lines  # head, 8 blocks, tail
    assert sum(l.startswith("[vship] plan for [1,1,40,70]: 10 launches") for l in lines) == 1
    for r, out_shape in ((1, y1), (2, y2)):
        mine = [l for l in lines if re.match(r"\[run\] (enter |built |done |fail )?#%d\b" % r, l)]
        assert mine[0].startswith("[run] enter #%d run in=0x" % r), mine
        assert mine[1] == "[run] built #%d" % r, mine
        ops = mine[2:-1]
        assert [l.split()[2] for l in ops] == ["op%d" % k for k in range(10)], ops
        assert "direct_conv" in ops[0] and all("winograd_block" in l for l in ops[1:9])
        assert "+dts2" in ops[9], ops
        assert mine[-1].startswith("[run] done #%d out=0x" % r), mine
    dumps = [l for l in lines if l.startswith("[dump] op ")]
    assert len(dumps) == 20, dumps
    assert all(" in=" in l and " out=" in l for l in dumps)
    assert dumps[0].split(" in=")[1].startswith("input(0x"), dumps[0]  # the head reads the input
    assert dumps[9].split(" out=")[1].startswith("output(0x"), dumps[9]  # the tail writes the output
    prof = [l for l in lines if l.startswith("[hipprof]")]
    assert len(prof) == 4, prof
    assert re.match(r"\[hipprof\] build=[0-9.]+ms memin=[0-9.]+ms launch=[0-9.]+ms "
                    r"readback\+wait=[0-9.]+ms$", prof[0]), prof
    assert re.match(r"\[hipprof\] memout=[0-9.]+ms total=[0-9.]+ms$", prof[1]), prof


def test_vs_trace_lines(capfd, monkeypatch):
    """VSHIP_TRACE=1 at filter creation: an enter and a leave line on stderr
    around every frame, naming the pool's engine (vs_hip.cpp:239-246)."""
    import re

    from arthip_amd import vs

    monkeypatch.setenv("VSHIP_TRACE", "1")
    frame = models.synthetic_input((1, 1, 24, 40), seed=3)[0, 0]
    with vs.Model("GRAYH", 40, 24, op.encode_model(models.c4f32(seed=0).model),
                  num_streams=2) as m:
        monkeypatch.delenv("VSHIP_TRACE")
        capfd.readouterr()
        for _ in range(3):
            m.get_frame([frame])
    err = capfd.readouterr().err.splitlines()
    enters = [l for l in err if l.startswith("[trace] enter")]
    leaves = [l for l in err if l.startswith("[trace] leave")]
    assert len(enters) == 3 and len(leaves) == 3, err
    for k, (a, b) in enumerate(zip(enters, leaves)):
        ma = re.match(r"\[trace\] enter eng=([01]) n=(\d+) t=(\d+)$", a)
        mb = re.match(r"\[trace\] leave eng=([01]) n=(\d+) t=(\d+)$", b)
        assert ma and mb, (a, b)
        assert ma.group(1) == mb.group(1) and int(ma.group(2)) == int(mb.group(2)) == k
        assert int(mb.group(3)) >= int(ma.group(3))
