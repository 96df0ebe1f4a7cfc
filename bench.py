#!/usr/bin/env python3
"""Frames/s of the ArtCNN-style R8F64 2x luma upscaler at 1920x1080 on one MI355X.

A step is one frame: a 1x1x1080x1920 fp16 luma frame already resident in HBM
goes through the whole engine (head conv, 8 residual blocks, global skip, tail
conv with fused DepthToSpace) to a 1x1x2160x3840 fp16 frame in HBM. W warmup
steps, then K timed steps bracketed by a device synchronize on both sides.
Prints one JSON line.

Extra objects in the line:
  roofline      the dominant kernel of the frame (the fused residual block,
                winograd_block, when the model has 64-channel blocks; else the
                Winograd body conv). Every launch of a second pass of K frames is
                bracketed by HIP events on the launch stream (the timed pass runs
                without them); per kernel: algorithmic bytes (each tensor the
                launch reads or writes, fp16, once, plus weights) and algorithmic
                flops (direct-conv equivalent, 2*9*Cin*Cout per pixel and conv, and
                the share a Winograd kernel executes: 16/36 for F(2x2,3x3), 6/9 for
                the fused block's F(2,3) along x) over the mean launch time.
                The bound follows the kernel's algorithmic intensity against the
                MI355X ridge (2.5 PFLOP/s fp16 dense / 8 TB/s = 312 flop/B): a
                fused block does 2 convs' flops per input/output pass (384
                flop/B), so it is MFMA-bound; a single 64->64 conv (288 flop/B)
                is HBM-bound. `kernels` lists every launch kind with its own
                figures. traffic: measured HBM bytes per launch (rocprofv3
                FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's reading) and
                trace_mean_us (rocprofv3 kernel trace) from the committed
                profiles/traffic.json for this workload, when present.
                stream_copy_gbs: a plain device copy of one activation-sized
                buffer, what streaming code reaches on this device.
  cpu_baseline  the CPU oracle (oracle/, plain C + OpenMP, fp32 math with fp16
                storage between nodes) on a bounded band of the same frame on the
                host's cores (2 warm-up runs, median of 5 timed runs), scaled to
                frames/s; with the thread count used, the physical cores and the
                CPU model.
  cpu_library   the same band through torch's CPU conv2d (oneDNN) in fp32 on all
                host threads: what an optimized CPU library reaches on this model
                (ONNX Runtime is not installed), for scale beside the oracle.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
MFMA_FP16_PEAK_TFLOPS = 2500.0


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--height", type=int, default=1080)
    p.add_argument("--width", type=int, default=1920)
    p.add_argument("--model", default="r8f64",
                   choices=["r8f64", "r16f96", "c4f32", "shipped_like", "single64"],
                   help="r8f64 (default, the headline workload); shipped_like: the shipped "
                        "luma model's architecture (SiLU, 3-conv blocks, Clip) with synthetic "
                        "weights; single64: one 64->64 conv + bias + ReLU on a 64-channel "
                        "N(0, 0.5) input")
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--cpu-rows", type=int, default=-1,
                   help="rows of the frame in the CPU baseline sample (0 disables it; default: "
                        "about 2-3 s of CPU work per run, 2 warm-up and 5 timed runs: r8f64 80, "
                        "shipped_like 56, r16f96 16, single64 and c4f32 the whole frame)")
    p.add_argument("--no-profile", action="store_true",
                   help="skip the per-launch event timing (roofline becomes null)")
    p.add_argument("--no-e2e", action="store_true",
                   help="skip the host-buffer (PCIe-inclusive) rates (end_to_end becomes null)")
    p.add_argument("--host-path", type=int, default=0, metavar="STREAMS",
                   help="instead of the device-resident bench, time the VapourSynth filter "
                        "path (host planes in and out, PCIe included) with STREAMS engines and "
                        "STREAMS + 1 caller threads; prints its own JSON line")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                   help="instead of the bench, run a plain device copy of MB megabytes "
                        "(--steps times): the known-traffic kernel that scales rocprofv3 "
                        "FETCH_SIZE / WRITE_SIZE readings")
    p.add_argument("--summarize-profile", default="", metavar="DIR",
                   help="instead of the bench, summarize rocprofv3 csv output under DIR "
                        "(DIR/kt: --kernel-trace --stats; DIR/fetch, DIR/write: --pmc "
                        "FETCH_SIZE / WRITE_SIZE; DIR/cal_fetch, DIR/cal_write: the same "
                        "counters on --calibrate-copy; optional DIR/p1, DIR/p2: the SQ "
                        "counter passes listed in the output) into per-launch figures of one "
                        "frame; prints markdown tables and writes JSON to --profile-json")
    p.add_argument("--profile-json", default="", metavar="FILE")
    p.add_argument("--profile-key", default="", metavar="KEY",
                   help="workload key of the summary, e.g. r8f64_1080x1920")
    p.add_argument("--frames", type=int, default=0,
                   help="with --summarize-profile: frames in the trace run (warmup + steps)")
    p.add_argument("--skip-frames", type=int, default=0,
                   help="with --summarize-profile: leading (warmup) frames of the trace run "
                        "left out of the launch times")
    return p.parse_args()


def calibrate_copy(mb: int, steps: int) -> int:
    import torch
    n = mb * (1 << 20) // 2
    x = torch.ones(n, dtype=torch.float16, device="cuda")
    y = torch.empty_like(x)
    for _ in range(steps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes_read": 2 * n, "calibrate_copy_bytes_written": 2 * n,
                      "launches": steps}), flush=True)
    return 0


def host_cpu() -> tuple[str, int]:
    """CPU model name and physical core count of this host (/proc/cpuinfo)."""
    model, cores = "unknown", set()
    try:
        phys = core = None
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model == "unknown":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    return model, len(cores) or (os.cpu_count() or 0)


def cpu_baseline(spec, x_full, rows: int) -> dict | None:
    """Times the C oracle on a band of `rows` input rows (full width): two
    warm-up runs, then the median of five timed runs."""
    if rows <= 0:
        return None
    import statistics

    import numpy as np

    from oracle import ops as orc
    from oracle.model import run_model

    threads = orc.num_threads()
    band = np.ascontiguousarray(x_full[:, :, :rows, :])
    for _ in range(2):
        run_model(spec.model, band)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        run_model(spec.model, band)
        times.append(time.perf_counter() - t0)
    dt = statistics.median(times)
    frac = rows / x_full.shape[2]
    cpu_model, phys = host_cpu()
    return {
        "value": round(frac / dt, 4),
        "unit": "frames/s",
        "cores": threads,
        "physical_cores": phys,
        "cpu_model": cpu_model,
        "kind": "port",
        "sample": (f"{spec.name} on a {rows}x{x_full.shape[3]} row band of the "
                   f"{x_full.shape[2]}x{x_full.shape[3]} frame ({frac:.1%} of a frame); "
                   f"2 warm-up runs, median of 5 timed runs ({', '.join(f'{t:.2f}' for t in times)} s); "
                   f"C oracle, fp32 math + fp16 storage per node, OpenMP on {threads} threads; "
                   f"frames/s = band fraction / time"),
    }


def torch_cpu_runner(model, x):
    """A callable that evaluates `model` (an arthip_amd.onnx_proto Model of the
    conv-chain ops) on NCHW input x with torch's CPU kernels, fp32 throughout,
    and returns the output tensor."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    g = model.graph
    consts = {t.name: torch.from_numpy(t.to_numpy().astype(np.float32)) for t in g.initializers}
    inp = next(v for v in g.inputs if v.name not in consts)
    xin = torch.from_numpy(np.ascontiguousarray(x).astype(np.float32))

    def run():
        vals = {inp.name: xin}
        for n in g.nodes:
            a, t = n.inputs, n.op_type
            if t == "Conv":
                b = consts[a[2]] if len(a) > 2 and a[2] else None
                y = F.conv2d(vals[a[0]], consts[a[1]], b, padding=1)
            elif t == "Relu":
                y = torch.relu(vals[a[0]])
            elif t == "Sigmoid":
                y = torch.sigmoid(vals[a[0]])
            elif t in ("Add", "Mul"):
                u, v = (vals[k] if k in vals else consts[k] for k in a[:2])
                y = u + v if t == "Add" else u * v
            elif t == "Clip":
                lo = consts[a[1]].item() if len(a) > 1 and a[1] else None
                hi = consts[a[2]].item() if len(a) > 2 and a[2] else None
                y = torch.clamp(vals[a[0]], lo, hi)
            elif t == "DepthToSpace":
                bs = int(n.attr("blocksize"))
                v = vals[a[0]]
                N, C, H, W = v.shape
                y = (v.reshape(N, bs, bs, C // (bs * bs), H, W).permute(0, 3, 4, 1, 5, 2)
                     .reshape(N, C // (bs * bs), H * bs, W * bs))
            elif t == "Cast":
                y = vals[a[0]]
            else:
                raise NotImplementedError(t)
            vals[n.outputs[0]] = y
        return vals[g.outputs[0].name]

    return run


def cpu_library(spec, x_full, rows: int) -> dict | None:
    """The same band through torch's CPU conv2d (oneDNN) in fp32, all host
    threads: what an optimized CPU library reaches on this model, for scale
    beside the oracle figure (ONNX Runtime, whose CPU EP would be the reference's
    own baseline, is not installed). Two warm-up runs, the median of five."""
    if rows <= 0:
        return None
    import statistics

    import torch

    run = torch_cpu_runner(spec.model, x_full[:, :, :rows, :])
    with torch.inference_mode():
        for _ in range(2):
            run()
        times = []
        for _ in range(5):
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
    dt = statistics.median(times)
    frac = rows / x_full.shape[2]
    return {
        "value": round(frac / dt, 4),
        "unit": "frames/s",
        "threads": torch.get_num_threads(),
        "what": (f"torch {torch.__version__} CPU conv2d (oneDNN), fp32 throughout, on the same "
                 f"{rows}-row band; median of 5 runs ({', '.join(f'{t:.3f}' for t in times)} s)"),
    }


def host_path_wall(spec, h: int, w: int, streams: int, warmup: int, steps: int) -> float:
    """Seconds for `steps` frames through arthip_vs_model_get_frame: fp16 planes
    in host memory (GRAYH), copied to pinned staging, uploaded, run, downloaded
    and copied into the caller's output plane, from streams + 1 threads over a
    pool of `streams` engines."""
    import threading

    from arthip_amd import models, vs
    from arthip_amd import onnx_proto as op

    frame = models.synthetic_input((1, 1, h, w), seed=1)[0, 0]
    threads = streams + 1
    with vs.Model("GRAYH", w, h, op.encode_model(spec.model), num_streams=streams) as m:
        for _ in range(max(warmup, threads)):
            m.get_frame([frame])
        counter = iter(range(steps))
        lock = threading.Lock()

        def work():
            while True:
                with lock:
                    if next(counter, None) is None:
                        return
                m.get_frame([frame])

        pool = [threading.Thread(target=work) for _ in range(threads)]
        t0 = time.perf_counter()
        for t in pool:
            t.start()
        for t in pool:
            t.join()
        return time.perf_counter() - t0


def host_path(args) -> int:
    """The VapourSynth filter path's frame rate as a JSON line of its own."""
    from arthip_amd import models

    builder = {"r8f64": models.r8f64, "r16f96": models.r16f96, "c4f32": models.c4f32,
               "shipped_like": models.shipped_like}[args.model]
    spec = builder(seed=0)
    h, w = args.height, args.width
    streams = args.host_path
    wall = host_path_wall(spec, h, w, streams, args.warmup, args.steps)
    print(json.dumps({
        "metric": f"frames/sec @{w}x{h} {spec.name} through the VapourSynth filter path "
                  "(host planes in and out, PCIe included)",
        "value": round(args.steps / wall, 3), "unit": "frames/s", "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(1000 * wall / args.steps, 4),
        "num_streams": streams, "threads": streams + 1, "clip_format": "GRAYH",
        "data": "synthetic (seeded He-normal fp16 weights, uniform[0,1) luma)",
    }), flush=True)
    return 0


def end_to_end(spec, eng, x_host, frames: int, vs_frames: int) -> dict:
    """Frame rates with host buffers (PCIe included), beside the device-resident
    value: the engine's own Run (pinned staging, upload, run, download, one
    engine, synchronous) and the VapourSynth filter path with two engines and
    three caller threads (transfers of one frame overlap another's run; timed
    over vs_frames after 20 warm-up frames, since a new filter's first frames
    run slower)."""
    t0 = time.perf_counter()
    for _ in range(frames):
        eng.run(x_host)
    sync_fps = frames / (time.perf_counter() - t0)
    n, _, h, w = x_host.shape
    out = {"engine_run_fps": round(n * sync_fps, 3),
           "engine_run_what": f"arthip_engine_run host->host, one engine, {frames} frames"}
    if spec.in_channels == 1 and n == 1:
        # In its own process, as a VapourSynth host runs it: in this process,
        # after the device-resident passes, the same measurement reads ~12%
        # lower (468-490 against 548 frames/s on one box).
        # A side figure: a failure is reported in the line, never fatal to it.
        import subprocess
        cmd = [sys.executable, str(Path(__file__).resolve()), "--host-path", "2", "--model",
               spec.name, "--height", str(h), "--width", str(w), "--steps", str(vs_frames),
               "--warmup", "20"]
        out["vs_filter_what"] = (f"VapourSynth filter core (GRAYH planes in host memory) in a "
                                 f"process of its own, num_streams=2, 3 caller threads, "
                                 f"{vs_frames} frames after 20")
        try:
            res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
            if res.returncode != 0:
                raise RuntimeError(f"exit {res.returncode}: {res.stderr.strip()[-300:]}")
            out["vs_filter_fps"] = json.loads(res.stdout.strip().splitlines()[-1])["value"]
        except (OSError, RuntimeError, ValueError, KeyError, IndexError,
                subprocess.TimeoutExpired) as exc:
            out["vs_filter_fps"] = None
            out["vs_filter_error"] = str(exc)
    return out


def stream_copy_gbs(nbytes: int, reps: int = 20) -> float:
    """Read + write GB/s of a device-to-device copy of nbytes (best of reps)."""
    import torch
    n = nbytes // 2
    a = torch.ones(n, dtype=torch.float16, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        b.copy_(a)
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) / 1000.0)
    del a, b
    return 2.0 * n * 2 / best / 1e9


def profile_launches(key: str):
    """Per-launch figures of one frame of workload `key` from the committed
    rocprofv3 summary (profiles/traffic.json), or None."""
    f = REPO / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get(key, {}).get("launches")
    except (OSError, ValueError):
        return None


def launch_work(spec, steps, px: int):
    """Algorithmic bytes and flops of each engine launch of one frame, in launch
    order (the engine's profile step names): a conv step takes the next conv of
    the model, a fused block step the next two. Bytes: every distinct tensor the
    launch reads or writes, fp16, once (input, residual inputs, output; the
    boundary input / output of the head / tail at their own sizes), plus fp16
    weights. A fused block whose residual input is its own input tensor (every
    R8F64 block) reads that tensor once: 531 MB at 1080p, not 796."""
    convs = list(zip(spec.convs, spec.skips_per_conv))
    ci = 0
    out = []
    for name in steps:
        if name.startswith("winograd_block"):
            (c1, m1), _ = convs[ci]
            (c2, m2), nsk = convs[ci + 1]
            if spec.conv_inputs is not None:
                block_in = spec.conv_inputs[ci]
                nsk = sum(1 for t in spec.skip_names[ci + 1] if t != block_in)
            ci += 2
            b = 2.0 * px * (c1 + m2 * (1 + nsk)) + 18.0 * (c1 * m1 + c2 * m2)
            fd = 2.0 * 9 * px * (c1 * m1 + c2 * m2)
            # The fused block runs F(2,3) along x, the kernel rows direct: 6 of
            # the 9 products per output and channel pair.
            out.append({"bytes": b, "flops_direct": fd, "flops_wino": fd * 6 / 9, "convs": 2})
        elif name.startswith(("winograd_conv", "direct_conv")):
            (c, m), nsk = convs[ci]
            ci += 1
            b = 2.0 * px * (c + m * (1 + nsk)) + 18.0 * c * m
            fd = 2.0 * 9 * px * c * m
            # The row pipes run the fused block's row scheme (6/9 of direct): a
            # lone 64 -> 64 conv without residual inputs, a 96 -> 96 conv with
            # at most one. Other convs F(2x2,3x3) (16/36).
            rows = (c == m == 64 and nsk == 0) or (c == m == 96 and nsk <= 1)
            fw = fd if c == 1 else fd * 6 / 9 if rows else fd * 16 / 36
            out.append({"bytes": b, "flops_direct": fd, "flops_wino": fw, "convs": 1})
        else:
            out.append(None)
    return out


def frame_bytes(spec, work, n, h, w, oshape, roofline) -> dict:
    """HBM bytes of one frame three ways: every conv launched alone
    (layer-at-a-time), the launches as the engine runs them (each distinct tensor
    a launch touches once), and the fused lower bound (the frame's boundary
    input and output plus the weights: what an engine keeping every
    intermediate on chip would move)."""
    weights = sum(18.0 * c * m for c, m in spec.convs)
    lower = 2.0 * n * h * w * spec.in_channels + 2.0 * oshape[0] * oshape[1] * oshape[2] * oshape[3] + weights
    out = {"layer_at_a_time": round(work["bytes"]), "fused_lower_bound": round(lower)}
    if roofline:
        per_launch = sum(k["alg_bytes"] * k["launches_per_frame"] for k in roofline["kernels"])
        out["as_launched"] = round(per_launch)
        meas = [k.get("hbm_bytes_measured") for k in roofline["kernels"]]
        if all(m is not None for m in meas):
            out["measured"] = round(sum(m * k["launches_per_frame"]
                                        for m, k in zip(meas, roofline["kernels"])))
    return out


def summarize_profile(args) -> int:
    """Per-launch figures of one frame from rocprofv3 csv output (see
    --summarize-profile). Engine kernels (namespace arthip) only: every frame of
    the trace run is averaged per launch index, and each counter per launch
    index over the frames of its run."""
    import csv
    import statistics

    d = Path(args.summarize_profile)

    def rows(sub, pattern):
        files = sorted((d / sub).rglob(pattern))
        if not files:
            return []
        with open(files[0], newline="") as f:
            return list(csv.DictReader(f))

    def engine(name):
        return "arthip::" in name

    def short(name):
        n = name.split("(")[0].replace("void ", "").replace("arthip::", "")
        return n.strip()

    trace = [r for r in rows("kt", "*kernel_trace.csv") if engine(r["Kernel_Name"])]
    trace.sort(key=lambda r: int(r["Start_Timestamp"]))
    frames = args.frames
    if not trace or frames <= 0 or len(trace) % frames:
        print(f"summarize: {len(trace)} engine dispatches do not split into {frames} frames",
              file=sys.stderr)
        return 1
    per = len(trace) // frames
    timed = trace[per * args.skip_frames:]
    launches = []
    for i in range(per):
        ts = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
              for r in timed[i::per]]
        launches.append({"kernel": short(trace[i]["Kernel_Name"]),
                         "trace_mean_us": round(statistics.mean(ts), 2),
                         "trace_median_us": round(statistics.median(ts), 2)})

    def counter(sub, name):
        rs = [r for r in rows(sub, "*counter_collection.csv")
              if engine(r["Kernel_Name"]) and r["Counter_Name"] == name]
        rs.sort(key=lambda r: int(r["Dispatch_Id"]))
        if not rs or len(rs) % per:
            return None
        return [statistics.mean(float(r["Counter_Value"]) for r in rs[i::per])
                for i in range(per)]

    def cal(sub, name):
        rs = [r for r in rows(sub, "*counter_collection.csv")
              if "copy" in r["Kernel_Name"].lower() and r["Counter_Name"] == name]
        return statistics.median(float(r["Counter_Value"]) for r in rs) if rs else None

    fetch, write = counter("fetch", "FETCH_SIZE"), counter("write", "WRITE_SIZE")
    cal_bytes = args.calibrate_copy * (1 << 20) if args.calibrate_copy else 512 * (1 << 20)
    cf, cw = cal("cal_fetch", "FETCH_SIZE"), cal("cal_write", "WRITE_SIZE")
    fscale = cal_bytes / (cf * 1024) if cf else None
    wscale = cal_bytes / (cw * 1024) if cw else None
    if fetch and write and fscale and wscale:
        for i, L in enumerate(launches):
            L["read_bytes"] = round(fetch[i] * 1024 * fscale)
            L["write_bytes"] = round(write[i] * 1024 * wscale)
            L["hbm_bytes"] = L["read_bytes"] + L["write_bytes"]
    # SQ counter passes (MFMA, VALU, LDS, waits), averaged per kernel name.
    sq = {}
    # Effective shader clock of each dispatch of the counter passes:
    # GRBM_GUI_ACTIVE (GPU busy cycles, summed over the 8 XCDs) over the
    # dispatch's own start / end timestamps (ns).
    clock = {}
    for sub in ("p1", "p2"):
        for r in rows(sub, "*counter_collection.csv"):
            if engine(r["Kernel_Name"]):
                k = short(r["Kernel_Name"])
                sq.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(
                    float(r["Counter_Value"]))
                if r["Counter_Name"] == "GRBM_GUI_ACTIVE" and r.get("End_Timestamp"):
                    ns = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                    if ns > 0:
                        clock.setdefault(k, []).append((ns / 1000.0,
                                                        float(r["Counter_Value"]) / 8 / ns * 1000.0))
    summary = {"launches": launches, "fetch_scale": fscale, "write_scale": wscale,
               "frames": frames}
    if args.profile_json:
        f = Path(args.profile_json)
        data = json.loads(f.read_text()) if f.exists() else {}
        data[args.profile_key] = summary
        f.write_text(json.dumps(data, indent=1) + "\n")
    print(f"| # | kernel | trace mean us | HBM read MB | HBM write MB |")
    print("|---|---|---|---|---|")
    for i, L in enumerate(launches):
        print(f"| {i} | `{L['kernel']}` | {L['trace_mean_us']} | "
              f"{L.get('read_bytes', 0) / 1e6:.1f} | {L.get('write_bytes', 0) / 1e6:.1f} |")
    print(f"\nframe: {sum(L['trace_mean_us'] for L in launches):.1f} us of kernels "
          f"({per} launches, mean over {frames - args.skip_frames} frames); "
          f"FETCH scale {fscale:.4f}, WRITE scale {wscale:.4f} (plain copy calibration)")
    if clock:
        print("\n| kernel | dispatch us (counter passes) | shader clock MHz (GRBM_GUI_ACTIVE / 8 / duration) |")
        print("|---|---|---|")
        for k in dict.fromkeys(L["kernel"] for L in launches):
            if k in clock:
                print(f"| `{k}` | {statistics.mean(d for d, _ in clock[k]):.1f} | "
                      f"{statistics.mean(m for _, m in clock[k]):.0f} |")
        summary["clock_mhz"] = {k: round(statistics.mean(m for _, m in v)) for k, v in clock.items()}
        if args.profile_json:
            f = Path(args.profile_json)
            data = json.loads(f.read_text())
            data[args.profile_key] = summary
            f.write_text(json.dumps(data, indent=1) + "\n")
    if sq:
        def av(k, c):
            v = sq[k].get(c)
            return statistics.mean(v) if v else float("nan")
        print("\n| kernel | trace us | MFMA util % | F16 MFMA GFLOP | LDS active % | "
              "LDS bank conflicts | waiting % | VALU instr (M) | MFMA instr (M) | LDS instr (M) |")
        print("|---|---|---|---|---|---|---|---|---|---|")
        for k in dict.fromkeys(L["kernel"] for L in launches):
            if k not in sq:
                continue
            gui = av(k, "GRBM_GUI_ACTIVE") / 8  # summed over the 8 XCDs
            simds, cus = 1024, 256
            mfma = av(k, "SQ_VALU_MFMA_BUSY_CYCLES") / (gui * simds) * 100
            lds_act = av(k, "SQ_LDS_IDX_ACTIVE") / (gui * cus) * 100
            conf = av(k, "SQ_LDS_BANK_CONFLICT")
            conf_ratio = conf / max(av(k, "SQ_LDS_IDX_ACTIVE") - conf, 1.0)
            wait = av(k, "SQ_WAIT_ANY") / av(k, "SQ_WAVE_CYCLES") * 100
            tus = statistics.mean(L["trace_mean_us"] for L in launches if L["kernel"] == k)
            print(f"| `{k}` | {tus:.1f} | {mfma:.1f} | "
                  f"{av(k, 'SQ_INSTS_VALU_MFMA_MOPS_F16') * 512 / 1e9:.1f} | {lds_act:.1f} | "
                  f"{conf_ratio:.3f} | {wait:.0f} | {av(k, 'SQ_INSTS_VALU') / 1e6:.2f} | "
                  f"{av(k, 'SQ_INSTS_MFMA') / 1e6:.2f} | {av(k, 'SQ_INSTS_LDS') / 1e6:.2f} |")
    return 0


def main() -> int:
    args = parse()
    if args.summarize_profile:
        return summarize_profile(args)
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy, args.steps)
    if args.host_path:
        return host_path(args)
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only; --gpus {args.gpus} is not supported "
              "(frames are independent: several GPUs would each run whole frames)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from arthip_amd import models
    from arthip_amd.engine import Engine

    builder = {"r8f64": models.r8f64, "r16f96": models.r16f96, "c4f32": models.c4f32,
               "shipped_like": models.shipped_like, "single64": models.single64}[args.model]
    spec = builder(seed=0)
    n, h, w = args.batch, args.height, args.width
    x_host = models.synthetic_input((n, spec.in_channels, h, w), seed=1,
                                    kind="normal" if spec.in_channels > 1 else "uniform")

    eng = Engine(0).build(spec)
    oshape = eng.output_shape(x_host.shape)
    dev = torch.device("cuda")
    x = torch.from_numpy(x_host).to(dev)
    y = torch.empty(oshape, dtype=torch.float16, device=dev)
    stream = torch.cuda.Stream()  # default priority
    sh = stream.cuda_stream

    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            eng.run_device(x, y, sh)
    torch.cuda.synchronize()

    # Timed region: K frames, no per-launch instrumentation.
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(args.steps):
            eng.run_device(x, y, sh)
        stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = gpu_ms / args.steps
    fps = n * args.steps / (gpu_ms / 1000.0)

    work = models.work_per_frame(spec, n, h, w)
    roofline = None
    steps_report = []
    profile = not args.no_profile
    if profile:
        # A second pass of K frames with HIP events around every launch (on the
        # launch stream) for the per-kernel figures behind `roofline`.
        eng.set_profiling(True)
        eng.profile_read()  # reset counters
        with torch.cuda.stream(stream):
            for _ in range(args.steps):
                eng.run_device(x, y, sh)
        torch.cuda.synchronize()
        prof = eng.profile_read()
        eng.set_profiling(False)
        names = [name for name, _, _ in prof]
        lw = launch_work(spec, names, n * h * w)
        key = f"{args.model}_{h}x{w}" + (f"_b{n}" if n > 1 else "")
        measured = profile_launches(key)
        if measured is not None and len(measured) != len(prof):
            measured = None  # a different plan than the one profiled
        kinds = {}
        for i, ((name, ms, cnt), work_i) in enumerate(zip(prof, lw)):
            mean_us = 1000.0 * ms / max(cnt, 1)
            entry = {"step": name, "mean_us": round(mean_us, 2), "launches": cnt}
            if work_i:
                entry.update({"alg_bytes": round(work_i["bytes"]),
                              "gbs": round(work_i["bytes"] / mean_us / 1e3, 1),
                              "tflops_direct": round(work_i["flops_direct"] / mean_us / 1e6, 1)})
            m = measured[i] if measured else None
            if m:
                entry["kernel"] = m["kernel"]
                entry["trace_mean_us"] = m.get("trace_mean_us")
                if "hbm_bytes" in m:
                    entry["hbm_bytes"] = m["hbm_bytes"]
            steps_report.append(entry)
            if work_i:
                k = name.split(" [")[0]
                agg = kinds.setdefault(k, {"ms": 0.0, "launches": 0, "bytes": 0.0, "fd": 0.0,
                                           "fw": 0.0, "trace_us": 0.0, "hbm": 0.0,
                                           "n_meas": 0, "kernel": None})
                agg["ms"] += ms
                agg["launches"] += cnt
                agg["bytes"] += work_i["bytes"] * cnt
                agg["fd"] += work_i["flops_direct"] * cnt
                agg["fw"] += work_i["flops_wino"] * cnt
                if m and "hbm_bytes" in m:
                    agg["trace_us"] += m["trace_mean_us"]
                    agg["hbm"] += m["hbm_bytes"]
                    agg["n_meas"] += 1
                    agg["kernel"] = m["kernel"]
        table = []
        for k, a in kinds.items():
            mean_s = a["ms"] / 1000.0 / max(a["launches"], 1)
            per_b = a["bytes"] / max(a["launches"], 1)
            per_fd = a["fd"] / max(a["launches"], 1)
            per_fw = a["fw"] / max(a["launches"], 1)
            row = {"step": k, "kernel": a["kernel"], "launches_per_frame": a["launches"] // args.steps,
                   "mean_us": round(mean_s * 1e6, 2),
                   "alg_bytes": round(per_b), "alg_gbs": round(per_b / mean_s / 1e9, 1),
                   "hbm_frac": round(per_b / mean_s / 1e9 / HBM_PEAK_GBS, 4),
                   "tflops_direct": round(per_fd / mean_s / 1e12, 1),
                   "mfma_frac_direct": round(per_fd / mean_s / 1e12 / MFMA_FP16_PEAK_TFLOPS, 4),
                   "tflops_winograd": round(per_fw / mean_s / 1e12, 1)}
            if a["n_meas"]:
                tr = a["trace_us"] / a["n_meas"]
                row["trace_mean_us"] = round(tr, 2)
                row["hbm_bytes_measured"] = round(a["hbm"] / a["n_meas"])
                row["traffic_ratio"] = round(a["hbm"] / a["n_meas"] / per_b, 3)
            table.append(row)
        # Dominant kernel: the kind with the most time per frame.
        dom = max(table, key=lambda r: r["mean_us"] * r["launches_per_frame"]) if table else None
        if dom:
            a = kinds[dom["step"]]
            mean_s = a["ms"] / 1000.0 / a["launches"]
            per_b = a["bytes"] / a["launches"]
            per_fd = a["fd"] / a["launches"]
            intensity = per_fd / per_b
            ridge = MFMA_FP16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
            copy_gbs = stream_copy_gbs(2 * n * h * w * 64)
            if intensity > ridge:
                achieved, peak, unit, bound = per_fd / mean_s / 1e12, MFMA_FP16_PEAK_TFLOPS, "TFLOP/s", "mfma"
            else:
                achieved, peak, unit, bound = per_b / mean_s / 1e9, HBM_PEAK_GBS, "GB/s", "hbm"
            roofline = {
                "bound": bound,
                "kernel": dom["kernel"] or dom["step"],
                "achieved": round(achieved, 1),
                "peak": peak,
                "unit": unit,
                "frac": round(achieved / peak, 4),
                "traffic": dom.get("hbm_bytes_measured"),
                "mean_launch_us": round(mean_s * 1e6, 2),
                "trace_mean_launch_us": dom.get("trace_mean_us"),
                "frac_from_trace": (round(achieved * mean_s * 1e6 / dom["trace_mean_us"] / peak, 4)
                                    if dom.get("trace_mean_us") else None),
                "launches": a["launches"],
                "alg_bytes_per_launch": round(per_b),
                "alg_flops_direct_per_launch": round(per_fd),
                "intensity_flop_per_byte": round(intensity, 1),
                "ridge_flop_per_byte": round(ridge, 1),
                "hbm_gbs_alg": round(per_b / mean_s / 1e9, 1),
                "tflops_winograd_executed": round(a["fw"] / a["launches"] / mean_s / 1e12, 1),
                "stream_copy_gbs": round(copy_gbs, 1),
                "kernels": table,
            }

    # Host-buffer rates (PCIe included): reported beside the device-resident value.
    e2e = (end_to_end(spec, eng, x_host, max(4, min(args.steps, 40)), max(4, min(2 * args.steps, 200)))
           if not args.no_e2e else None)

    rows = args.cpu_rows
    if rows < 0:
        rows = {"r8f64": 80, "shipped_like": 56, "r16f96": 16}.get(args.model, h)
    cpu = cpu_baseline(spec, x_host, min(rows, h)) if rows else None
    cpu_lib = cpu_library(spec, x_host, min(rows, h)) if rows else None

    tflops_direct = work["flops_direct"] * fps / n / 1e12
    line = {
        "metric": ("frames/sec @1920x1080 ArtCNN-style R8F64 fp16; % of fp16 MFMA peak"
                   if (args.model, h, w) == ("r8f64", 1080, 1920) else
                   f"frames/sec @{w}x{h} one fp16 conv3x3 64->64 + bias + ReLU; % of fp16 MFMA peak"
                   if args.model == "single64" else
                   f"frames/sec @{w}x{h} ArtCNN-style {spec.name} fp16; % of fp16 MFMA peak"),
        "value": round(fps, 3),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": ("synthetic (seeded He-normal fp16 weights, uniform(-0.1, 0.1) bias, "
                 "N(0, 0.5) 64-channel input)" if args.model == "single64" else
                 "synthetic (seeded He-normal fp16 weights, zero bias, uniform[0,1) luma)"),
        "config": {"workload": (f"{spec.name} {'2x luma upscale ' if spec.scale == 2 else ''}"
                                f"{n}x{spec.in_channels}x{h}x{w} fp16 -> "
                                f"{oshape[0]}x{oshape[1]}x{oshape[2]}x{oshape[3]}"),
                   "global_batch": n, "height": h, "width": w},
        "mfma_frac_direct_equiv": round(tflops_direct / MFMA_FP16_PEAK_TFLOPS, 4),
        "tflops_direct_equiv": round(tflops_direct, 2),
        "tflops_winograd": round(work["flops_wino"] * fps / n / 1e12, 2),
        "hbm_gbs_layer_at_a_time": round(work["bytes"] * fps / n / 1e9, 1),
        "frame_bytes": frame_bytes(spec, work, n, h, w, oshape, roofline),
        "end_to_end": e2e,
        "wall_s": round(wall, 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_library": cpu_lib,
    }
    if os.environ.get("ARTHIP_BENCH_STEPS_REPORT"):
        line["steps_report"] = steps_report
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
