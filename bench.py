#!/usr/bin/env python3
"""Frames/s of the ArtCNN-style R8F64 2x luma upscaler at 1920x1080 on one MI355X.

A step is one frame: a 1x1x1080x1920 fp16 luma frame already resident in HBM
goes through the whole engine (head conv, 8 residual blocks, global skip, tail
conv with fused DepthToSpace) to a 1x1x2160x3840 fp16 frame in HBM. W warmup
steps, then K timed steps bracketed by a device synchronize on both sides.
Prints one JSON line.

Extra objects in the line:
  roofline      the dominant kernel (winograd_conv 64->64): algorithmic bytes per
                launch (layer-at-a-time compulsory traffic: input + residual inputs
                + output, fp16) / its mean launch time, measured with HIP events on
                the launch stream over a second pass of K frames (the timed pass
                runs without per-launch events); against 8 TB/s HBM peak.
                traffic: HBM bytes per launch from the committed rocprofv3
                FETCH_SIZE/WRITE_SIZE summary (profiles/), when present.
                stream_copy_gbs: achievable HBM bandwidth on this device, a plain
                device copy (torch copy_) of one activation-sized buffer
                (265 MB read + 265 MB written), for reading `achieved` against
                what a streaming kernel reaches rather than only the 8 TB/s peak.
  cpu_baseline  the CPU oracle (oracle/, plain C + OpenMP, fp32 math with fp16
                storage between nodes) on a bounded band of the same frame on the
                host's cores, scaled to frames/s.
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
    p.add_argument("--model", default="r8f64", choices=["r8f64", "r16f96", "c4f32", "shipped_like"],
                   help="r8f64 (default, the headline workload); shipped_like: the shipped "
                        "luma model's architecture (SiLU, 3-conv blocks, Clip) with synthetic weights")
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--cpu-rows", type=int, default=360,
                   help="rows of the frame in the CPU baseline sample (0 disables it)")
    p.add_argument("--no-profile", action="store_true",
                   help="skip the per-launch event timing (roofline becomes null)")
    p.add_argument("--host-path", type=int, default=0, metavar="STREAMS",
                   help="instead of the device-resident bench, time the VapourSynth filter "
                        "path (host planes in and out, PCIe included) with STREAMS engines and "
                        "STREAMS + 1 caller threads; prints its own JSON line")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MB",
                   help="instead of the bench, run a plain device copy of MB megabytes "
                        "(--steps times): the known-traffic kernel that scales rocprofv3 "
                        "FETCH_SIZE / WRITE_SIZE readings")
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


def cpu_baseline(spec, x_full, rows: int) -> dict | None:
    """Times the C oracle on a band of `rows` input rows (full width)."""
    if rows <= 0:
        return None
    from oracle import ops as orc
    from oracle.model import run_model

    threads = orc.num_threads()
    band = x_full[:, :, :rows, :]
    run_model(spec.model, band[:, :, :8, :])  # warm the library and thread pool
    t0 = time.perf_counter()
    run_model(spec.model, band)
    dt = time.perf_counter() - t0
    frac = rows / x_full.shape[2]
    return {
        "value": round(frac / dt, 4),
        "unit": "frames/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{spec.name} on a {rows}x{x_full.shape[3]} row band of the "
                   f"{x_full.shape[2]}x{x_full.shape[3]} frame ({frac:.1%} of a frame, "
                   f"{dt:.1f} s), C oracle fp32 math + fp16 storage per node, OpenMP; "
                   f"frames/s = band fraction / time"),
    }


def host_path(args) -> int:
    """Frames/s through arthip_vs_model_get_frame: fp16 planes in host memory
    (GRAYH), copied to pinned staging, uploaded, run, downloaded and copied
    into the caller's output plane, from several threads over an engine pool."""
    import threading

    from arthip_amd import models, vs
    from arthip_amd import onnx_proto as op

    builder = {"r8f64": models.r8f64, "r16f96": models.r16f96, "c4f32": models.c4f32,
               "shipped_like": models.shipped_like}[args.model]
    spec = builder(seed=0)
    h, w = args.height, args.width
    frame = models.synthetic_input((1, 1, h, w), seed=1)[0, 0]
    streams = args.host_path
    threads = streams + 1
    with vs.Model("GRAYH", w, h, op.encode_model(spec.model), num_streams=streams) as m:
        for _ in range(max(args.warmup, threads)):
            m.get_frame([frame])
        counter = iter(range(args.steps))
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
        wall = time.perf_counter() - t0
    print(json.dumps({
        "metric": f"frames/sec @{w}x{h} {spec.name} through the VapourSynth filter path "
                  "(host planes in and out, PCIe included)",
        "value": round(args.steps / wall, 3), "unit": "frames/s", "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(1000 * wall / args.steps, 4),
        "num_streams": streams, "threads": threads, "clip_format": "GRAYH",
        "data": "synthetic (seeded He-normal fp16 weights, uniform[0,1) luma)",
    }), flush=True)
    return 0


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


def traffic_from_profiles(kernel_key: str):
    f = REPO / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        return d.get(kernel_key, {}).get("hbm_bytes_per_launch")
    except Exception:
        return None


def main() -> int:
    args = parse()
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
               "shipped_like": models.shipped_like}[args.model]
    spec = builder(seed=0)
    n, h, w = args.batch, args.height, args.width
    x_host = models.synthetic_input((n, 1, h, w), seed=1)

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
        # launch stream) for the per-kernel times behind `roofline`.
        eng.set_profiling(True)
        eng.profile_read()  # reset counters
        with torch.cuda.stream(stream):
            for _ in range(args.steps):
                eng.run_device(x, y, sh)
        torch.cuda.synchronize()
        prof = eng.profile_read()
        eng.set_profiling(False)
        # Per-step algorithmic bytes, in execution order of the conv steps.
        px = n * h * w
        conv_bytes = [2.0 * px * (ci + co * (1 + sk)) + 18.0 * ci * co
                      for (ci, co), sk in zip(spec.convs, spec.skips_per_conv)]
        conv_flops = [2.0 * 9 * ci * co * px for (ci, co) in spec.convs]
        ci = 0
        dom_ms = dom_bytes = dom_flops = 0.0
        dom_launches = 0
        for name, ms, cnt in prof:
            entry = {"step": name, "mean_us": round(1000 * ms / max(cnt, 1), 2), "launches": cnt}
            if name.startswith(("winograd_conv", "direct_conv")):
                entry["alg_bytes"] = conv_bytes[ci]
                if name.startswith("winograd_conv") and " C64 M64" in name or \
                   name.startswith("winograd_conv") and " C96 M96" in name:
                    dom_ms += ms
                    dom_bytes += conv_bytes[ci] * cnt
                    dom_flops += conv_flops[ci] * cnt
                    dom_launches += cnt
                ci += 1
            steps_report.append(entry)
        if dom_launches:
            mean_s = dom_ms / 1000.0 / dom_launches
            achieved = dom_bytes / dom_launches / mean_s / 1e9
            copy_gbs = stream_copy_gbs(2 * px * 64)
            roofline = {
                "bound": "hbm",
                "kernel": "winograd_conv (F(2x2,3x3), C=M=%d)" % spec.convs[1][0],
                "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS,
                "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic_from_profiles(f"{args.model}_{h}x{w}"),
                "mean_launch_us": round(mean_s * 1e6, 2),
                "launches": dom_launches,
                "alg_bytes_per_launch": round(dom_bytes / dom_launches),
                "mfma_frac_direct_equiv": round(dom_flops / dom_launches / mean_s / 1e12
                                                / MFMA_FP16_PEAK_TFLOPS, 4),
                "stream_copy_gbs": round(copy_gbs, 1),
                "frac_of_stream_copy": round(achieved / copy_gbs, 4),
            }

    cpu = cpu_baseline(spec, x_host, min(args.cpu_rows, h)) if args.cpu_rows else None

    tflops_direct = work["flops_direct"] * fps / n / 1e12
    line = {
        "metric": ("frames/sec @1920x1080 ArtCNN-style R8F64 fp16; % of fp16 MFMA peak"
                   if (args.model, h, w) == ("r8f64", 1080, 1920) else
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
        "data": "synthetic (seeded He-normal fp16 weights, zero bias, uniform[0,1) luma)",
        "config": {"workload": f"{spec.name} 2x luma upscale {n}x1x{h}x{w} fp16 -> "
                               f"{oshape[0]}x{oshape[1]}x{oshape[2]}x{oshape[3]}",
                   "global_batch": n, "height": h, "width": w},
        "mfma_frac_direct_equiv": round(tflops_direct / MFMA_FP16_PEAK_TFLOPS, 4),
        "tflops_direct_equiv": round(tflops_direct, 2),
        "tflops_winograd": round(work["flops_wino"] * fps / n / 1e12, 2),
        "hbm_gbs_layer_at_a_time": round(work["bytes"] * fps / n / 1e9, 1),
        "wall_s": round(wall, 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if os.environ.get("ARTHIP_BENCH_STEPS_REPORT"):
        line["steps_report"] = steps_report
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
