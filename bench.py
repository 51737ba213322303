#!/usr/bin/env python3
"""Benchmark of the libstrict_hip kernel path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A "step" is one pass of the hot path over one batch of synthetic input that is
already resident in HBM. The default workload is BASELINE configs[1]: a
4096x4096 RGBA8 image, AdjustBrightness(+40) then the 5x5 box blur
(clamp-to-edge, (sum+12)/25), run as the fused brightness+blur kernel. The
other kernels of the path (sigmoid 2^24, brightness alone, blur alone, the
unfused two-kernel pipeline) are timed the same way and listed under
"kernels".

Timing: HIP events recorded on the library context's own stream around every
launch of the timed region (the kernels run on that stream, not torch's).
Inputs rotate over >= 1 GiB of buffers so the 256 MB MALL cannot serve
repeats. Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published
GEMM_N = 4096
IMG_W = IMG_H = 4096
IMG_BYTES = IMG_W * IMG_H * 4
SIGMOID_N = 1 << 24
ROTATE_BYTES = 1 << 30


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default="image",
                   choices=["image", "sigmoid"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="approximate CPU time budget of the cpu_baseline sample")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Rotation:
    """R input/output pairs covering >= 1 GiB, cycled per launch."""

    def __init__(self, ctx, host_in: np.ndarray, out_dtype, out_shape):
        pair = host_in.nbytes + int(np.prod(out_shape)) * np.dtype(out_dtype).itemsize
        self.n = max(2, -(-ROTATE_BYTES // pair))
        self.ins = [ctx.upload(host_in) for _ in range(self.n)]
        self.outs = [ctx.empty(out_shape, out_dtype) for _ in range(self.n)]

    def __getitem__(self, k):
        return self.ins[k % self.n], self.outs[k % self.n]

    def free(self):
        for v in self.ins + self.outs:
            v.free()


def time_launches(ctx, launch, steps: int, warmup: int):
    """Runs `launch(k)` warmup + steps times on the context stream.

    Two HIP events bracket the `steps` timed launches, recorded on the
    library's stream (where the kernels run) right after the warmup launches
    are queued, so the device is already busy when the start event fires and
    the timed launches run back to back. Returns (total_ms, avg_ms, wall_ms).
    """
    for k in range(warmup):
        launch(k)
    ctx.sync()
    lead = min(3, warmup)
    for k in range(lead):
        launch(k)
    start, stop = ctx.event(), ctx.event()
    t0 = time.perf_counter()
    start.record()
    for k in range(steps):
        launch(warmup + k)
    stop.record()
    ctx.sync()
    wall_ms = (time.perf_counter() - t0) * 1e3
    total = start.elapsed_ms(stop)
    start.destroy()
    stop.destroy()
    return total, total / steps, wall_ms


def kernel_entry(name, alg_bytes, avg_ms):
    gbs = alg_bytes / (avg_ms * 1e-3) / 1e9
    return {"kernel": name, "alg_bytes": alg_bytes, "avg_ms": round(avg_ms, 5),
            "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def read_traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    f = ROOT / "profiles" / f"{kernel}_traffic.txt"
    if not f.exists():
        return None
    vals = {}
    for line in f.read_text().splitlines():
        if ":" in line and line.split(":")[0].strip() in ("fetch_bytes_per_launch",
                                                          "write_bytes_per_launch"):
            k, v = line.split(":", 1)
            vals[k.strip()] = float(v.split()[0])
    if len(vals) != 2:
        return None
    return int(vals["fetch_bytes_per_launch"] + vals["write_bytes_per_launch"])


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline_image(seconds: float):
    import oracle

    img = np.random.default_rng(42).integers(0, 256, IMG_BYTES, dtype=np.uint8)
    nt = cpu_threads()
    reps, t_total = 0, 0.0
    while t_total < seconds and reps < 50:
        t0 = time.perf_counter()
        oracle.brightness_blur5_config(img, IMG_W, IMG_H, 40, 4, nthreads=nt)
        t_total += time.perf_counter() - t0
        reps += 1
    gbs = 2 * IMG_BYTES * reps / t_total / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": nt, "kind": "port",
            "sample": f"{reps} x fused brightness(+40)+5x5 blur on the 4096x4096 RGBA8 config "
                      f"image, C restatement (oracle/oracle.c) over {nt} threads, "
                      f"{t_total:.1f} s wall"}


def cpu_baseline_sigmoid(seconds: float):
    import oracle

    x = np.random.default_rng(42).uniform(-8, 8, SIGMOID_N).astype(np.float32)
    nt = cpu_threads()
    reps, t_total = 0, 0.0
    while t_total < seconds and reps < 50:
        t0 = time.perf_counter()
        oracle.sigmoid_f32(x, nthreads=nt)
        t_total += time.perf_counter() - t0
        reps += 1
    gbs = 8 * SIGMOID_N * reps / t_total / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": nt, "kind": "port",
            "sample": f"{reps} x sigmoid over 2^24 floats (SigmoidPerformanceTests.cs:27 "
                      f"restated in C, double exp) over {nt} threads, {t_total:.1f} s wall"}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box of this build has one MI355X, and the "
              f"kernel path has no multi-GPU leg (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2

    import strict_amd

    ctx = strict_amd.Context(0)
    info = ctx.info()
    log(f"device {info['name']} {info['arch']} CUs={info['compute_units']}")

    kernels = []
    rng = np.random.default_rng(42)

    # -- image kernels --
    img = rng.integers(0, 256, IMG_BYTES, dtype=np.uint8)
    rot = Rotation(ctx, img, np.uint8, (IMG_BYTES,))
    log(f"image buffers: {rot.n} pairs")

    def fused(k):
        s, d = rot[k]
        ctx.brightness_blur5(s, d, IMG_W, IMG_H, 4, 40 if k % 2 == 0 else -40, 0,
                             strict_amd.BLUR_CONFIG)

    def brightness(k):
        s, d = rot[k]
        ctx.adjust_brightness(s, d, IMG_W, IMG_H, 4, 40 if k % 2 == 0 else -40, 0)

    def blur(k):
        s, d = rot[k]
        ctx.box_blur5(s, d, IMG_W, IMG_H, 4, strict_amd.BLUR_CONFIG)

    def pipeline(k):
        s, d = rot[k]
        ctx.adjust_brightness(s, d, IMG_W, IMG_H, 4, 40, 0)
        s2, _ = rot[k + 1]
        ctx.box_blur5(d, s2, IMG_W, IMG_H, 4, strict_amd.BLUR_CONFIG)

    table_steps = max(20, min(args.steps, 100))
    results = {}
    def copy(k):
        s, d = rot[k]
        ctx.copy(d, s)

    for name, fn, alg in [("copy_u8 (HBM calibration)", copy, 2 * IMG_BYTES),
                          ("brightness_u8", brightness, 2 * IMG_BYTES),
                          ("box_blur5_u8", blur, 2 * IMG_BYTES),
                          ("brightness_then_blur_2_kernels", pipeline, 4 * IMG_BYTES)]:
        _, avg, _ = time_launches(ctx, fn, table_steps, 5)
        kernels.append(kernel_entry(name, alg, avg))
        log(f"{name}: {kernels[-1]}")

    # -- sigmoid --
    x = rng.uniform(-8, 8, SIGMOID_N).astype(np.float32)
    srot = Rotation(ctx, x, np.float32, (SIGMOID_N,))

    def sigmoid(k):
        s, d = srot[k]
        ctx.sigmoid(s, d, SIGMOID_N)

    # -- bf16 GEMM: compute-bound, operands reused across launches --
    ga = rng.normal(0, 0.02, (GEMM_N, GEMM_N)).astype(np.float32)
    gbits = (ga.view(np.uint32) + 0x7FFF + ((ga.view(np.uint32) >> 16) & 1)) >> 16
    dA = ctx.upload(gbits.astype(np.uint16))
    dB = ctx.upload(np.ascontiguousarray(gbits.T).astype(np.uint16))
    dC = ctx.empty((GEMM_N, GEMM_N), np.uint16)

    def gemm(k):
        ctx.gemm_bf16(dA, dB, dC, GEMM_N, GEMM_N, GEMM_N)

    _, gavg, _ = time_launches(ctx, gemm, 20, 3)
    gflop = 2.0 * GEMM_N ** 3
    tflops = gflop / (gavg * 1e-3) / 1e12
    kernels.append({"kernel": "gemm_bf16 4096^3", "alg_flop": gflop, "avg_ms": round(gavg, 5),
                    "TFLOP/s": round(tflops, 1),
                    "frac_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4)})
    log(f"gemm: {kernels[-1]}")
    for v in (dA, dB, dC):
        v.free()

    # -- the workload of the headline line --
    if args.workload == "image":
        total, avg, wall = time_launches(ctx, fused, args.steps, args.warmup)
        head = kernel_entry("brightness_blur5_u8 (fused)", 2 * IMG_BYTES, avg)
        _, savg, _ = time_launches(ctx, sigmoid, table_steps, 5)
        kernels.append(kernel_entry("sigmoid_f32", 8 * SIGMOID_N, savg))
        alg = 2 * IMG_BYTES
        workload = {"workload": "configs[1]: AdjustBrightness(+/-40) then 5x5 box blur "
                                "(clamp-to-edge, (sum+12)/25), fused, 4096x4096 RGBA8",
                    "width": IMG_W, "height": IMG_H, "channels": 4,
                    "alg_bytes_per_step": alg}
        dtype = "u8"
        traffic_kernel = "brightness_blur5_u8"
    else:
        total, avg, wall = time_launches(ctx, sigmoid, args.steps, args.warmup)
        head = kernel_entry("sigmoid_f32", 8 * SIGMOID_N, avg)
        _, favg, _ = time_launches(ctx, fused, table_steps, 5)
        kernels.append(kernel_entry("brightness_blur5_u8 (fused)", 2 * IMG_BYTES, favg))
        alg = 8 * SIGMOID_N
        workload = {"workload": "configs[0]: sigmoid fp32 over N=2^24 uniform[-8,8]",
                    "n": SIGMOID_N, "alg_bytes_per_step": alg}
        dtype = "f32"
        traffic_kernel = "sigmoid_f32"
    kernels.insert(0, head)
    log(f"headline: {head}")

    ms_per_step = total / args.steps
    value = alg / (ms_per_step * 1e-3) / 1e9
    achieved = head["GB/s"]
    roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": read_traffic(traffic_kernel)}

    rot.free()
    srot.free()
    ctx.dispose()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = (cpu_baseline_image if args.workload == "image" else cpu_baseline_sigmoid)(
            args.cpu_seconds)
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": "HBM GB/s (% peak) per kernel",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (numpy PCG64 seed 42), resident in HBM, rotated over >= 1 GiB",
        "config": workload,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "host_wall_ms": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
