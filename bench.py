#!/usr/bin/env python3
"""Benchmark of the libstrict_hip kernel path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode|image|sigmoid]

BASELINE.json's metric is "HBM GB/s (% peak) per kernel; decode tokens/s
Qwen3-0.6B-shape FP8 b=1". The headline line (workload "decode") is
configs[4] at batch 1: a Qwen3-0.6B-shaped decoder with random FP8-E4M3
weights (per-output-channel fp32 scales), fp16 activations, a 4096-token KV
cache filled by a 4096-token random prompt, then K greedy decode steps timed
(a "step" = one token for every sequence). Its roofline is the step's
algorithmic bytes (weights + scales + norms + K/V of every cached position)
over the measured step time, against 8 TB/s.

Every other kernel of the path is timed the same way and listed under
"kernels" with its algorithmic GB/s (or TFLOP/s) and fraction of peak:
copy (HBM calibration), brightness, 5x5 blur, the fused brightness+blur of
configs[1], the unfused pipeline, sigmoid, the bf16 GEMM
(configs[2]), the FP8 GEMV at the LM-head shape, Qwen3 decode at b=4 and
b=16, GPT-2 decode.

Timing: two HIP events on the library context's stream (where the kernels
run) bracket K back-to-back launches after W warmup launches. Inputs of the
memory-bound kernels rotate over >= 1 GiB of buffers so the 256 MB MALL
cannot serve repeats. Prints ONE JSON line on stdout; progress on stderr.
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

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA, published
FP8_PEAK_TFLOPS = 5000.0    # MI355X dense fp8 MFMA, published
IMG_W = IMG_H = 4096
IMG_BYTES = IMG_W * IMG_H * 4
SIGMOID_N = 1 << 24
GEMM_N = 4096
ROTATE_BYTES = 1 << 30
KV_PROMPT = 4096


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=128)
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--workload", default="decode", choices=["decode", "image", "sigmoid"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true", help="skip the kernels table")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="approximate CPU time budget of the cpu_baseline sample")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class _Roctx:
    """roctxProfilerResume / roctxProfilerPause around each timed region, so
    that `rocprofv3 --selected-regions` records the timed launches only (the
    4096-step prompt fill of the decode workload is then left out of the
    trace). Without a profiler attached the calls do nothing."""

    def __init__(self):
        import ctypes

        self.lib = None
        for name in ("librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1"):
            try:
                self.lib = ctypes.CDLL(name)
                break
            except OSError:
                continue

    def resume(self) -> None:
        if self.lib is not None:
            self.lib.roctxProfilerResume(0)

    def pause(self) -> None:
        if self.lib is not None:
            self.lib.roctxProfilerPause(0)


PROFILER = _Roctx()


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
    PROFILER.resume()
    t0 = time.perf_counter()
    start.record()
    for k in range(steps):
        launch(warmup + k)
    stop.record()
    ctx.sync()
    wall_ms = (time.perf_counter() - t0) * 1e3
    PROFILER.pause()
    total = start.elapsed_ms(stop)
    start.destroy()
    stop.destroy()
    return total, total / steps, wall_ms


def hbm_entry(name, alg_bytes, avg_ms):
    gbs = alg_bytes / (avg_ms * 1e-3) / 1e9
    return {"kernel": name, "alg_bytes": int(alg_bytes), "avg_ms": round(avg_ms, 5),
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


def bf16_bits(a: np.ndarray) -> np.ndarray:
    u = a.astype(np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


# ---- GPU workloads -------------------------------------------------------------

def image_kernels(ctx, rng, steps):
    import strict_amd

    out = {}
    img = rng.integers(0, 256, IMG_BYTES, dtype=np.uint8)
    rot = Rotation(ctx, img, np.uint8, (IMG_BYTES,))

    def copy(k):
        s, d = rot[k]
        ctx.copy(d, s)

    def brightness(k):
        s, d = rot[k]
        ctx.adjust_brightness(s, d, IMG_W, IMG_H, 4, 40 if k % 2 == 0 else -40, 0)

    def blur(k):
        s, d = rot[k]
        ctx.box_blur5(s, d, IMG_W, IMG_H, 4, strict_amd.BLUR_CONFIG)

    def fused(k):
        s, d = rot[k]
        ctx.brightness_blur5(s, d, IMG_W, IMG_H, 4, 40 if k % 2 == 0 else -40, 0,
                             strict_amd.BLUR_CONFIG)

    def pipeline(k):
        s, d = rot[k]
        ctx.adjust_brightness(s, d, IMG_W, IMG_H, 4, 40, 0)
        s2, _ = rot[k + 1]
        ctx.box_blur5(d, s2, IMG_W, IMG_H, 4, strict_amd.BLUR_CONFIG)

    for name, fn, alg in [("copy_u8 (HBM calibration)", copy, 2 * IMG_BYTES),
                          ("brightness_u8", brightness, 2 * IMG_BYTES),
                          ("box_blur5_u8", blur, 2 * IMG_BYTES),
                          ("brightness_blur5_u8 (fused, configs[1])", fused, 2 * IMG_BYTES),
                          ("brightness_then_blur_2_kernels", pipeline, 4 * IMG_BYTES)]:
        total, avg, wall = time_launches(ctx, fn, steps, 5)
        out[name] = (hbm_entry(name, alg, avg), total, wall)
        log(f"{name}: {out[name][0]}")
    rot.free()
    return out


def sigmoid_kernel(ctx, rng, steps):
    x = rng.uniform(-8, 8, SIGMOID_N).astype(np.float32)
    rot = Rotation(ctx, x, np.float32, (SIGMOID_N,))

    def sigmoid(k):
        s, d = rot[k]
        ctx.sigmoid(s, d, SIGMOID_N)

    total, avg, wall = time_launches(ctx, sigmoid, steps, 5)
    rot.free()
    e = hbm_entry("sigmoid_f32 (configs[0])", 8 * SIGMOID_N, avg)
    log(f"sigmoid: {e}")
    return e, total, wall


def library_gemm_ms(ctx, gemm):
    """The same GEMM through hipBLASLt (strict_amd.yardstick, a library of its
    own that libstrict_hip does not link) as a yardstick for the hand-written
    kernel; None when hipBLASLt has no algorithm or the library is absent."""
    try:
        _, avg, _ = time_launches(ctx, gemm, 20, 3)
        return round(avg, 5)
    except Exception as exc:  # noqa: BLE001 -- a missing yardstick only drops this figure
        log(f"hipBLASLt GEMM: {exc}")
        return None


def gemm_kernel(ctx, rng):
    a = rng.normal(0, 0.02, (GEMM_N, GEMM_N)).astype(np.float32)
    b = rng.normal(0, 0.02, (GEMM_N, GEMM_N)).astype(np.float32)
    dA, dB = ctx.upload(bf16_bits(a)), ctx.upload(bf16_bits(b))
    dC = ctx.empty((GEMM_N, GEMM_N), np.uint16)

    def gemm(k):
        ctx.gemm_bf16(dA, dB, dC, GEMM_N, GEMM_N, GEMM_N)

    _, avg, _ = time_launches(ctx, gemm, 20, 3)

    def vendor(k):
        from strict_amd import yardstick

        yardstick.gemm_bf16(ctx, dA, dB, dC, GEMM_N, GEMM_N, GEMM_N)

    lib = library_gemm_ms(ctx, vendor)
    for v in (dA, dB, dC):
        v.free()
    flop = 2.0 * GEMM_N ** 3
    tflops = flop / (avg * 1e-3) / 1e12
    e = {"kernel": "gemm_bf16 4096^3 (configs[2])", "alg_flop": flop, "avg_ms": round(avg, 5),
         "TFLOP/s": round(tflops, 1), "frac_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
         "hipblaslt_avg_ms": lib}
    log(f"gemm: {e}")
    return e


def gemm_fp8_kernel(ctx, rng):
    """FP8 E4M3 GEMM 4096^3, per-row / per-column scales, bf16 output."""
    qa = rng.integers(0, 256, (GEMM_N, GEMM_N), dtype=np.uint8)
    qa[(qa & 0x7f) == 0x7f] = 0  # no NaN codes
    qb = rng.integers(0, 256, (GEMM_N, GEMM_N), dtype=np.uint8)
    qb[(qb & 0x7f) == 0x7f] = 0
    s = rng.uniform(0.5, 1.5, GEMM_N).astype(np.float32)
    dA, dB, dS = ctx.upload(qa), ctx.upload(qb), ctx.upload(s)
    dC = ctx.empty((GEMM_N, GEMM_N), np.uint16)

    def gemm(k):
        ctx.gemm_fp8(dA, dS, dB, dS, dC, GEMM_N, GEMM_N, GEMM_N)

    _, avg, _ = time_launches(ctx, gemm, 20, 3)

    def vendor(k):
        from strict_amd import yardstick

        yardstick.gemm_fp8(ctx, dA, dS, dB, dS, dC, GEMM_N, GEMM_N, GEMM_N)

    lib = library_gemm_ms(ctx, vendor)
    for v in (dA, dB, dS, dC):
        v.free()
    flop = 2.0 * GEMM_N ** 3
    tflops = flop / (avg * 1e-3) / 1e12
    e = {"kernel": "gemm_fp8 e4m3 4096^3, row/column scales", "alg_flop": flop,
         "avg_ms": round(avg, 5), "TFLOP/s": round(tflops, 1),
         "frac_fp8_peak": round(tflops / FP8_PEAK_TFLOPS, 4), "hipblaslt_avg_ms": lib}
    log(f"gemm_fp8: {e}")
    return e


def gemv_kernel(ctx, rng, steps):
    """FP8 W8A16 GEMV at the Qwen3 LM-head shape (151936 x 1024, b = 1)."""
    n, k = 151936, 1024
    q = rng.integers(0, 256, (n, k), dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0  # no NaN codes
    tiles = [ctx.empty((n * k,), np.uint8) for _ in range(-(-ROTATE_BYTES // (n * k)))]
    dq = ctx.upload(q)
    for t in tiles:
        ctx.pack_e4m3_tiles(dq, t, n, k)
    dq.free()
    ds = ctx.upload(np.full(n, 1e-3, np.float32))
    dx = ctx.upload(rng.normal(0, 1, (1, k)).astype(np.float16).view(np.uint16))
    dy = ctx.empty((1, n), np.float32)

    def gemv(j):
        ctx.gemv_w8a16(dx, tiles[j % len(tiles)], ds, dy, 1, k, n)

    _, avg, _ = time_launches(ctx, gemv, steps, 5)
    for v in tiles + [ds, dx, dy]:
        v.free()
    e = hbm_entry("gemv_w8a16 151936x1024 b=1 (LM head)", n * k + n * 4 + k * 2 + n * 4, avg)
    log(f"gemv: {e}")
    return e


def decode_run(ctx, cfg, batch, prompt_len, steps, warmup, seed=42):
    """Prefill `prompt_len` random tokens per sequence, then time `steps`
    greedy decode steps, enqueued back to back. Returns (ms_per_step, context_avg)."""
    from strict_amd import llm

    m = llm.Model(ctx, cfg)
    try:
        t0 = time.perf_counter()
        m.init_random(seed=seed, stddev=0.02)
        m.reset(batch)
        prompt = np.random.default_rng(seed).integers(0, cfg.vocab, (batch, prompt_len))
        for i in range(prompt_len):
            m.step(prompt[:, i], logits=(i == prompt_len - 1))
        for _ in range(warmup):
            m.step(None, logits=True)
        ctx.sync()
        log(f"decode b={batch}: init + {prompt_len}-token prefill + warmup in "
            f"{time.perf_counter() - t0:.1f} s")
        start, stop = ctx.event(), ctx.event()
        PROFILER.resume()
        start.record()
        for _ in range(steps):
            m.step(None, logits=True)
        stop.record()
        ctx.sync()
        PROFILER.pause()
        ms = start.elapsed_ms(stop) / steps
        start.destroy()
        stop.destroy()
        tokens = m.next_tokens()
        log(f"decode b={batch}: {ms:.4f} ms/step, last tokens {tokens[:4].tolist()}")
    finally:
        m.close()
    context_avg = prompt_len + warmup + (steps + 1) / 2.0
    return ms, context_avg


# ---- CPU baselines (the oracle, timed on this host) ------------------------

def cpu_baseline_decode(seconds: float):
    """numpy oracle of the Qwen3 configs[4] decode step at b = 1 on a 4096-token
    KV cache (random fp32 weights of the config's shapes, random K/V)."""
    import oracle.llm as ollm
    from strict_amd import llm

    cfg = llm.QWEN3_0_6B
    rng = np.random.default_rng(0)
    shapes = llm.linear_shapes(cfg)

    def mat(r, c):
        return rng.standard_normal((r, c), dtype=np.float32) * np.float32(0.02)

    t_build = time.perf_counter()
    layers = []
    for _ in range(cfg.layers):
        L = {}
        for name in ("qkv", "o", "gate_up", "down"):
            r, c = shapes[name]
            L[name] = mat(r, c)
            L[name + ".scale"] = np.ones(r, np.float32)
        for name in ("norm1.g", "norm2.g"):
            L[name] = np.ones(cfg.hidden, np.float32)
        L["q_norm"] = np.ones(cfg.head_dim, np.float32)
        L["k_norm"] = np.ones(cfg.head_dim, np.float32)
        layers.append(L)
    r, c = shapes["head"]
    w = ollm.Weights(cfg, layers, mat(r, c), np.ones(r, np.float32),
                     np.ones(cfg.hidden, np.float32),
                     inv_freq=ollm.inv_freq(cfg.rope_theta, cfg.head_dim))
    dec = ollm.Decoder(w)
    for li in range(cfg.layers):
        dec.k[li] = ollm.f16(rng.standard_normal((KV_PROMPT, cfg.kv_heads, cfg.head_dim),
                                                 dtype=np.float32))
        dec.v[li] = ollm.f16(rng.standard_normal((KV_PROMPT, cfg.kv_heads, cfg.head_dim),
                                                 dtype=np.float32))
    dec.pos = KV_PROMPT
    log(f"cpu baseline: oracle weights built in {time.perf_counter() - t_build:.1f} s")
    steps, t_total, tok = 0, 0.0, 1
    while t_total < seconds and steps < 64:
        t0 = time.perf_counter()
        tok = int(np.argmax(dec.forward([tok])[-1]))
        t_total += time.perf_counter() - t0
        steps += 1
    nt = cpu_threads()
    return {"value": round(steps / t_total, 3), "unit": "tokens/s", "cores": nt, "kind": "port",
            "sample": f"{steps} greedy decode steps of the numpy oracle (oracle/llm.py) of the "
                      f"configs[4] Qwen3 shape at b=1 on a {KV_PROMPT}-token KV cache, fp32 "
                      f"dequantized weights, BLAS over up to {nt} threads, {t_total:.1f} s"}


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
    from strict_amd import llm

    ctx = strict_amd.Context(0)
    info = ctx.info()
    log(f"device {info['name']} {info['arch']} CUs={info['compute_units']}")
    rng = np.random.default_rng(42)
    kernels = []
    table_steps = 50
    steps, warmup = args.steps, args.warmup

    if args.workload == "decode":
        cfg = llm.QWEN3_0_6B.with_(max_positions=KV_PROMPT + warmup + steps + 1, max_batch=1)
        ms, ctx_avg = decode_run(ctx, cfg, 1, KV_PROMPT, steps, warmup)
        nbytes = llm.decode_step_bytes(cfg, 1, ctx_avg)
        achieved = nbytes["total"] / (ms * 1e-3) / 1e9
        value, unit, dtype = 1e3 / ms, "tokens/s", "fp8-e4m3 weights, fp16 act, fp32 acc"
        total_ms = ms * steps
        workload = {"workload": "configs[4]: Qwen3-0.6B-shaped decoder (28 layers, hidden 1024, "
                                "16 Q / 8 KV heads, head_dim 128, SwiGLU 3072, vocab 151936), "
                                "FP8-E4M3 weights with per-channel fp32 scales, greedy decode "
                                "at batch 1 after a 4096-token random prompt",
                    "batch": 1, "kv_context_avg": ctx_avg,
                    "alg_bytes_per_step": nbytes}
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": read_traffic("qwen3_decode_step"),
                    "kernel": "decode step: embed, then decode_layers_kernel (all 28 layers, "
                              "final RMSNorm and LM head with greedy argmax in one persistent "
                              "launch)"}
        log(f"headline: {value:.1f} tokens/s, {achieved:.1f} GB/s algorithmic")
        if not args.no_extra:
            for b, st in ((4, 32), (16, 16)):
                c = llm.QWEN3_0_6B.with_(max_positions=KV_PROMPT + 4 + st + 1, max_batch=b)
                bms, bctx = decode_run(ctx, c, b, KV_PROMPT, st, 4)
                by = llm.decode_step_bytes(c, b, bctx)["total"]
                e = hbm_entry(f"qwen3 decode step b={b} (configs[4])", by, bms)
                e["tokens/s"] = round(b * 1e3 / bms, 1)
                kernels.append(e)
            g = llm.GPT2_SMALL
            gms, gctx = decode_run(ctx, g, 1, 128, 256, 0)
            e = hbm_entry("gpt2 decode step b=1 (configs[3], 128-token prompt, 256 steps)",
                          llm.decode_step_bytes(g, 1, gctx)["total"], gms)
            e["tokens/s"] = round(1e3 / gms, 1)
            kernels.append(e)
    if not args.no_extra or args.workload != "decode":
        img = image_kernels(ctx, rng, table_steps if args.workload != "image" else steps)
        kernels += [v[0] for v in img.values()]
        sig = sigmoid_kernel(ctx, rng, table_steps if args.workload != "sigmoid" else steps)
        kernels.append(sig[0])
    if not args.no_extra:
        kernels.append(gemm_kernel(ctx, rng))
        kernels.append(gemm_fp8_kernel(ctx, rng))
        kernels.append(gemv_kernel(ctx, rng, table_steps))

    if args.workload == "image":
        head, total_ms, _ = img["brightness_blur5_u8 (fused, configs[1])"]
        value, unit, dtype = head["GB/s"], "GB/s", "u8"
        achieved = head["GB/s"]
        workload = {"workload": "configs[1]: AdjustBrightness(+/-40) then 5x5 box blur "
                                "(clamp-to-edge, (sum+12)/25), fused, 4096x4096 RGBA8",
                    "width": IMG_W, "height": IMG_H, "channels": 4,
                    "alg_bytes_per_step": 2 * IMG_BYTES}
        roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": read_traffic("brightness_blur5_u8")}
        warmup = 5
    elif args.workload == "sigmoid":
        head, total_ms, _ = sig
        value, unit, dtype = head["GB/s"], "GB/s", "f32"
        achieved = head["GB/s"]
        workload = {"workload": "configs[0]: sigmoid fp32 over N=2^24 uniform[-8,8]",
                    "n": SIGMOID_N, "alg_bytes_per_step": 8 * SIGMOID_N}
        roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": read_traffic("sigmoid_f32")}
        warmup = 5
    from strict_amd import yardstick

    yardstick.release()  # hipBLASLt handles and workspace, before the context goes
    ctx.dispose()

    cpu = None
    if not args.no_cpu_baseline:
        cpu = {"decode": cpu_baseline_decode, "image": cpu_baseline_image,
               "sigmoid": cpu_baseline_sigmoid}[args.workload](args.cpu_seconds)
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": "HBM GB/s (% peak) per kernel; decode tokens/s Qwen3-0.6B-shape FP8 b=1",
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(total_ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic: seeded random weights / prompts / pixels, resident in HBM",
        "config": workload,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    # a successful run ends by returning from the script, not through
    # sys.exit(0): under rocprofv3 that path lost the profiler's output at exit
    _rc = main()
    if _rc:
        sys.exit(_rc)
