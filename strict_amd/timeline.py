"""Per-phase timelines of the persistent decode kernels, from their diagnostic
builds: compiled with -DSH_DECODE_TRACE (Qwen3 decode-layers kernel) or
-DSH_GPT2_TRACE (GPT-2 layers kernel), the kernels keep wall-clock marks
(100 MHz) per workgroup, layer and event of the last step, which
sh_debug_decode_trace / sh_debug_gpt2_trace copy out. The product library
has neither mark nor entry point.

Build a diagnostic library beside the product one and point the package at
it (a command-line EXTRA_HIPFLAGS replaces the Makefile's per-file
-ffp-contract=off of decode_layers.hip, hence the flag here):

    make -C strict_amd/csrc OUT=$PWD/trace/libstrict_hip.so OBJDIR=$PWD/trace/obj \\
        EXTRA_HIPFLAGS="-DSH_DECODE_TRACE -DSH_GPT2_TRACE -ffp-contract=off" \\
        $PWD/trace/libstrict_hip.so
    STRICT_HIP_LIBRARY=$PWD/trace/libstrict_hip.so python3 -m strict_amd.timeline decode
    STRICT_HIP_LIBRARY=$PWD/trace/libstrict_hip.so python3 -m strict_amd.timeline gpt2

``decode``: the Qwen3-0.6B shape at batch 1 after a random prompt (default
4,096 tokens), 8 greedy steps. ``gpt2``: GPT-2 small at batch 1, a 128-token
prompt and 128 greedy steps (context 256). Both print, averaged over the
inner layers, each phase's hop (the consumers' completed waits after the
producing phase's last item), item work and phase span, and the sub-phases
inside items. The marks cost a few percent of the step; compare timelines
with timelines, and step times with the product library's.
"""
from __future__ import annotations

import argparse
import ctypes
import sys

import numpy as np


def _trace(lib, name: str, shape) -> np.ndarray:
    fn = getattr(lib, name, None)
    if fn is None:
        raise SystemExit(f"{name} is missing: the library was not built with the kernel's trace flag")
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    buf = np.zeros(shape, np.uint64)
    if fn(buf.ctypes.data, buf.nbytes) != 0:
        raise SystemExit(f"{name} failed")
    return buf.astype(np.int64)


def _ns(t: np.ndarray, base: int) -> np.ndarray:
    """Marks as ns after `base`; -1 where a mark was not written."""
    return np.where(t > 0, (t - base) * 10, -1)


def _med(x: np.ndarray) -> float:
    x = x[x >= 0]
    return float(np.median(x)) if x.size else float("nan")


def _max(x: np.ndarray) -> float:
    x = x[x >= 0]
    return float(x.max()) if x.size else float("nan")


def _sub(a: np.ndarray, b: np.ndarray) -> float:
    """Median over workgroups of b - a where both marks exist."""
    ok = (a >= 0) & (b >= 0)
    return float(np.median(b[ok] - a[ok])) if ok.any() else float("nan")


def decode(prompt_len: int) -> str:
    """Qwen3 decode-layers kernel, batch 1 (tr[0]: per phase start / end /
    wait end, merge end, first attention items' ends; tr[1]: marks inside
    items, and at layer n_layers the LM head's final-RMSNorm wait end and
    the workgroup's end)."""
    import strict_amd
    from strict_amd import _lib, llm

    ctx = strict_amd.Context(0)
    cfg = llm.QWEN3_0_6B.with_(max_positions=prompt_len + 64, max_batch=1)
    m = llm.Model(ctx, cfg)
    try:
        m.init_random(seed=42, stddev=0.02)
        m.reset(1)
        prompt = np.random.default_rng(42).integers(0, cfg.vocab, (1, prompt_len))
        for i in range(prompt_len):
            m.step(prompt[:, i], logits=(i == prompt_len - 1))
        for _ in range(8):
            m.step(None, logits=True)
        ctx.sync()
        buf = _trace(_lib.load(), "sh_debug_decode_trace", (2, 256, 32, 24))
    finally:
        m.close()
        ctx.dispose()
    starts = buf[0][:, 0, 0]
    base = int(starts[starts > 0].min())
    t, t2 = _ns(buf[0], base), _ns(buf[1], base)
    L = cfg.layers
    names = ["QKV", "attention", "O", "gate/up", "down"]
    rows = {n: [] for n in names}
    for l in range(1, L - 1):
        prev = _max(t[:, l - 1, 9])  # the previous layer's last down item
        for ph, n in enumerate(names):
            end, wait = t[:, l, 2 * ph + 1], t[:, l, 10 + ph]
            ok = (end >= 0) & (wait >= 0)
            rows[n].append((_med(wait[ok]) - prev, _sub(wait, end), _max(end) - prev))
            prev = _max(end)
    out = [f"Qwen3 decode-layers kernel, batch 1, context {prompt_len + 9}; means over layers 1..{L - 2} (ns)",
           "  phase       wait done after the previous phase's last end | item work | phase span"]
    for n in names:
        h, wk, sp = np.nanmean(np.array(rows[n]), axis=0)
        out.append(f"  {n:9s} {h:10.0f} {wk:36.0f} {sp:11.0f}")
    per = lambda f: np.nanmean([f(l) for l in range(1, L - 1)])  # noqa: E731
    out.append("  QKV item: staged %.0f, MFMA %.0f, cross-wave sum %.0f, store %.0f" % (
        per(lambda l: _sub(t[:, l, 10], t2[:, l, 0])), per(lambda l: _sub(t2[:, l, 0], t2[:, l, 1])),
        per(lambda l: _sub(t2[:, l, 1], t2[:, l, 2])), per(lambda l: _sub(t2[:, l, 2], t2[:, l, 3]))))
    out.append("  attention item: start -> q/k/v polled %.0f, RoPE %.0f, scores %.0f, softmax %.0f, "
               "V sums %.0f, stores %.0f" % (
                   per(lambda l: _sub(t2[:, l, 22], t2[:, l, 8])),
                   *[per(lambda l, k=k: _sub(t2[:, l, k], t2[:, l, k + 1])) for k in range(8, 13)]))
    out.append("  merge: polled %.0f after the last attention item, then %.0f to its stores" % (
        per(lambda l: _med(t2[:, l, 14]) - _max(t[:, l, 3])), per(lambda l: _sub(t2[:, l, 14], t2[:, l, 15]))))
    out.append("  down item: staged %.0f, MFMA %.0f, cross-wave sum %.0f, store %.0f" % (
        per(lambda l: _sub(t[:, l, 14], t2[:, l, 4])), per(lambda l: _sub(t2[:, l, 4], t2[:, l, 5])),
        per(lambda l: _sub(t2[:, l, 5], t2[:, l, 6])), per(lambda l: _sub(t2[:, l, 6], t2[:, l, 7]))))
    hw, he, de = t2[:, L, 0], t2[:, L, 1], _max(t[:, L - 1, 9])
    head_bytes = cfg.vocab * cfg.hidden + cfg.vocab * 4  # FP8 rows and their scales
    if (hw >= 0).any() and (he >= 0).any():
        span = _max(he) - _med(hw)
        out.append(f"  LM head: final-RMSNorm input arrived {_med(hw) - de:.0f} after the last down end "
                   f"(median), then {span:.0f} to the last workgroup's end: {head_bytes / span / 1e3:.2f} TB/s "
                   f"over {head_bytes:,} B of head rows and scales")
    return "\n".join(out)


def gpt2(steps: int) -> str:
    """GPT-2 layers kernel, batch 1 (per workgroup and layer: slots 0..4 the
    ends of its QKV / attention / O / fc / proj items, 5..9 the ends of their
    waits; layer 0 slot 10 the kernel's start, slot 11 the head's end;
    12..15 the attention item's q / k / v staged, scores, softmax, V sums;
    layer n_layers slot 0 the end of the head's final-LayerNorm wait)."""
    import strict_amd
    from strict_amd import _lib, llm

    ctx = strict_amd.Context(0)
    cfg = llm.GPT2_SMALL
    m = llm.Model(ctx, cfg)
    try:
        m.init_random(seed=42, stddev=0.02)
        m.reset(1)
        prompt = np.random.default_rng(42).integers(0, cfg.vocab, (1, 128))
        for i in range(128):
            m.step(prompt[:, i], logits=(i == 127))
        for _ in range(steps):
            m.step(None, logits=True)
        ctx.sync()
        buf = _trace(_lib.load(), "sh_debug_gpt2_trace", (256, 16, 16))
    finally:
        m.close()
        ctx.dispose()
    starts = buf[:, 0, 10]
    t = _ns(buf, int(starts[starts > 0].min()))
    L = cfg.layers
    names = ["QKV", "attention", "O", "fc", "proj"]
    hops = {n: [] for n in names}
    work = {n: [] for n in names}
    for l in range(1, L - 1):
        prev = _max(t[:, l - 1, 4])
        for ph, n in enumerate(names):
            end, wait = t[:, l, ph], t[:, l, 5 + ph]
            hops[n].append(_med(wait) - prev)
            work[n].append(_sub(wait, end))
            prev = _max(end)
    spans = [_max(t[:, l + 1, 4]) - _max(t[:, l, 4]) for l in range(L - 1)]
    out = [f"GPT-2 layers kernel, batch 1, context {128 + steps}; means over layers 1..{L - 2} (ns)",
           f"  layer span (last proj end to last proj end): {np.mean(spans):.0f}",
           "  phase       wait done after the previous phase's last end | item work"]
    for n in names:
        out.append(f"  {n:9s} {np.nanmean(hops[n]):10.0f} {np.nanmean(work[n]):36.0f}")
    sub = [("q/k/v staged", 6, 12), ("scores", 12, 13), ("softmax", 13, 14), ("V sums", 14, 15),
           ("stores", 15, 1)]
    out.append("  attention item: " + ", ".join(
        f"{n} {np.nanmean([_sub(t[:, l, a0], t[:, l, a1]) for l in range(1, L - 1)]):.0f}" for n, a0, a1 in sub))
    hw, he, pe = t[:, L, 0], t[:, 0, 11], _max(t[:, L - 1, 4])
    head_bytes = cfg.vocab * cfg.hidden * 2
    if (hw >= 0).any() and (he >= 0).any():
        span = _max(he) - _med(hw)
        out.append(f"  LM head: final-LayerNorm input arrived {_med(hw) - pe:.0f} after the last proj end "
                   f"(median), then {span:.0f} to the last workgroup's end: {head_bytes / span / 1e3:.2f} TB/s "
                   f"over {head_bytes:,} B of head rows")
    return "\n".join(out)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m strict_amd.timeline", description=__doc__.split("\n\n")[0])
    sp = p.add_subparsers(dest="kernel", required=True)
    d = sp.add_parser("decode", help="Qwen3 decode-layers kernel, batch 1")
    d.add_argument("--prompt", type=int, default=4096)
    g = sp.add_parser("gpt2", help="GPT-2 layers kernel, batch 1")
    g.add_argument("--steps", type=int, default=128)
    a = p.parse_args(argv)
    print(decode(a.prompt) if a.kernel == "decode" else gpt2(a.steps), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
