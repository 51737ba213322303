"""CPU oracle of the LLM decode path -- TEST INFRASTRUCTURE ONLY.

The reference (strict-lang/Strict) has no LLM, GEMM, FP8, attention or norm
code at all (SURVEY rows a13-a16 are defined by BASELINE.json configs[3] and
configs[4] alone), so this module restates the two model definitions from
their published architectures in numpy:

- Qwen3: RMSNorm (eps 1e-6) -> fused QKV projection -> per-head
  RMSNorm of q and k -> RoPE rotate-half (theta 1e6) -> GQA softmax attention
  -> O projection + residual -> RMSNorm -> SwiGLU MLP + residual; final
  RMSNorm; LM head tied to the token embedding. Linear weights are OCP E4M3
  with one fp32 scale per output row.
- GPT-2: token + learned position embedding -> LayerNorm (eps
  1e-5) -> QKV (+bias) -> MHA -> O (+bias) + residual -> LayerNorm -> GELU
  (tanh) MLP (+biases) + residual; final LayerNorm; LM head tied to wte.
  Weights fp16.

It rounds to fp16 exactly where the GPU path does (normalised activations
fed to a projection, K/V written to the cache, the attention output, the MLP
activation) and otherwise computes in fp32 (projections: fp32 BLAS sums of
exact products) or fp64 (norm statistics, softmax, RoPE sin/cos). Only the
order of fp32 summation differs from the GPU, so the two agree to ~1e-5 and
greedy tokens agree except where two logits tie to that precision.

Only tests/ import this module, as the checker of strict_amd's HIP path.
"""
from __future__ import annotations

import numpy as np

import oracle

QWEN3, GPT2 = 0, 1


def f16(x) -> np.ndarray:
    """Round to fp16 (nearest even) and widen back to fp32."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def rms_norm(x: np.ndarray, g: np.ndarray, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * g over the last axis, statistics in fp64,
    applied in fp32 as (x * inv) * g."""
    ms = np.mean(np.square(x.astype(np.float64)), axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(ms + eps)).astype(np.float32)
    return (x.astype(np.float32) * inv) * g.astype(np.float32)


def layer_norm(x: np.ndarray, g: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    x64 = x.astype(np.float64)
    mean = x64.mean(axis=-1, keepdims=True)
    var = np.square(x64 - mean).mean(axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    return ((x.astype(np.float32) - mean.astype(np.float32)) * inv) * g + b


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float32)
    c = np.float32(0.7978845608028654)
    return np.float32(0.5) * x * (np.float32(1.0) + np.tanh(c * (x + np.float32(0.044715) * x * x * x)))


def silu(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float32)
    return x / (np.float32(1.0) + np.exp(-x))


def rope_tables(inv_freq: np.ndarray, positions: np.ndarray):
    """cos/sin [T, d/2] of angle = float32(pos) * inv_freq (an fp32 product)."""
    ang = positions.astype(np.float32)[:, None] * inv_freq.astype(np.float32)[None, :]
    a64 = ang.astype(np.float64)
    return np.cos(a64).astype(np.float32), np.sin(a64).astype(np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE of x [T, H, d] with cos/sin [T, d/2]."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c, s = cos[:, None, :], sin[:, None, :]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1).astype(np.float32)


def attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, visible=None) -> np.ndarray:
    """softmax(q k^T) v in fp64 for query rows q [T, d] (already scaled) over
    keys / values [P, d]; visible [T, P] (bool) hides positions where False."""
    s = np.asarray(q, np.float64) @ np.asarray(k, np.float64).T
    if visible is not None:
        s = np.where(visible, s, -np.inf)
    s = s - s.max(axis=1, keepdims=True)
    e = np.exp(s)
    return (e @ np.asarray(v, np.float64)) / e.sum(axis=1, keepdims=True)


def attn_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, lengths, scale: float) -> np.ndarray:
    """Grouped-query decode attention: out[b, h] = attend(fp32(q[b, h] * scale),
    k[b, h // G, :L], v[b, h // G, :L]) with L = min(lengths[b], P), zeros for
    L <= 0; q [B, H, d] fp32, k / v [B, KVH, P, d], G = H / KVH."""
    B, H, d = q.shape
    KVH, P = k.shape[1], k.shape[2]
    G = H // KVH
    qs = (q.astype(np.float32) * np.float32(scale)).astype(np.float32)
    out = np.zeros((B, H, d), np.float32)
    for b in range(B):
        L = min(int(lengths[b]), P)
        if L <= 0:
            continue
        for h in range(H):
            out[b, h] = attend(qs[b, h][None, :], k[b, h // G, :L], v[b, h // G, :L])[0]
    return out


class Weights:
    """Dequantized per-layer weights as fp32 [rows, cols] (logical order) with
    per-row scales (1 for fp16 models), norms and biases."""

    def __init__(self, cfg, layers, head_w, head_scale, final_g, final_b=None, wpe=None,
                 inv_freq=None):
        self.cfg = cfg
        self.layers = layers
        self.head_w = head_w
        self.head_scale = head_scale
        self.final_g = final_g
        self.final_b = final_b
        self.wpe = wpe
        self.inv_freq = inv_freq


def linear(h16: np.ndarray, w: np.ndarray, scale: np.ndarray, bias=None,
           accumulate=np.float32) -> np.ndarray:
    """(h16 @ w.T) * scale (+ bias), fp32. The dot products are summed in
    `accumulate` (fp32 BLAS by default; np.float64 gives the exactly rounded
    sum of the exact products, a second valid order used to show how far two
    correct implementations drift apart through fp16 re-rounding)."""
    y = (h16.astype(accumulate) @ w.T.astype(accumulate)).astype(np.float32) * scale.astype(np.float32)
    if bias is not None:
        y = y + bias.astype(np.float32)
    return y.astype(np.float32)


class Decoder:
    """Greedy decoder over one sequence with a KV cache."""

    def __init__(self, weights: Weights, accumulate=np.float32):
        self.w = weights
        self.acc = accumulate  # the linears' summation type (see linear)
        c = weights.cfg
        self.c = c
        self.k = [np.zeros((0, c.kv_heads, c.head_dim), np.float32) for _ in range(c.layers)]
        self.v = [np.zeros((0, c.kv_heads, c.head_dim), np.float32) for _ in range(c.layers)]
        self.pos = 0

    def embed(self, tokens: np.ndarray, positions: np.ndarray) -> np.ndarray:
        w = self.w
        if self.c.arch == QWEN3:
            return (w.head_w[tokens] * w.head_scale[tokens][:, None]).astype(np.float32)
        return (w.head_w[tokens] + w.wpe[positions]).astype(np.float32)

    def norm(self, x, g, b):
        if self.c.arch == QWEN3:
            return f16(rms_norm(x, g, self.c.norm_eps))
        return f16(layer_norm(x, g, b, self.c.norm_eps))

    # query rows per attention block of a long forward: a block's rows see the
    # keys up to its last row's position only, which halves a long prompt's
    # score work; every row's softmax covers exactly its visible keys either way
    QUERY_BLOCK = 256

    def forward(self, tokens, last_only: bool = False) -> np.ndarray:
        """Runs tokens [T] (appended after the cached ones); returns logits
        [T, vocab], or [1, vocab] of the last token when last_only."""
        c, w = self.c, self.w
        tokens = np.asarray(tokens, np.int64)
        T = len(tokens)
        positions = np.arange(self.pos, self.pos + T)
        x = self.embed(tokens, positions)
        d, H, KVH = c.head_dim, c.heads, c.kv_heads
        G = H // KVH
        if c.arch == QWEN3:
            cos, sin = rope_tables(w.inv_freq, positions)
        scale = np.float32(1.0 / np.sqrt(np.float32(d)))
        for li, L in enumerate(w.layers):
            h = self.norm(x, L["norm1.g"], L.get("norm1.b"))
            qkv = linear(h, L["qkv"], L["qkv.scale"], L.get("qkv.bias"), self.acc)
            q = qkv[:, : H * d].reshape(T, H, d)
            k = qkv[:, H * d:(H + KVH) * d].reshape(T, KVH, d)
            v = qkv[:, (H + KVH) * d:].reshape(T, KVH, d)
            if c.arch == QWEN3:
                q = rope(rms_norm(q, L["q_norm"], c.norm_eps), cos, sin)
                k = rope(rms_norm(k, L["k_norm"], c.norm_eps), cos, sin)
            q = (q * scale).astype(np.float32)
            self.k[li] = np.concatenate([self.k[li], f16(k)])
            self.v[li] = np.concatenate([self.v[li], f16(v)])
            K_ = self.k[li].astype(np.float64)  # [P, KVH, d]
            V_ = self.v[li].astype(np.float64)
            out = np.empty((T, H, d), np.float32)
            # causal: token t (absolute pos self.pos + t) sees positions <= it
            for t0 in range(0, T, self.QUERY_BLOCK):
                t1 = min(T, t0 + self.QUERY_BLOCK)
                P = self.pos + t1  # keys any row of the block can see
                visible = np.arange(P)[None, :] <= (self.pos + np.arange(t0, t1))[:, None]
                for hh in range(H):
                    kv = hh // G
                    out[t0:t1, hh, :] = attend(q[t0:t1, hh, :], K_[:P, kv, :], V_[:P, kv, :],
                                               visible)
            attn = f16(out.reshape(T, H * d))
            x = x + linear(attn, L["o"], L["o.scale"], L.get("o.bias"), self.acc)
            h2 = self.norm(x, L["norm2.g"], L.get("norm2.b"))
            if c.arch == QWEN3:
                gu = linear(h2, L["gate_up"], L["gate_up.scale"], None, self.acc)
                act = f16(silu(gu[:, : c.intermediate]) * gu[:, c.intermediate:])
                x = x + linear(act, L["down"], L["down.scale"], None, self.acc)
            else:
                act = f16(gelu_tanh(linear(h2, L["fc"], L["fc.scale"], L.get("fc.bias"), self.acc)))
                x = x + linear(act, L["proj"], L["proj.scale"], L.get("proj.bias"), self.acc)
            x = x.astype(np.float32)
        self.pos += T
        if last_only:
            x = x[-1:]
        hf = self.norm(x, w.final_g, w.final_b)
        return linear(hf, w.head_w[: c.vocab], w.head_scale[: c.vocab], None, self.acc)


def load_from_model(model) -> Weights:
    """Reads every weight of a strict_amd.llm.Model back from the device and
    dequantizes it (E4M3 bytes decoded by oracle.e4m3_to_f32; fp16 bits widened)."""
    from strict_amd.llm import (QWEN3 as Q, interleaved_to_logical, linear_shapes, untile_f16,
                                untile_fp8)

    cfg = model.cfg
    qwen = cfg.arch == Q
    shapes = linear_shapes(cfg)

    def lin(name, layer):
        rows, cols = shapes[name]
        stored_rows = rows
        raw = model.read(f"{name}.w", layer, np.uint8)
        if qwen:
            q = untile_fp8(raw, stored_rows, cols)
            w = oracle.e4m3_to_f32(q)
            s = model.read(f"{name}.scale", layer, np.float32)
        else:
            h = untile_f16(raw.view(np.uint16), stored_rows, cols)
            w = oracle.f16_to_f32(h)
            s = np.ones(stored_rows, np.float32)
        if name == "gate_up":
            w = interleaved_to_logical(w, cfg.intermediate)
            s = interleaved_to_logical(s[:, None], cfg.intermediate)[:, 0]
        return w, s

    layers = []
    for li in range(cfg.layers):
        L = {}
        for name in ("qkv", "o", "gate_up" if qwen else "fc", "down" if qwen else "proj"):
            w, s = lin(name, li)
            L[name] = w
            L[name + ".scale"] = s
            if not qwen:
                L[name + ".bias"] = model.read(f"{name}.bias", li, np.float32)
        L["norm1.g"] = model.read("norm1.g", li, np.float32)
        L["norm2.g"] = model.read("norm2.g", li, np.float32)
        if qwen:
            L["q_norm"] = model.read("q_norm", li, np.float32)
            L["k_norm"] = model.read("k_norm", li, np.float32)
        else:
            L["norm1.b"] = model.read("norm1.b", li, np.float32)
            L["norm2.b"] = model.read("norm2.b", li, np.float32)
        layers.append(L)
    head_w, head_s = lin("head", 0)
    final_g = model.read("final.g", 0, np.float32)
    if qwen:
        return Weights(cfg, layers, head_w, head_s, final_g,
                       inv_freq=model.read("inv_freq", 0, np.float32))
    wpe = oracle.f16_to_f32(model.read("wpe", 0, np.uint16)).reshape(cfg.max_positions, cfg.hidden)
    return Weights(cfg, layers, head_w, head_s, final_g, model.read("final.b", 0, np.float32),
                   wpe=wpe)


def inv_freq(theta: float, d: int) -> np.ndarray:
    """float32(theta ** (-2i/d)) computed in fp64, i = 0 .. d/2-1."""
    return np.array([theta ** (-2.0 * i / d) for i in range(d // 2)], np.float64).astype(np.float32)


def greedy_compare(gpu_tokens, decoder: Decoder, prompt, steps: int, logit_fn=None):
    """Teacher-forced comparison: feeds the prompt, then at each step the GPU's
    token; returns (oracle argmax per step, per-step top-2 margin, oracle logits
    of each step when logit_fn is None)."""
    logits = decoder.forward(prompt, last_only=True)[-1]
    ours, margins, all_logits = [], [], []
    for j in range(steps):
        top = int(np.argmax(logits))
        srt = np.sort(logits)
        ours.append(top)
        margins.append(float(srt[-1] - srt[-2]))
        all_logits.append(logits)
        if j + 1 < steps:
            logits = decoder.forward([int(gpu_tokens[j])], last_only=True)[-1]
    return np.array(ours), np.array(margins), all_logits
