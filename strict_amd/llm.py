"""Greedy decoding of the BASELINE LLM configs through libstrict_hip's sh_llm_*
C ABI: GPT-2 small (fp16 weights) and the Qwen3-0.6B shape (FP8-E4M3
weights with per-output-channel fp32 scales). The reference has no LLM path
at all; the configs in BASELINE.json define these models.

Weights are random (``init_random``: N(0, stddev) from a counter-based
generator on the device) or loaded per linear from fp32 arrays
(``load_linear``); ``tensor`` exposes every device buffer for read-back.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, replace

import numpy as np

from . import _lib
from . import Context, _check

QWEN3, GPT2 = 0, 1


@dataclass(frozen=True)
class Config:
    arch: int
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    max_positions: int
    max_batch: int = 1
    rope_theta: float = 1e6
    norm_eps: float = 1e-6

    def with_(self, **kw) -> "Config":
        return replace(self, **kw)

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    @property
    def vocab_pad(self) -> int:
        return (self.vocab + 15) // 16 * 16


# Qwen3-0.6B shape, 4096-token KV cache (+ 256 decode steps)
QWEN3_0_6B = Config(QWEN3, layers=28, hidden=1024, heads=16, kv_heads=8, head_dim=128,
                    intermediate=3072, vocab=151936, max_positions=4096 + 256,
                    rope_theta=1e6, norm_eps=1e-6)
# GPT-2 small, ctx 1024
GPT2_SMALL = Config(GPT2, layers=12, hidden=768, heads=12, kv_heads=12, head_dim=64,
                    intermediate=3072, vocab=50257, max_positions=1024, norm_eps=1e-5)


def linear_shapes(cfg: Config) -> dict:
    """(rows, cols) of every per-layer linear in logical order, plus the head."""
    d = cfg.head_dim
    up = "gate_up" if cfg.arch == QWEN3 else "fc"
    down = "down" if cfg.arch == QWEN3 else "proj"
    return {
        "qkv": (cfg.qkv_rows, cfg.hidden),
        "o": (cfg.hidden, cfg.heads * d),
        up: ((2 if cfg.arch == QWEN3 else 1) * cfg.intermediate, cfg.hidden),
        down: (cfg.hidden, cfg.intermediate),
        "head": (cfg.vocab_pad, cfg.hidden),
    }


class Model:
    """One decoder on a Context's device (sh_llm)."""

    def __init__(self, ctx: Context, cfg: Config):
        self.ctx = ctx
        self.cfg = cfg
        self._l = ctx._l
        c = _lib.LlmConfig(cfg.arch, cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads,
                           cfg.head_dim, cfg.intermediate, cfg.vocab, cfg.max_positions,
                           cfg.max_batch, cfg.rope_theta, cfg.norm_eps)
        h = ctypes.c_void_p()
        _check(self._l.sh_llm_create(ctx.handle, ctypes.byref(c), ctypes.byref(h)))
        self.handle = h
        self.batch = 0

    def close(self) -> None:
        if self.handle:
            self._l.sh_llm_destroy(self.handle)
            self.handle = ctypes.c_void_p(0)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def init_random(self, seed: int = 42, stddev: float = 0.02) -> None:
        _check(self._l.sh_llm_init_random(self.handle, seed, stddev))

    def load_linear(self, name: str, layer: int, w: np.ndarray) -> None:
        """w: fp32 [rows, cols] in logical row order (gate_up: gate rows then up rows)."""
        w = np.ascontiguousarray(w, np.float32)
        dev = self.ctx.upload(w)
        try:
            _check(self._l.sh_llm_load_linear(self.handle, name.encode(), layer,
                                              ctypes.c_void_p(dev.ptr)))
            self.ctx.sync()
        finally:
            dev.free()

    def tensor(self, name: str, layer: int = 0) -> tuple[int, int]:
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        _check(self._l.sh_llm_tensor(self.handle, name.encode(), layer, ctypes.byref(p),
                                     ctypes.byref(n)))
        return p.value, n.value

    @property
    def uses_layers_kernel(self) -> bool:
        """True when one persistent kernel runs all layers of a step."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        status = self._l.sh_llm_tensor(self.handle, b"layers.err", 0, ctypes.byref(p),
                                       ctypes.byref(n))
        return status == 0

    def read(self, name: str, layer: int = 0, dtype=np.uint8) -> np.ndarray:
        ptr, nbytes = self.tensor(name, layer)
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
        _check(self._l.sh_download(self.ctx.handle, out.ctypes.data_as(ctypes.c_void_p),
                                   ctypes.c_void_p(ptr), out.nbytes))
        return out

    def write(self, name: str, layer: int, values: np.ndarray) -> None:
        ptr, nbytes = self.tensor(name, layer)
        a = np.ascontiguousarray(values)
        if a.nbytes != nbytes:
            raise ValueError(f"{name}: {a.nbytes} bytes given, tensor holds {nbytes}")
        _check(self._l.sh_upload(self.ctx.handle, ctypes.c_void_p(ptr),
                                 a.ctypes.data_as(ctypes.c_void_p), a.nbytes))

    def reset(self, batch: int = 1) -> None:
        _check(self._l.sh_llm_reset(self.handle, batch))
        self.batch = batch

    def step(self, tokens=None, logits: bool = True) -> None:
        if tokens is None:
            _check(self._l.sh_llm_step(self.handle, None, 1 if logits else 0))
        else:
            t = np.ascontiguousarray(tokens, np.int32)
            _check(self._l.sh_llm_step(self.handle, t.ctypes.data_as(ctypes.c_void_p),
                                       1 if logits else 0))

    def next_tokens(self) -> np.ndarray:
        out = np.empty(self.batch, np.int32)
        _check(self._l.sh_llm_next_tokens(self.handle, out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def logits(self) -> np.ndarray:
        """fp32 logits of the last step with logits, [batch, vocab]."""
        full = self.read("logits", 0, np.float32).reshape(self.cfg.max_batch, self.cfg.vocab_pad)
        return full[: self.batch, : self.cfg.vocab]

    def generate(self, prompt: np.ndarray, steps: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.int32)
        if p.ndim == 1:
            p = p[None, :]
        out = np.empty((p.shape[0], steps), np.int32)
        _check(self._l.sh_llm_generate(self.handle, p.ctypes.data_as(ctypes.c_void_p),
                                       p.shape[1], steps, out.ctypes.data_as(ctypes.c_void_p)))
        return out


def untile_fp8(tiled: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Row-major [rows, cols] bytes from the FP8 tiled layout (16-row x 64-col
    1 KiB tiles; lane l of a tile holds row l%16, cols 8*(l//16)+e of two
    32-col halves in bytes 0-7 and 8-15)."""
    t = tiled.reshape(rows // 16, cols // 64, 4, 16, 2, 8)  # [nt, kt, lane/16, lane%16, half, e]
    return np.ascontiguousarray(t.transpose(0, 3, 1, 4, 2, 5)).reshape(rows, cols)


def untile_f16(tiled: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Row-major [rows, cols] fp16 bit patterns from the fp16 tiled layout
    (16-row x 32-col tiles; lane l holds row l%16, cols 8*(l//16)+e)."""
    t = tiled.reshape(rows // 16, cols // 32, 4, 16, 8)  # [nt, kt, lane/16, lane%16, e]
    return np.ascontiguousarray(t.transpose(0, 3, 1, 2, 4)).reshape(rows, cols)


def interleaved_to_logical(rows: np.ndarray, intermediate: int) -> np.ndarray:
    """gate/up rows as stored (16-row tiles alternating gate, up) -> [gate; up]."""
    t = rows.reshape(intermediate // 16, 2, 16, -1)
    return np.concatenate([t[:, 0].reshape(intermediate, -1), t[:, 1].reshape(intermediate, -1)])


def decode_step_bytes(cfg: Config, batch: int, context: float) -> dict:
    """Algorithmic HBM bytes of one decode step of `batch` sequences attending
    over `context` cached positions: every weight byte the step reads once
    (linears, their scales, the LM head, norms, biases, one embedding row per
    sequence) plus K and V of every cached position. Activations are excluded
    (< 0.1 %)."""
    shapes = linear_shapes(cfg)
    wbytes = 1 if cfg.arch == QWEN3 else 2
    per_layer = sum(r * c for name, (r, c) in shapes.items() if name != "head") * wbytes
    head = shapes["head"][0] * shapes["head"][1] * wbytes
    scales = 0
    norms = cfg.layers * 2 * cfg.hidden * 4 + cfg.hidden * 4
    if cfg.arch == QWEN3:
        scales = cfg.layers * sum(r for name, (r, c) in shapes.items() if name != "head") * 4
        scales += shapes["head"][0] * 4
        norms += cfg.layers * 2 * cfg.head_dim * 4
    else:
        scales = cfg.layers * sum(r for name, (r, c) in shapes.items() if name != "head") * 4  # biases
        norms *= 2  # LayerNorm gains and biases
    embed = batch * cfg.hidden * wbytes
    kv = batch * cfg.layers * cfg.kv_heads * cfg.head_dim * 2 * 2 * context
    weights = cfg.layers * per_layer + head + scales + norms + embed
    return {"weights": int(weights), "kv": int(kv), "total": int(weights + kv)}
