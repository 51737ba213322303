"""CPU oracle for the Strict GPU kernel path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package, and only as the checker. The product path
(``strict_amd``) never imports it.

``liboracle.so`` is the C restatement in ``oracle.c`` (built by ``make -C
oracle``); this module wraps it for numpy arrays. ``oracle.llm`` holds the
float32/float64 numpy oracle for the LLM ops, for which the reference has no
implementation.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

ADD, SUBTRACT, MULTIPLY, DIVIDE = 0, 1, 2, 3


def build() -> None:
    """Compile liboracle.so from oracle.c (gcc)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(l) -> None:
    P = ctypes.c_void_p
    sz = ctypes.c_size_t
    i = ctypes.c_int
    f = ctypes.c_float
    l.or_binary_f32.argtypes = [i, P, P, P, sz]
    l.or_fill_f32.argtypes = [f, P, sz]
    l.or_saxpy_f32.argtypes = [f, P, P, P, sz]
    l.or_sigmoid_f32.argtypes = [P, P, sz, i]
    l.or_adjust_brightness.argtypes = [P, P, sz, i, i, i, i]
    l.or_blur5_reference.argtypes = [P, P, i, i, i, i]
    l.or_blur5_config.argtypes = [P, P, i, i, i, i]
    l.or_brightness_blur5_config.argtypes = [P, P, i, i, i, i, i, i]
    l.or_f32_to_bf16_array.argtypes = [P, P, sz]
    l.or_bf16_to_f32_array.argtypes = [P, P, sz]
    l.or_f32_to_f16_array.argtypes = [P, P, sz]
    l.or_f16_to_f32_array.argtypes = [P, P, sz]
    l.or_e4m3_to_f32_array.argtypes = [P, P, sz]
    l.or_f32_to_e4m3.argtypes = [f]
    l.or_f32_to_e4m3.restype = ctypes.c_uint8
    l.or_e4m3_to_f32.argtypes = [ctypes.c_uint8]
    l.or_e4m3_to_f32.restype = f
    l.or_quantize_e4m3_rows.argtypes = [P, i, i, P, P, i]
    l.or_gemm_f32.argtypes = [P, P, P, i, i, i, i]
    lg = ctypes.c_long
    d = ctypes.c_double
    l.or_perf_sigmoid.argtypes = [i, P, P, lg, i, i]
    l.or_perf_sigmoid.restype = d
    l.or_perf_brightness.argtypes = [i, P, P, lg, i, i, i, i]
    l.or_perf_brightness.restype = d
    l.or_perf_blur5.argtypes = [i, i, P, P, i, i, i, i, lg, i, i]
    l.or_perf_blur5.restype = d
    l.or_perf_blur5_from.argtypes = [i, i, P, P, i, i, i, i, lg, lg, i, i]
    l.or_perf_blur5_from.restype = d
    l.or_perf_cross_blur.argtypes = [i, P, i, i, lg, i, i]
    l.or_perf_cross_blur.restype = d


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def binary_f32(op: int, first, second) -> np.ndarray:
    a = np.ascontiguousarray(first, np.float32)
    b = np.ascontiguousarray(second, np.float32)
    out = np.empty_like(a)
    lib().or_binary_f32(op, _p(a), _p(b), _p(out), a.size)
    return out


def fill_f32(value: float, count: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().or_fill_f32(value, _p(out), count)
    return out


def saxpy_f32(a: float, x, y) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    out = np.empty_like(x)
    lib().or_saxpy_f32(a, _p(x), _p(y), _p(out), x.size)
    return out


def sigmoid_f32(x, nthreads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().or_sigmoid_f32(_p(x), _p(y), x.size, nthreads)
    return y


def adjust_brightness(img, delta: int, channels: int = 4, all_channels: bool = False,
                      nthreads: int = 1) -> np.ndarray:
    img = np.ascontiguousarray(img, np.uint8)
    out = np.empty_like(img)
    lib().or_adjust_brightness(_p(img), _p(out), img.size // channels, channels, int(delta),
                               int(all_channels), nthreads)
    return out


def blur5_reference(img, width: int, height: int, channels: int = 4,
                    nthreads: int = 1) -> np.ndarray:
    img = np.ascontiguousarray(img, np.uint8)
    assert img.size == width * height * channels
    out = np.empty_like(img)
    lib().or_blur5_reference(_p(img), _p(out), width, height, channels, nthreads)
    return out


def blur5_config(img, width: int, height: int, channels: int = 4,
                 nthreads: int = 1) -> np.ndarray:
    img = np.ascontiguousarray(img, np.uint8)
    assert img.size == width * height * channels
    out = np.empty_like(img)
    lib().or_blur5_config(_p(img), _p(out), width, height, channels, nthreads)
    return out


def brightness_blur5_config(img, width: int, height: int, delta: int, channels: int = 4,
                            all_channels: bool = False, nthreads: int = 1) -> np.ndarray:
    img = np.ascontiguousarray(img, np.uint8)
    assert img.size == width * height * channels
    out = np.empty_like(img)
    lib().or_brightness_blur5_config(_p(img), _p(out), width, height, channels, int(delta),
                                     int(all_channels), nthreads)
    return out


def bgr_to_rgba(src, width: int, height: int, bytes_per_pixel: int, src_stride: int) -> np.ndarray:
    """CreateColorImageFromBitmapData (Cuda.Tests/BlurPerformanceTests.cs:87-101):
    R, G, B = bitmap bytes 2, 1, 0 of each pixel, alpha 0 (a new zeroed array)."""
    src = np.asarray(src, np.uint8)
    rows = np.lib.stride_tricks.as_strided(
        src, (height, width, bytes_per_pixel), (src_stride, bytes_per_pixel, 1))
    out = np.zeros((height, width, 4), np.uint8)
    out[..., 0], out[..., 1], out[..., 2] = rows[..., 2], rows[..., 1], rows[..., 0]
    return out.reshape(-1)


def rgb_to_bgr(src, width: int, height: int, dst_stride: int, dst) -> np.ndarray:
    """SwitchRgbToBgr (Cuda.Tests/BlurPerformanceTests.cs:202-213) into a copy
    of `dst`: bitmap byte y * stride + 3 x + c = RGB byte 3 (y w + x) + 2 - c;
    the row padding keeps dst's bytes."""
    rgb = np.asarray(src, np.uint8).reshape(height, width, 3)
    out = np.array(dst, np.uint8, copy=True)
    for y in range(height):
        out[y * dst_stride:y * dst_stride + 3 * width] = rgb[y, :, ::-1].reshape(-1)
    return out


def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_array(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_bf16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def e4m3_to_f32(q) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    out = np.empty(q.shape, np.float32)
    lib().or_e4m3_to_f32_array(_p(q), _p(out), q.size)
    return out


def f32_to_e4m3_scalar(f: float) -> int:
    return int(lib().or_f32_to_e4m3(f))


def quantize_e4m3_rows(w, nthreads: int | None = None):
    """Per-row OCP E4M3 quantization: returns (q uint8 [rows, cols], scales f32 [rows])."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty(rows, np.float32)
    lib().or_quantize_e4m3_rows(_p(w), rows, cols, _p(q), _p(s),
                                nthreads or default_threads())
    return q, s


def gemm_f32(a, b, nthreads: int | None = None) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().or_gemm_f32(_p(a), _p(b), _p(c), m, n, k, nthreads or default_threads())
    return c


# ---- TestPerformance's CPU modes (Strict.Compiler.Cuda.Tests/TestPerformance.cs:34-49) ----

PERF_MODES = ("SingleThread", "SingleThreadChunks", "ParallelCpu", "ParallelCpuChunks")
CHUNK_SIZE = 100  # the reference tests' ChunkSize (SigmoidPerformanceTests.cs:20, Cuda BlurPerformanceTests.cs:40)
BLUR_REFERENCE, BLUR_CONFIG, BLUR_FUSED = 0, 1, 2


def perf_sigmoid(mode: int, x, y, nthreads: int, chunk: int = CHUNK_SIZE) -> float:
    """ms for one TestPerformance mode of sigmoid over the array x -> y."""
    return lib().or_perf_sigmoid(mode, _p(x), _p(y), x.size, chunk, nthreads)


def perf_brightness(mode: int, img, out, channels: int, delta: int, nthreads: int,
                    pixels: int | None = None, chunk: int = CHUNK_SIZE) -> float:
    n = img.size // channels if pixels is None else pixels
    return lib().or_perf_brightness(mode, _p(img), _p(out), n, channels, delta, chunk, nthreads)


def perf_blur5(mode: int, kind: int, img, out, width: int, height: int, channels: int,
               nthreads: int, delta: int = 0, pixels: int | None = None,
               chunk: int = CHUNK_SIZE) -> float:
    n = width * height if pixels is None else pixels
    return lib().or_perf_blur5(mode, kind, _p(img), _p(out), width, height, channels, delta, n,
                               chunk, nthreads)


def perf_blur5_from(mode: int, kind: int, img, out, width: int, height: int, channels: int,
                    nthreads: int, first: int, pixels: int, delta: int = 0,
                    chunk: int = CHUNK_SIZE) -> float:
    """ms for one mode over output pixels [first, first + pixels) (a CudaGpuAndCpu CPU share)."""
    return lib().or_perf_blur5_from(mode, kind, _p(img), _p(out), width, height, channels, delta,
                                    first, pixels, chunk, nthreads)


def perf_cross_blur(mode: int, image, width: int, height: int, iterations: int, nthreads: int,
                    chunk: int = CHUNK_SIZE) -> float:
    """ms for one mode of the CUDA harness's in-place cross blur (modifies image)."""
    assert image.size == width * height * 4
    return lib().or_perf_cross_blur(mode, _p(image), width, height, iterations, chunk, nthreads)
