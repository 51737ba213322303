"""strict_amd -- Python host surface of libstrict_hip (MI355X / gfx950).

Mirrors the object surface the reference's C# code uses through ManagedCuda
(Strict.Compiler.Cuda/Kernel.cs, Strict.Compiler.Cuda.Tests/*.cs):

=============================  ==============================================
reference (ManagedCuda)         here
=============================  ==============================================
``new CudaContext(0)``          ``Context(0)``
``CudaDeviceVariable<T>``       ``DeviceVariable`` (``Context.upload``/``alloc``)
``CudaRuntimeCompiler``         ``RuntimeCompiler`` (hipRTC, gfx950)
``ctx.LoadKernelPTX(code, n)``  ``Context.load_kernel(code, name)``
``CudaKernel.Run(args...)``     ``KernelFunction.run(*args)`` (sync, returns ms)
``Kernel`` (Kernel.cs:7)        ``Kernel``
``NVRTCException``              ``CompileError``
=============================  ==============================================

Every call goes through the C ABI in ``include/strict_hip.h``; the typed ops
(``sigmoid``, ``adjust_brightness``, ``box_blur5`` ...) run hand-written HIP
kernels. Nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes
from typing import Iterable, Sequence

import numpy as np

from . import _lib
from ._lib import (SH_ERR_COMPILE, SH_ERR_INVALID_ARGUMENT, SH_ERR_NO_DEVICE, SH_ERR_NOT_FOUND,
                   SH_OK, STATUS_NAMES)

__all__ = [
    "StrictHipError", "CompileError", "Context", "DeviceVariable", "RuntimeCompiler",
    "KernelFunction", "Module", "Kernel", "device_count", "SAXPY_SOURCE",
    "ADD", "SUBTRACT", "MULTIPLY", "DIVIDE", "BLUR_CONFIG", "BLUR_REFERENCE",
    "BRIGHTNESS_ALL_CHANNELS",
]

ADD, SUBTRACT, MULTIPLY, DIVIDE = 0, 1, 2, 3
BLUR_CONFIG, BLUR_REFERENCE = 0, 1
BRIGHTNESS_ALL_CHANNELS = 1


class StrictHipError(RuntimeError):
    """A non-zero sh_status with the library's sh_last_error() text."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.message = message
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


class CompileError(StrictHipError):
    """hipRTC compile failure (the reference's NVRTCException); carries the log."""

    def __init__(self, status: int, message: str, log: str):
        super().__init__(status, message)
        self.log = log


def _check(status: int) -> None:
    if status != SH_OK:
        msg = _lib.load().sh_last_error()
        raise StrictHipError(status, msg.decode(errors="replace") if msg else "")


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(_lib.load().sh_device_count(ctypes.byref(n)))
    return n.value


def _ptr(x) -> ctypes.c_void_p:
    if isinstance(x, DeviceVariable):
        return ctypes.c_void_p(x.ptr)
    if isinstance(x, int):
        return ctypes.c_void_p(x)
    if x is None:
        return ctypes.c_void_p(0)
    raise TypeError(f"expected a DeviceVariable or device address, got {type(x).__name__}")


class DeviceVariable:
    """Device buffer owned by a Context (CudaDeviceVariable<T>)."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int, dtype=np.uint8, shape=None):
        self.ctx = ctx
        self.ptr = ptr
        self.nbytes = nbytes
        self.dtype = np.dtype(dtype)
        self.shape = tuple(shape) if shape is not None else (nbytes // self.dtype.itemsize,)

    @property
    def device_pointer(self) -> int:
        return self.ptr

    @property
    def size(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    def copy_from_host(self, host) -> None:
        a = np.ascontiguousarray(host)
        if a.nbytes > self.nbytes:
            raise ValueError(f"host array of {a.nbytes} B does not fit {self.nbytes} B")
        _check(self.ctx._l.sh_upload(self.ctx.handle, ctypes.c_void_p(self.ptr),
                                     a.ctypes.data_as(ctypes.c_void_p), a.nbytes))

    def to_host(self, dtype=None, shape=None) -> np.ndarray:
        dtype = np.dtype(dtype) if dtype is not None else self.dtype
        shape = shape if shape is not None else (
            self.shape if dtype == self.dtype else (self.nbytes // dtype.itemsize,))
        out = np.empty(shape, dtype)
        _check(self.ctx._l.sh_download(self.ctx.handle, out.ctypes.data_as(ctypes.c_void_p),
                                       ctypes.c_void_p(self.ptr), out.nbytes))
        return out

    def view(self, offset_bytes: int, nbytes: int, dtype=None, shape=None) -> "DeviceVariable":
        """A non-owning sub-range (address arithmetic only)."""
        if offset_bytes < 0 or offset_bytes + nbytes > self.nbytes:
            raise ValueError("view outside the buffer")
        v = DeviceVariable.__new__(DeviceVariable)
        v.ctx, v.ptr, v.nbytes = self.ctx, self.ptr + offset_bytes, nbytes
        v.dtype = np.dtype(dtype) if dtype is not None else self.dtype
        v.shape = tuple(shape) if shape is not None else (nbytes // v.dtype.itemsize,)
        v._view = True
        return v

    def free(self) -> None:
        if getattr(self, "_view", False):
            return
        if self.ptr and self.ctx.handle:
            _check(self.ctx._l.sh_free(self.ctx.handle, ctypes.c_void_p(self.ptr)))
        self.ptr = 0

    dispose = free

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()


class RuntimeCompiler:
    """hipRTC program (CudaRuntimeCompiler): compile(options), code, log."""

    def __init__(self, source: str, name: str):
        self.source = source
        self.name = name
        self._prog = ctypes.c_void_p(0)
        self._l = _lib.load()

    def compile(self, options: Sequence[str] = ()) -> None:
        self._release()
        opts = (ctypes.c_char_p * max(1, len(options)))(*[o.encode() for o in options])
        status = self._l.sh_compile(self.source.encode(), self.name.encode(), opts, len(options),
                                    ctypes.byref(self._prog))
        if status != SH_OK:
            msg = (self._l.sh_last_error() or b"").decode(errors="replace")
            raise CompileError(status, msg, self.get_log())

    def get_log(self) -> str:
        if not self._prog:
            return ""
        return (self._l.sh_program_log(self._prog) or b"").decode(errors="replace")

    def get_code(self) -> bytes:
        code = ctypes.c_void_p(0)
        size = ctypes.c_size_t(0)
        _check(self._l.sh_program_code(self._prog, ctypes.byref(code), ctypes.byref(size)))
        return ctypes.string_at(code, size.value)

    def _release(self) -> None:
        if self._prog:
            self._l.sh_program_destroy(self._prog)
            self._prog = ctypes.c_void_p(0)

    def dispose(self) -> None:
        self._release()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


def _arg(value):
    """Launch-argument marshalling: DeviceVariable -> pointer, Python int ->
    int32 (C# int), Python float -> float32 (C# float); ctypes values pass
    through unchanged (e.g. ctypes.c_size_t for size_t parameters)."""
    if isinstance(value, DeviceVariable):
        return ctypes.c_void_p(value.ptr)
    if isinstance(value, ctypes._SimpleCData):
        return value
    if isinstance(value, bool):
        return ctypes.c_int(int(value))
    if isinstance(value, int):
        return ctypes.c_int(value)
    if isinstance(value, float):
        return ctypes.c_float(value)
    raise TypeError(f"unsupported kernel argument {value!r}")


class KernelFunction:
    """A loaded kernel (CudaKernel) with settable grid/block dimensions (default 1)."""

    def __init__(self, module: "Module", handle: ctypes.c_void_p, name: str):
        self.module = module
        self.handle = handle
        self.name = name
        self.grid_dimensions = (1, 1, 1)
        self.block_dimensions = (1, 1, 1)
        self.dynamic_shared_memory = 0

    @staticmethod
    def _dim3(d) -> tuple:
        if isinstance(d, int):
            return (d, 1, 1)
        d = tuple(d) + (1,) * (3 - len(d))
        return d[:3]

    def run(self, *args) -> float:
        """Launches synchronously and returns the kernel time in ms."""
        vals = [_arg(a) for a in args]
        ptrs = (ctypes.c_void_p * max(1, len(vals)))(
            *[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in vals])
        g = (ctypes.c_uint * 3)(*self._dim3(self.grid_dimensions))
        b = (ctypes.c_uint * 3)(*self._dim3(self.block_dimensions))
        ms = ctypes.c_float(0)
        _check(self.module.ctx._l.sh_launch(self.handle, g, b, self.dynamic_shared_memory,
                                            ptrs, ctypes.byref(ms)))
        return ms.value


class Module:
    def __init__(self, ctx: "Context", handle: ctypes.c_void_p, code: bytes):
        self.ctx = ctx
        self.handle = handle
        self._code = code  # keep the image alive while loaded

    def function(self, name: str) -> KernelFunction:
        f = ctypes.c_void_p(0)
        _check(self.ctx._l.sh_module_function(self.handle, name.encode(), ctypes.byref(f)))
        return KernelFunction(self, f, name)

    def unload(self) -> None:
        if self.handle:
            _check(self.ctx._l.sh_module_unload(self.handle))
            self.handle = ctypes.c_void_p(0)


class Context:
    """One device + one ordered stream (CudaContext). Typed ops are methods."""

    def __init__(self, device: int = 0):
        self._l = _lib.load()
        self.handle = ctypes.c_void_p(0)
        _check(self._l.sh_create(device, ctypes.byref(self.handle)))
        self.device = device

    # -- lifetime --
    def dispose(self) -> None:
        if self.handle:
            self._l.sh_destroy(self.handle)
            self.handle = ctypes.c_void_p(0)

    close = dispose

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()

    def __del__(self):
        try:
            self.dispose()
        except Exception:
            pass

    def info(self) -> dict:
        i = _lib.DeviceInfo()
        _check(self._l.sh_device_info(self.handle, ctypes.byref(i)))
        return {f: (getattr(i, f).decode() if isinstance(getattr(i, f), bytes) else getattr(i, f))
                for f, _ in i._fields_}

    def sync(self) -> None:
        _check(self._l.sh_sync(self.handle))

    def stream(self) -> int:
        s = ctypes.c_void_p(0)
        _check(self._l.sh_stream(self.handle, ctypes.byref(s)))
        return s.value or 0

    # -- buffers --
    def alloc(self, nbytes: int, dtype=np.uint8, shape=None) -> DeviceVariable:
        p = ctypes.c_void_p(0)
        _check(self._l.sh_alloc(self.handle, int(nbytes), ctypes.byref(p)))
        return DeviceVariable(self, p.value, int(nbytes), dtype, shape)

    def empty(self, shape, dtype) -> DeviceVariable:
        shape = (shape,) if isinstance(shape, int) else tuple(shape)
        nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return self.alloc(max(nbytes, 1), dtype, shape)

    def upload(self, host) -> DeviceVariable:
        """T[] -> CudaDeviceVariable<T> (allocate + host-to-device copy)."""
        a = np.ascontiguousarray(host)
        v = self.alloc(max(a.nbytes, 1), a.dtype, a.shape)
        if a.nbytes:
            v.copy_from_host(a)
        return v

    def memset(self, buf: DeviceVariable, value: int = 0) -> None:
        _check(self._l.sh_memset(self.handle, _ptr(buf), value, buf.nbytes))

    def copy(self, dst: DeviceVariable, src: DeviceVariable, nbytes: int | None = None) -> None:
        n = min(dst.nbytes, src.nbytes) if nbytes is None else nbytes
        _check(self._l.sh_copy(self.handle, _ptr(dst), _ptr(src), n))

    def register_external(self, ptr: int, nbytes: int) -> None:
        _check(self._l.sh_register_external(self.handle, ctypes.c_void_p(ptr), nbytes))

    def unregister_external(self, ptr: int) -> None:
        _check(self._l.sh_unregister_external(self.handle, ctypes.c_void_p(ptr)))

    # -- timing --
    def timer_start(self) -> None:
        _check(self._l.sh_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = ctypes.c_float(0)
        _check(self._l.sh_timer_stop(self.handle, ctypes.byref(ms)))
        return ms.value

    def event(self) -> "Event":
        return Event(self)

    # -- modules --
    def load_module(self, code: bytes) -> Module:
        buf = ctypes.create_string_buffer(code, len(code))
        m = ctypes.c_void_p(0)
        _check(self._l.sh_module_load(self.handle, buf, len(code), ctypes.byref(m)))
        return Module(self, m, buf)

    def load_kernel(self, code: bytes, name: str) -> KernelFunction:
        """ctx.LoadKernelPTX(ptx, name) counterpart for gfx950 code objects."""
        return self.load_module(code).function(name)

    # -- typed ops (device buffers in, device buffers out; stream-ordered) --
    def binary(self, op: int, first, second, output, count: int) -> None:
        _check(self._l.sh_binary_f32(self.handle, op, _ptr(first), _ptr(second), _ptr(output),
                                     count))

    def fill(self, value: float, output, count: int) -> None:
        _check(self._l.sh_fill_f32(self.handle, value, _ptr(output), count))

    def saxpy(self, a: float, x, y, out, n: int) -> None:
        _check(self._l.sh_saxpy_f32(self.handle, a, _ptr(x), _ptr(y), _ptr(out), n))

    def sigmoid(self, x, y, n: int) -> None:
        _check(self._l.sh_sigmoid_f32(self.handle, _ptr(x), _ptr(y), n))

    def adjust_brightness(self, src, dst, width: int, height: int, channels: int, delta: int,
                          flags: int = 0) -> None:
        _check(self._l.sh_adjust_brightness_u8(self.handle, _ptr(src), _ptr(dst), width, height,
                                               channels, delta, flags))

    def bgr_to_rgba(self, src, bytes_per_pixel: int, src_stride: int, dst, width: int,
                    height: int) -> None:
        """Bitmap BGR(A) pixels to RGBA with alpha 0 (sh_bgr_to_rgba_u8)."""
        _check(self._l.sh_bgr_to_rgba_u8(self.handle, _ptr(src), bytes_per_pixel, src_stride,
                                         _ptr(dst), width, height))

    def rgb_to_bgr(self, src, dst, width: int, height: int, dst_stride: int) -> None:
        """Packed RGB to 24-bpp bitmap rows (sh_rgb_to_bgr_u8)."""
        _check(self._l.sh_rgb_to_bgr_u8(self.handle, _ptr(src), _ptr(dst), width, height,
                                        dst_stride))

    def box_blur5(self, src, dst, width: int, height: int, channels: int,
                  mode: int = BLUR_CONFIG) -> None:
        _check(self._l.sh_box_blur5_u8(self.handle, _ptr(src), _ptr(dst), width, height,
                                       channels, mode))

    def brightness_blur5(self, src, dst, width: int, height: int, channels: int, delta: int,
                         flags: int = 0, mode: int = BLUR_CONFIG) -> None:
        _check(self._l.sh_brightness_blur5_u8(self.handle, _ptr(src), _ptr(dst), width, height,
                                              channels, delta, flags, mode))


    def gemm_bf16(self, a, b, c, m: int, n: int, k: int, lda: int | None = None,
                  ldb: int | None = None, ldc: int | None = None) -> None:
        """C[m,n] = A[m,k] @ B[k,n]; bf16 operands (uint16 bit patterns), fp32
        accumulation, bf16 result, row-major with leading dimensions."""
        _check(self._l.sh_gemm_bf16(self.handle, _ptr(a), _ptr(b), _ptr(c), m, n, k,
                                    k if lda is None else lda, n if ldb is None else ldb,
                                    n if ldc is None else ldc))


    def gemm_fp8(self, a, sa, bt, sb, c, m: int, n: int, k: int, lda: int | None = None,
                 ldb: int | None = None, ldc: int | None = None) -> None:
        """C[m,n] = sa[m] sb[n] (A[m,:] . Bt[n,:]); OCP E4M3 bytes A [m,k] and
        Bt [n,k] (B transposed), fp32 scales, fp32 accumulation, bf16 result."""
        _check(self._l.sh_gemm_fp8(self.handle, _ptr(a), _ptr(sa), _ptr(bt), _ptr(sb), _ptr(c),
                                   m, n, k, k if lda is None else lda, k if ldb is None else ldb,
                                   n if ldc is None else ldc))

    def quantize_e4m3(self, w, q, scales, n: int, k: int) -> None:
        """Per-row OCP E4M3 quantization of a device fp32 [n, k] matrix."""
        _check(self._l.sh_quantize_e4m3(self.handle, _ptr(w), n, k, _ptr(q), _ptr(scales)))

    def pack_e4m3_tiles(self, q, tiled, n: int, k: int) -> None:
        _check(self._l.sh_pack_e4m3_tiles(self.handle, _ptr(q), n, k, _ptr(tiled)))

    def gemv_w8a16(self, x, w_tiled, scales, y, batch: int, k: int, n: int) -> None:
        """y[b] = scales * (x[b] @ e4m3(q).T); x fp16 [batch, k], y fp32 [batch, n]."""
        _check(self._l.sh_gemv_w8a16(self.handle, _ptr(x), _ptr(w_tiled), _ptr(scales), _ptr(y),
                                     batch, k, n))

    # -- decoder building blocks (fp32 device buffers) --
    def rmsnorm(self, x, gain, y, rows: int, n: int, eps: float) -> None:
        """y = (x * fp32(1 / sqrt(mean(x^2) + eps))) * gain, per row of n."""
        _check(self._l.sh_rmsnorm_f32(self.handle, _ptr(x), _ptr(gain), _ptr(y), rows, n, eps))

    def layernorm(self, x, gain, bias, y, rows: int, n: int, eps: float) -> None:
        _check(self._l.sh_layernorm_f32(self.handle, _ptr(x), _ptr(gain), _ptr(bias), _ptr(y),
                                        rows, n, eps))

    def rope(self, x, positions, rows: int, heads: int, head_dim: int, theta: float) -> None:
        """Rotate-half RoPE in place on x [rows, heads, head_dim] at positions [rows] (int32)."""
        _check(self._l.sh_rope_f32(self.handle, _ptr(x), _ptr(positions), rows, heads, head_dim,
                                   theta))

    def swiglu(self, gate, up, out, n: int) -> None:
        _check(self._l.sh_swiglu_f32(self.handle, _ptr(gate), _ptr(up), _ptr(out), n))

    def gelu(self, x, y, n: int) -> None:
        _check(self._l.sh_gelu_f32(self.handle, _ptr(x), _ptr(y), n))

    def argmax(self, x, rows: int, n: int, index) -> None:
        _check(self._l.sh_argmax_f32(self.handle, _ptr(x), rows, n, _ptr(index)))

    def attn_decode(self, q, k, v, lengths, out, batch: int, heads: int, kv_heads: int,
                    head_dim: int, max_positions: int, scale: float) -> None:
        """Grouped-query decode attention of q [batch, heads, d] (fp32) over fp16
        caches [batch, kv_heads, max_positions, d] up to lengths [batch] (int32)."""
        _check(self._l.sh_attn_decode_f16(self.handle, _ptr(q), _ptr(k), _ptr(v), _ptr(lengths),
                                          _ptr(out), batch, heads, kv_heads, head_dim,
                                          max_positions, scale))

    def attn_decode_noalloc(self, q, k, v, lengths, out, batch: int, heads: int, kv_heads: int,
                            head_dim: int, max_positions: int, scale: float) -> None:
        """attn_decode without allocating: the partials use the library's fixed
        per-GPU array (SH_ATTN_NOALLOC_MAX_BYTES); concurrent calls on one GPU race."""
        _check(self._l.sh_attn_decode_f16_noalloc(self.handle, _ptr(q), _ptr(k), _ptr(v),
                                                  _ptr(lengths), _ptr(out), batch, heads,
                                                  kv_heads, head_dim, max_positions, scale))


class Event:
    """A HIP event on a context's stream (per-launch timing)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.handle = ctypes.c_void_p(0)
        _check(ctx._l.sh_event_create(ctx.handle, ctypes.byref(self.handle)))

    def record(self) -> None:
        _check(self.ctx._l.sh_event_record(self.handle))

    def elapsed_ms(self, stop: "Event") -> float:
        """ms from this event to `stop` (waits for `stop`)."""
        ms = ctypes.c_float(0)
        _check(self.ctx._l.sh_event_elapsed(self.handle, stop.handle, ctypes.byref(ms)))
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            self.ctx._l.sh_event_destroy(self.handle)
            self.handle = ctypes.c_void_p(0)


SAXPY_SOURCE = r'''extern "C" __global__ void saxpy(float a, float *x, float *y, float *out, size_t n)
{
  size_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (tid < n) {
    out[tid] = a * x[tid] + y[tid];
  }
}'''


class Kernel:
    """Kernel.cs:7-58: owns a context on device 0; compiles the fixed saxpy
    with the runtime compiler and writes the code object to a file (the
    reference writes VectorAdd.ptx)."""

    def __init__(self, device: int = 0):
        self.context = Context(device)

    def compile_kernel_and_save_code_object(self, path: str = "VectorAdd.hsaco") -> int:
        """Returns SH_OK or the compile status (CompileInTryCatch, Kernel.cs:36-52)."""
        with RuntimeCompiler(SAXPY_SOURCE, "saxpy") as rtc:
            try:
                rtc.compile(["--offload-arch=gfx950"])
            except CompileError as e:
                return e.status
            with open(path, "wb") as f:
                f.write(rtc.get_code())
        return SH_OK

    def dispose(self) -> None:
        self.context.dispose()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()
