"""hipBLASLt GEMMs as the benchmark's yardstick for the hand-written kernels.

Loads ``libsh_blaslt_yardstick.so`` (strict_amd/csrc/yardstick/blaslt.cpp),
a library of its own: ``libstrict_hip.so`` does not link it and the package
does not import this module, so ``sh_gemm_bf16`` / ``sh_gemm_fp8`` always run
the hand-written MFMA kernels. ``bench.py`` and the yardstick's parity tests
use it to time and check the vendor GEMM on the same device buffers, on the
library context's stream.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsh_blaslt_yardstick.so"
OK, ERR_HIP, UNSUPPORTED = 0, 3, 7

_lib = None


class YardstickError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"hipBLASLt yardstick status {status}: {message}")
        self.status = status


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is not built (make -C strict_amd/csrc)")
        l = ctypes.CDLL(str(LIB_PATH))
        P, i = ctypes.c_void_p, ctypes.c_int
        l.shy_gemm_bf16.argtypes = [P, P, P, P, i, i, i, i, i, i]
        l.shy_gemm_bf16.restype = i
        l.shy_gemm_fp8.argtypes = [P, P, P, P, P, P, i, i, i, i, i, i]
        l.shy_gemm_fp8.restype = i
        l.shy_last_error.restype = ctypes.c_char_p
        l.shy_release.restype = None
        _lib = l
    return _lib


def _check(status: int) -> None:
    if status != OK:
        raise YardstickError(status, load().shy_last_error().decode(errors="replace"))


def gemm_bf16(ctx, A, B, C, M, N, K, lda=None, ldb=None, ldc=None) -> None:
    """C = A B through hipBLASLt (sh_gemm_bf16's operand conventions)."""
    _check(load().shy_gemm_bf16(ctx.stream(), A.ptr, B.ptr, C.ptr, M, N, K, lda or K, ldb or N,
                                ldc or N))


def gemm_fp8(ctx, A, sa, Bt, sb, C, M, N, K, lda=None, ldb=None, ldc=None) -> None:
    """C = (sa sb^T) * (A Bt^T) through hipBLASLt (sh_gemm_fp8's conventions)."""
    _check(load().shy_gemm_fp8(ctx.stream(), A.ptr, sa.ptr, Bt.ptr, sb.ptr, C.ptr, M, N, K,
                               lda or K, ldb or K, ldc or N))


def release() -> None:
    if _lib is not None:
        _lib.shy_release()
