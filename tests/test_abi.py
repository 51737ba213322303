"""C-ABI surface checks that need no GPU: the library loads, exports every
entry point include/*.h declares, and its argument checks and error reporting
behave as documented (status code + thread-local sh_last_error)."""
import ctypes
import re
import threading
from pathlib import Path

import numpy as np
import pytest

import strict_amd
from strict_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"SH_API\s+[\w\s\*]+?\b(sh_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "sh_create" in names and "sh_sigmoid_f32" in names and len(names) >= 30


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_every_symbol():
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def _arity(params: str) -> int:
    params = params.strip()
    return 0 if params in ("", "void") else params.count(",") + 1


def declared_arities():
    out = {}
    for h in (ROOT / "include").glob("*.h"):
        for name, params in re.findall(r"SH_API\s+[\w\s\*]+?\b(sh_\w+)\s*\(([^)]*)\)", h.read_text()):
            out[name] = _arity(params)
    return out


def csharp_bindings():
    """name -> parameter count of every `static extern` in INTEGRATION.md's C# blocks."""
    text = (ROOT / "INTEGRATION.md").read_text()
    out = {}
    for block in re.findall(r"```csharp\n(.*?)```", text, re.S):
        block = re.sub(r"\[(?:MarshalAs|In|Out)\b[^\]]*\]", "", block)  # parameter attributes
        for name, params in re.findall(r"static\s+extern\s+[\w\[\]\?]+\s+(sh_\w+)\s*\(([^)]*)\)", block):
            out[name] = _arity(params)
    return out


def test_csharp_binding_covers_every_symbol():
    # the P/Invoke layer a C# host adds declares every
    # export of include/*.h, with the header's parameter count
    declared, bound = declared_arities(), csharp_bindings()
    assert set(declared) == set(declared_symbols())
    missing = sorted(set(declared) - set(bound))
    extra = sorted(set(bound) - set(declared))
    assert not missing and not extra, (missing, extra)
    wrong = {n: (declared[n], bound[n]) for n in declared if declared[n] != bound[n]}
    assert not wrong, wrong


def test_version_and_device_count():
    l = _lib.load()
    assert l.sh_version() >= 10000
    n = ctypes.c_int(-1)
    assert l.sh_device_count(ctypes.byref(n)) == 0
    assert n.value >= 0


def test_null_arguments_are_rejected():
    l = _lib.load()
    assert l.sh_device_count(None) == _lib.SH_ERR_INVALID_ARGUMENT
    assert b"NULL" in l.sh_last_error()
    assert l.sh_create(0, None) == _lib.SH_ERR_INVALID_ARGUMENT
    assert l.sh_sync(None) == _lib.SH_ERR_INVALID_ARGUMENT
    assert l.sh_sigmoid_f32(None, None, None, 4) == _lib.SH_ERR_INVALID_ARGUMENT
    assert l.sh_destroy(None) == 0  # destroying nothing is a no-op


def test_last_error_is_thread_local():
    l = _lib.load()
    assert l.sh_sync(None) == _lib.SH_ERR_INVALID_ARGUMENT
    seen = {}

    def worker():
        seen["msg"] = l.sh_last_error()

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert seen["msg"] == b""
    assert l.sh_last_error() != b""


def test_create_without_device_reports_no_device():
    if strict_amd.device_count() > 0:
        pytest.skip("a device is visible")
    with pytest.raises(strict_amd.StrictHipError) as e:
        strict_amd.Context(0)
    assert e.value.status == _lib.SH_ERR_NO_DEVICE


def test_runtime_compile_saxpy_and_log():
    # Kernel.CompileKernelAndSaveAsPtxFile (Kernel.cs:19-33) compiles the fixed saxpy
    with strict_amd.RuntimeCompiler(strict_amd.SAXPY_SOURCE, "saxpy") as rtc:
        rtc.compile(["--offload-arch=gfx950"])
        code = rtc.get_code()
    assert code[:4] == b"\x7fELF"  # an AMDGPU code object


def test_runtime_compile_error_carries_log():
    # NVRTCException + GetLogAsString (Cuda BlurPerformanceTests.cs:131-135)
    src = 'extern "C" __global__ void broken(float *x) { x[0] = not_declared; }'
    with strict_amd.RuntimeCompiler(src, "broken") as rtc:
        with pytest.raises(strict_amd.CompileError) as e:
            rtc.compile()
    assert e.value.status == _lib.SH_ERR_COMPILE
    assert "not_declared" in e.value.log


def test_empty_source_is_invalid():
    # CSharpToCudaTranspilerTests.EmptyInputWillNotWork: empty input throws
    with pytest.raises(strict_amd.StrictHipError) as e:
        strict_amd.RuntimeCompiler("", "empty").compile()
    assert e.value.status == _lib.SH_ERR_INVALID_ARGUMENT


def test_program_destroy_null_is_ok():
    assert _lib.load().sh_program_destroy(None) == 0
