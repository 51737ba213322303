"""BinaryExecutable over the C ABI: .strictbinary loading and kernel inputs.

Mirrors Strict.Bytecode's BinaryExecutable (BinaryExecutable.cs:19-160): a
.strictbinary ZIP of "<type>.bytecode" entries loads into `methods_per_type`
(type full name -> BinaryType with members and method groups), `entry_point`
is the first Run overload, `find_instructions` picks an overload by name,
parameter count and return type, `serialize` writes the file back. Parsing,
the ZIP and the serializer are libstrict_hip's (sh_strictbinary_*, native
C++); this module only shapes the results. On top of the reference's API,
`constants` lists a method's Number / List(Number) constants and
`upload_f32` puts one into a device buffer as a kernel input, and a loaded
binary feeds `InstructionsToHip.compile_binary` as the reference's
`Compile(BinaryExecutable, Platform)` does (InstructionsToCuda.cs:14-15).

Errors raise the reference's exception types: InvalidFile,
InvalidBytecodeEntry (BinaryType.cs:66), InvalidVersion (:69).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from . import _lib
from .codegen import Instruction, InstructionType, Method, Parameter

__all__ = ["BinaryExecutable", "BinaryType", "BinaryMethod", "BinaryMember", "Constant",
           "InvalidFile", "InvalidBytecodeEntry", "InvalidVersion", "EXTENSION",
           "BYTECODE_ENTRY_EXTENSION", "RUN"]

EXTENSION = ".strictbinary"             # BinaryExecutable.Extension (cs:159)
BYTECODE_ENTRY_EXTENSION = ".bytecode"  # BinaryType.BytecodeEntryExtension (BinaryType.cs:64)
RUN = "Run"                             # Method.Run


def _error_base():
    from . import StrictHipError
    return StrictHipError


class InvalidFile(Exception):
    """BinaryExecutable.InvalidFile (cs:102) and format errors of the stream."""


class InvalidBytecodeEntry(InvalidFile):
    """BinaryType.InvalidBytecodeEntry (BinaryType.cs:66): bad magic bytes."""


class InvalidVersion(InvalidFile):
    """BinaryType.InvalidVersion (BinaryType.cs:69-70): version 0 or newer than 1."""


_KINDS = {"InvalidFile": InvalidFile, "InvalidBytecodeEntry": InvalidBytecodeEntry,
          "InvalidVersion": InvalidVersion}


def _check(lib, status):
    if status == _lib.SH_OK:
        return
    msg = (lib.sh_last_error() or b"").decode(errors="replace")
    if status == _lib.SH_ERR_INVALID_FILE:
        kind, _, text = msg.partition(": ")
        raise _KINDS.get(kind, InvalidFile)(text)
    raise _error_base()(status, msg)


def _s(b: Optional[bytes]) -> Optional[str]:
    return None if b is None else b.decode("utf-8", errors="surrogateescape")


@dataclass(frozen=True)
class BinaryMember:
    """BinaryMember (Serialization/BinaryMember.cs:6-20)."""
    name: str
    full_type_name: str
    has_initial_value: bool = False

    @property
    def just_type_name(self) -> str:
        return self.full_type_name.split("/")[-1]

    def __str__(self):
        return f"{self.name} {self.just_type_name}"


@dataclass(frozen=True)
class Constant:
    """A value-carrying instruction (LoadConstant, StoreConstantToVariable,
    Set) or a member's initial value; `count` Numbers (0 if not numeric)."""
    index: int
    instruction: int
    instruction_type: int
    kind: int
    register: int
    identifier: Optional[str]
    count: int


@dataclass
class BinaryMethod:
    """BinaryMethod (Serialization/BinaryMethod.cs:5-47)."""
    name: str
    parameters: List[BinaryMember]
    return_type_name: str
    instructions: List[Instruction]
    type_index: int = field(repr=False, default=-1)
    method_index: int = field(repr=False, default=-1)

    def as_codegen_method(self) -> Method:
        """This overload as a method InstructionsToHip.compile takes."""
        params = [Parameter(p.name, p.just_type_name) for p in self.parameters]
        return Method(self.name, params, "", self.return_type_name.split("/")[-1],
                      _instructions=list(self.instructions))


@dataclass
class BinaryType:
    """BinaryType (Serialization/BinaryType.cs:9-143): members and method groups."""
    type_full_name: str
    members: List[BinaryMember]
    method_groups: Dict[str, List[BinaryMethod]]
    type_index: int = field(repr=False, default=-1)

    @property
    def just_type_name(self) -> str:
        return self.type_full_name.split("/")[-1]

    @property
    def total_instruction_count(self) -> int:
        return sum(len(m.instructions) for ms in self.method_groups.values() for m in ms)

    @staticmethod
    def reconstruct_method_name(method_name: str, method: BinaryMethod) -> str:
        """ReconstructMethodName (BinaryType.cs:139-142)."""
        params = "(" + ", ".join(str(p) for p in method.parameters) + ")" if method.parameters else ""
        rt = "" if method.return_type_name == "None" else " " + method.return_type_name
        return method_name + params + rt


def _instruction(bc: _lib.BcInstruction) -> Instruction:
    try:
        kind = InstructionType(bc.type)
    except ValueError:
        kind = bc.type  # a type the kernel generator does not read
    regs = tuple(bc.registers[i] for i in range(min(bc.register_count, 3)))
    return Instruction(kind, regs, _s(bc.identifier), float(bc.number))


class BinaryExecutable:
    """A loaded .strictbinary (BinaryExecutable(string filePath), cs:34-61)."""

    Extension = EXTENSION

    def __init__(self, file_path: Optional[str] = None, *, data: Optional[bytes] = None):
        if (file_path is None) == (data is None):
            raise ValueError("give a file path or the file's bytes")
        if data is None:
            with open(file_path, "rb") as f:
                data = f.read()
        self._lib = _lib.load()
        handle = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(data, len(data))
        _check(self._lib, self._lib.sh_strictbinary_load(buf, len(data), ctypes.byref(handle)))
        self._handle = handle
        self.methods_per_type: Dict[str, BinaryType] = {}
        self._types: List[BinaryType] = []
        self._read_types()

    # -- object model ---------------------------------------------------------

    def _read_types(self):
        lib, h = self._lib, self._handle
        n = ctypes.c_int()
        _check(lib, lib.sh_strictbinary_type_count(h, ctypes.byref(n)))
        for t in range(n.value):
            name, members, methods = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
            _check(lib, lib.sh_strictbinary_type(h, t, ctypes.byref(name), ctypes.byref(members),
                                                 ctypes.byref(methods)))
            groups: Dict[str, List[BinaryMethod]] = {}
            for m in range(methods.value):
                method = self._read_method(t, m)
                groups.setdefault(method.name, []).append(method)
            bt = BinaryType(_s(name.value), [self._member(t, -1, i) for i in range(members.value)],
                            groups, t)
            self._types.append(bt)
            self.methods_per_type[bt.type_full_name] = bt

    def _member(self, t: int, m: int, i: int) -> BinaryMember:
        name, type_name, init = ctypes.c_char_p(), ctypes.c_char_p(), ctypes.c_int()
        _check(self._lib, self._lib.sh_strictbinary_member(
            self._handle, t, m, i, ctypes.byref(name), ctypes.byref(type_name), ctypes.byref(init)))
        return BinaryMember(_s(name.value), _s(type_name.value), bool(init.value))

    def _read_method(self, t: int, m: int) -> BinaryMethod:
        lib, h = self._lib, self._handle
        name, params, ret, count = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_char_p(), ctypes.c_int()
        _check(lib, lib.sh_strictbinary_method(h, t, m, ctypes.byref(name), ctypes.byref(params),
                                               ctypes.byref(ret), ctypes.byref(count)))
        arr = (_lib.BcInstruction * max(1, count.value))()
        got = ctypes.c_int()
        _check(lib, lib.sh_strictbinary_instructions(h, t, m, arr, count.value, ctypes.byref(got)))
        return BinaryMethod(_s(name.value), [self._member(t, m, i) for i in range(params.value)],
                            _s(ret.value), [_instruction(arr[i]) for i in range(got.value)], t, m)

    # -- the reference's queries ----------------------------------------------

    def get_run_methods(self) -> List[BinaryMethod]:
        """GetRunMethods (cs:104-111)."""
        return [m for bt in self._types for m in bt.method_groups.get(RUN, [])]

    @property
    def entry_point(self) -> BinaryMethod:
        """EntryPoint (cs:101, :113-120); InvalidOperationException -> LookupError."""
        t, m = ctypes.c_int(), ctypes.c_int()
        status = self._lib.sh_strictbinary_entry_point(self._handle, ctypes.byref(t), ctypes.byref(m))
        if status == _lib.SH_ERR_NOT_FOUND:
            raise LookupError("No Run entry point found in binary executable")
        _check(self._lib, status)
        bt = self._types[t.value]
        return next(x for ms in bt.method_groups.values() for x in ms if x.method_index == m.value)

    def to_instructions(self) -> List[Instruction]:
        """ToInstructions (cs:158)."""
        return list(self.entry_point.instructions)

    def find_method(self, full_type_name: str, method_name: str, parameters_count: int,
                    return_type: str = "") -> Optional[BinaryMethod]:
        t, m = ctypes.c_int(), ctypes.c_int()
        status = self._lib.sh_strictbinary_find(
            self._handle, full_type_name.encode(), method_name.encode(), parameters_count,
            return_type.encode(), ctypes.byref(t), ctypes.byref(m))
        if status == _lib.SH_ERR_NOT_FOUND:
            return None
        _check(self._lib, status)
        bt = self._types[t.value]
        return next(x for ms in bt.method_groups.values() for x in ms if x.method_index == m.value)

    def find_instructions(self, full_type_name: str, method_name: str, parameters_count: int,
                          return_type: str = "") -> Optional[List[Instruction]]:
        """FindInstructions (cs:125-142)."""
        method = self.find_method(full_type_name, method_name, parameters_count, return_type)
        return None if method is None else list(method.instructions)

    # -- constants as kernel inputs -------------------------------------------

    def constants(self, method: Optional[BinaryMethod] = None, *,
                  type_full_name: Optional[str] = None) -> List[Constant]:
        """The value-carrying instructions of `method`, or the initial values of
        the members of type `type_full_name`."""
        t, m = self._where(method, type_full_name)
        n = ctypes.c_int()
        _check(self._lib, self._lib.sh_strictbinary_constants(self._handle, t, m, None, 0,
                                                              ctypes.byref(n)))
        arr = (_lib.StrictBinaryConstant * max(1, n.value))()
        _check(self._lib, self._lib.sh_strictbinary_constants(self._handle, t, m, arr, n.value,
                                                              ctypes.byref(n)))
        return [Constant(i, c.instruction, c.instruction_type, c.kind, c.register_id,
                         _s(c.identifier), int(c.count)) for i, c in enumerate(arr[:n.value])]

    def constant_values(self, constant: Constant, method: Optional[BinaryMethod] = None, *,
                        type_full_name: Optional[str] = None) -> np.ndarray:
        """The Numbers of a Number / List(Number) constant, as float64."""
        t, m = self._where(method, type_full_name)
        out = np.zeros(max(1, constant.count), np.float64)
        _check(self._lib, self._lib.sh_strictbinary_constant_values(
            self._handle, t, m, constant.index, out.ctypes.data, out.size))
        return out[:constant.count].copy()

    def upload_f32(self, ctx, constant: Constant, device_buffer, method: Optional[BinaryMethod] = None,
                   *, type_full_name: Optional[str] = None) -> None:
        """Writes the constant's Numbers, rounded to fp32, into `device_buffer`
        (a strict_amd DeviceBuffer holding at least `constant.count` floats)."""
        t, m = self._where(method, type_full_name)
        _check(self._lib, self._lib.sh_strictbinary_upload_f32(
            ctx.handle, self._handle, t, m, constant.index, device_buffer.ptr,
            device_buffer.nbytes // 4))

    def _where(self, method, type_full_name):
        if method is not None:
            return method.type_index, method.method_index
        if type_full_name is None:
            method = self.entry_point
            return method.type_index, method.method_index
        return self.methods_per_type[type_full_name].type_index, -1

    # -- writing --------------------------------------------------------------

    def to_bytes(self) -> bytes:
        n = ctypes.c_size_t()
        _check(self._lib, self._lib.sh_strictbinary_serialize(self._handle, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value)
        _check(self._lib, self._lib.sh_strictbinary_serialize(self._handle, buf, n.value,
                                                              ctypes.byref(n)))
        return buf.raw[:n.value]

    def serialize(self, file_path: str) -> None:
        """Serialize (cs:144-156)."""
        data = self.to_bytes()
        with open(file_path, "wb") as f:
            f.write(data)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            self._lib.sh_strictbinary_free(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def is_strictbinary(path: str) -> bool:
        return os.path.splitext(path)[1].lower() == EXTENSION
