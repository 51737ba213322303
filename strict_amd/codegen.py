"""Generated elementwise kernels: the host side of Strict.Compiler.Cuda's code
generation, over libstrict_hip's sh_instructions_to_hip.

Mirrors, with the same names, argument meaning and errors:
  - InstructionsToCuda (Strict.Compiler.Cuda/InstructionsToCuda.cs:12-110) as
    InstructionsToHip: Compile(Method) -> kernel source, Compile(binary) for an
    entry point with no parameters plus `count`, Extension;
  - CSharpToCudaTranspiler / CSharpType (CSharpToCudaTranspiler.cs:10-99) as
    CSharpToHipTranspiler / CSharpType: the line-pattern parse of a one-method
    C# file into a Strict type whose single method is then compiled.

The folding of bytecode registers into one C expression, the signature and
the bounds check run in C++ inside the library (strict_amd/csrc/codegen.cpp);
this module builds the flat instruction array it takes. `Method` carries the
small part of Strict this path needs: a method line `Name(a Number, ...)
Number`, a one-expression body, and the instruction list Strict's
BinaryGenerator emits for it (loads into consecutive registers R0..R15,
left operand first, result in the next register, then Return;
Strict.Bytecode/BinaryGenerator.cs:735-748, Registry.cs:18-24). Expressions
are names, numbers, + - * / % and parentheses, with * / % binding tighter.
"""
from __future__ import annotations

import ctypes
import enum
import os
import re
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

from . import _lib

__all__ = [
    "InstructionType", "Instruction", "Parameter", "Method", "InstructionsToHip",
    "CSharpToHipTranspiler", "CSharpType", "generate_instructions",
]


class InstructionType(enum.IntEnum):
    """Strict.Bytecode/InstructionType.cs:9-47 (the values the generator reads)."""
    LoadConstantToRegister = 0
    LoadVariableToRegister = 1
    Add = 11
    Subtract = 12
    Multiply = 13
    Divide = 14
    Modulo = 15
    Equal = 21
    NotEqual = 22
    LessThan = 23
    GreaterThan = 24
    Invoke = 31
    Return = 32
    LoopBegin = 33
    LoopEnd = 34


REGISTER_COUNT = 16  # Register.cs: R0 .. R15


@dataclass(frozen=True)
class Instruction:
    type: InstructionType
    registers: tuple
    identifier: Optional[str] = None
    number: float = 0.0

    def __str__(self):  # as Strict's Instruction.ToString
        regs = " ".join(f"R{r}" for r in self.registers)
        name = getattr(self.type, "name", str(self.type))  # a type outside the enum: its number
        if self.type == InstructionType.LoadVariableToRegister:
            return f"{name} {self.identifier} {regs}"
        if self.type == InstructionType.LoadConstantToRegister:
            return f"{name} {regs} {self.number:g}"
        return f"{name} {regs}"


def load_variable(register: int, identifier: str) -> Instruction:
    return Instruction(InstructionType.LoadVariableToRegister, (register,), identifier=identifier)


def load_constant(register: int, number: float) -> Instruction:
    return Instruction(InstructionType.LoadConstantToRegister, (register,), number=float(number))


def binary(kind: InstructionType, left: int, right: int, result: int) -> Instruction:
    return Instruction(kind, (left, right, result))


def return_register(register: int) -> Instruction:
    return Instruction(InstructionType.Return, (register,))


# ---- the expression subset of Strict a kernel body uses ----------------------

_TOKEN = re.compile(r"\s*(?:(\d+(?:\.\d+)?)|([A-Za-z_]\w*)|(.))")
_OPS = {"+": InstructionType.Add, "-": InstructionType.Subtract, "*": InstructionType.Multiply,
        "/": InstructionType.Divide, "%": InstructionType.Modulo}
_BINDING = {"+": 1, "-": 1, "*": 2, "/": 2, "%": 2}


class ParsingFailed(ValueError):
    pass


def _parse_expression(text: str):
    """Tree of ('name', s) / ('number', v) / (op, left, right)."""
    tokens = []
    pos = 0
    text = text.strip()
    while pos < len(text):
        m = _TOKEN.match(text, pos)
        if not m or m.end() == pos:
            break
        pos = m.end()
        number, name, other = m.groups()
        if number is not None:
            tokens.append(("number", float(number)))
        elif name is not None:
            tokens.append(("name", name))
        elif other.strip():
            tokens.append(("op", other))
    at = 0

    def peek():
        return tokens[at] if at < len(tokens) else (None, None)

    def primary():
        nonlocal at
        kind, value = peek()
        if kind in ("number", "name"):
            at += 1
            return (kind, value)
        if (kind, value) == ("op", "("):
            at += 1
            node = expression(1)
            if peek() != ("op", ")"):
                raise ParsingFailed(f"missing ')' in {text!r}")
            at += 1
            return node
        raise ParsingFailed(f"unexpected {value!r} in {text!r}")

    def expression(min_binding):
        nonlocal at
        left = primary()
        while True:
            kind, value = peek()
            if kind != "op" or value not in _BINDING or _BINDING[value] < min_binding:
                return left
            at += 1
            left = (value, left, expression(_BINDING[value] + 1))

    tree = expression(1)
    if at != len(tokens):
        raise ParsingFailed(f"trailing input in {text!r}")
    return tree


def _tree_text(node) -> str:
    """The body as Strict prints it back (Expression.ToString)."""
    if node[0] == "name":
        return node[1]
    if node[0] == "number":
        return f"{node[1]:g}"
    op, left, right = node
    lt, rt = _tree_text(left), _tree_text(right)
    if left[0] in _BINDING and _BINDING[left[0]] < _BINDING[op]:
        lt = f"({lt})"
    if right[0] in _BINDING and _BINDING[right[0]] <= _BINDING[op]:
        rt = f"({rt})"
    return f"{lt} {op} {rt}"


def generate_instructions(body: str) -> List[Instruction]:
    """Bytecode of a one-expression method body, in BinaryGenerator's order."""
    out: List[Instruction] = []
    next_register = 0

    def allocate():
        nonlocal next_register
        r = next_register % REGISTER_COUNT
        next_register += 1
        return r

    def emit(node) -> int:
        if node[0] == "name":
            r = allocate()
            out.append(load_variable(r, node[1]))
            return r
        if node[0] == "number":
            r = allocate()
            out.append(load_constant(r, node[1]))
            return r
        op, left, right = node
        lr = emit(left)
        rr = emit(right)
        res = allocate()
        out.append(binary(_OPS[op], lr, rr, res))
        return res

    out.append(return_register(emit(_parse_expression(body))))
    return out


@dataclass
class Parameter:
    name: str
    type: str = "Number"


@dataclass
class Method:
    """A Strict method: `name(parameters) return_type` with a one-line body."""
    name: str
    parameters: List[Parameter]
    body: str
    return_type: Optional[str] = "Number"
    _instructions: Optional[List[Instruction]] = field(default=None, repr=False)

    @classmethod
    def parse(cls, lines: Sequence[str]) -> "Method":
        """From Strict method lines: the header, then tab-indented body lines."""
        header = lines[0]
        m = re.fullmatch(r"(\w+)(?:\((.*)\))?(?:\s+(\w+))?", header.strip())
        if not m:
            raise ParsingFailed(f"not a method line: {header!r}")
        params = []
        if m.group(2):
            for p in m.group(2).split(","):
                parts = p.split()
                params.append(Parameter(parts[0], parts[1] if len(parts) > 1 else "Number"))
        body = " ".join(line.strip() for line in lines[1:] if line.strip())
        return cls(m.group(1), params, body, m.group(3))

    @property
    def instructions(self) -> List[Instruction]:
        if self._instructions is None:
            self._instructions = generate_instructions(self.body)
        return self._instructions

    def body_text(self) -> str:
        return _tree_text(_parse_expression(self.body))


def _flatten(instructions: Sequence[Instruction]):
    arr = (_lib.BcInstruction * max(1, len(instructions)))()
    keep = []
    for i, ins in enumerate(instructions):
        arr[i].type = int(ins.type)
        arr[i].register_count = len(ins.registers)
        for j, r in enumerate(ins.registers[:3]):
            arr[i].registers[j] = int(r)
        if ins.identifier is not None:
            b = ins.identifier.encode()
            keep.append(b)
            arr[i].identifier = b
        arr[i].number = float(ins.number)
    return arr, keep


def build_kernel(method_name: str, instructions: Sequence[Instruction],
                 parameters: Sequence[str], add_count_parameter: bool) -> str:
    """sh_instructions_to_hip: InstructionsToCuda.BuildCudaKernel (cs:25-74)."""
    lib = _lib.load()
    arr, keep = _flatten(instructions)
    names = [p.encode() for p in parameters]
    c_names = (ctypes.c_char_p * max(1, len(names)))(*names)
    length = ctypes.c_size_t(0)
    args = (method_name.encode(), c_names, len(names), 1 if add_count_parameter else 0,
            ctypes.cast(arr, ctypes.c_void_p), len(instructions))
    status = lib.sh_instructions_to_hip(*args, None, 0, ctypes.byref(length))
    if status not in (_lib.SH_OK, _lib.SH_ERR_INVALID_ARGUMENT) or length.value == 0:
        _raise(lib, status)
    buf = ctypes.create_string_buffer(length.value + 1)
    status = lib.sh_instructions_to_hip(*args, buf, len(buf), ctypes.byref(length))
    if status != _lib.SH_OK:
        _raise(lib, status)
    del keep
    return buf.value.decode()


def _raise(lib, status):
    from . import StrictHipError
    msg = (lib.sh_last_error() or b"").decode(errors="replace")
    if status == _lib.SH_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)  # the reference's NotSupportedException
    raise StrictHipError(status, msg)


class InstructionsToHip:
    """InstructionsToCuda (InstructionsToCuda.cs:12-110) for gfx950 HIP."""

    extension = ".hip"  # cs:17 ".cu"
    run_method = "Run"  # Method.Run, the entry point of a BinaryExecutable

    def compile(self, method: Method) -> str:
        """Compile(Method) (cs:19-23): kernel named after the method."""
        names = [p.name for p in method.parameters]
        return build_kernel(method.name, method.instructions, names,
                            self.needs_count_parameter(names))

    def compile_binary(self, binary) -> str:
        """Compile(BinaryExecutable, Platform) (cs:14-15): the entry point's
        instructions with no parameters plus `count`. `binary` is a loaded
        strictbinary.BinaryExecutable, or the entry point's instructions."""
        entry_point = binary.to_instructions() if hasattr(binary, "to_instructions") else binary
        return build_kernel(self.run_method, entry_point, [], True)

    @staticmethod
    def needs_count_parameter(parameter_names: Sequence[str]) -> bool:
        """cs:76-77: no count only when both width and height are parameters."""
        return "width" not in parameter_names or "height" not in parameter_names


# ---- CSharpToCudaTranspiler ---------------------------------------------------

class CSharpType:
    """CSharpType (CSharpToCudaTranspiler.cs:32-99): name + one method."""

    class MissingReturnStatement(Exception):
        pass

    def __init__(self, file_path: str):
        self.name, method_line, body_line = self._extract_method_info(file_path)
        self.methods = [Method.parse([method_line, "\t" + body_line])]

    @staticmethod
    def _ignored(line: str, type_name: str) -> bool:  # cs:77-84
        return (line == "" or "{" in line or "}" in line or line.startswith("using ")
                or line.startswith("namespace ") or type_name in line or "this." in line
                or line.startswith("\tprivate ") or line.startswith("\t\tfor "))

    @classmethod
    def _extract_method_info(cls, file_path: str):  # cs:46-75
        type_name = os.path.splitext(os.path.basename(file_path))[0]
        method_name = ""
        return_type = ""
        parameters: List[str] = []
        return_statement = ""
        with open(file_path, encoding="utf-8-sig") as f:
            lines = f.read().splitlines()
        for line in lines:
            if cls._ignored(line, type_name):
                continue
            if line.startswith("\t\treturn") or line.startswith("\t\t\t"):
                value = line.strip().replace(";", "")
                if value.startswith("return "):
                    value = value[7:]
                elif " = " in value:
                    value = value[value.rindex(" = ") + 3:]
                return_statement = value
            else:
                parts = [p for p in re.split(r"[ (),]", line.strip()) if p]
                if parts[1] == "float":
                    return_type = " Number"
                method_name = parts[2]
                cls._add_method_parameters(parts, parameters)
        if return_statement == "":
            raise cls.MissingReturnStatement(file_path)
        brackets = "(" + ", ".join(parameters) + ")" if parameters else ""
        return type_name, method_name + brackets + return_type, return_statement

    @staticmethod
    def _add_method_parameters(parts: List[str], parameters: List[str]) -> None:  # cs:86-98
        for index in range(3, len(parts), 2):
            if parts[index] == "DepthImage":
                parameters.extend(["input Number", "width Number", "height Number",
                                   "initialDepth Number"])
            elif parts[index] != "float":
                raise NotImplementedError(parts[index + 1] if index + 1 < len(parts)
                                          else parts[index])
            else:
                parameters.append(parts[index + 1] + " Number")


class CSharpToHipTranspiler:
    """CSharpToCudaTranspiler (CSharpToCudaTranspiler.cs:10-30)."""

    class InvalidCode(Exception):
        pass

    def convert(self, file_path: str) -> str:
        return self.generate_hip(self.parse_csharp(file_path))

    @staticmethod
    def generate_hip(type_: CSharpType) -> str:
        return InstructionsToHip().compile(type_.methods[0])

    def parse_csharp(self, file_path: str) -> CSharpType:
        if file_path == "":
            raise self.InvalidCode()
        return CSharpType(file_path)

    def dispose(self) -> None:
        pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.dispose()
