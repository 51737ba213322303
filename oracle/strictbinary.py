"""Pure-Python restatement of the .strictbinary format -- TEST INFRASTRUCTURE ONLY.

The checker for libstrict_hip's native loader (sh_strictbinary_*): tests build
.strictbinary files with `write_strictbinary`, read them with both this module
and the product, and compare. The product never imports it.

Restated from Strict.Bytecode (read as text):
  - .NET BinaryWriter / BinaryReader primitives (7-bit encoded ints, length-
    prefixed UTF-8 strings, little-endian int32 / double, one-byte booleans);
  - NameTable (Serialization/NameTable.cs:13-26 reader, :32-102 built-in names,
    :104-163 CollectStrings, :217-223 Write);
  - value instances (BinaryExecutable.cs:208-267 write, :278-292 read);
  - instructions (Instruction.cs WriteCompressed; Instructions/*.cs payloads;
    BinaryExecutable.cs:167-203 reader switch);
  - members, methods and types (BinaryMember.cs:9-28, BinaryMethod.cs:49-89,
    BinaryType.cs:11-28, :43-62, :88-137);
  - the ZIP container (BinaryExecutable.cs:40-61, :144-156), through Python's
    zipfile (deflate, as CompressionLevel.Optimal).
"""
from __future__ import annotations

import io
import math
import struct
import zipfile
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

# InstructionType (InstructionType.cs:9-47)
LOAD_CONSTANT, LOAD_VARIABLE, STORE_CONSTANT, STORE_REGISTER, SET, LIST_CALL = 0, 1, 2, 3, 4, 5
ADD, SUBTRACT, MULTIPLY, DIVIDE, MODULO = 11, 12, 13, 14, 15
EQUAL, NOT_EQUAL, LESS_THAN, GREATER_THAN = 21, 22, 23, 24
INVOKE, RETURN, LOOP_BEGIN, LOOP_END, JUMP, JUMP_IF_TRUE, JUMP_IF_FALSE = 31, 32, 33, 34, 35, 36, 37
JUMP_IF_NOT_ZERO, JUMP_END, JUMP_TO_ID_IF_FALSE, JUMP_TO_ID_IF_TRUE = 38, 39, 40, 41
WRITE_TO_LIST, WRITE_TO_TABLE, REMOVE, PRINT = 42, 43, 44, 45
INCLUDES_SOURCE_LINE = 128

# ValueKind (Serialization/ValueKind.cs)
V_NONE, V_SMALL, V_INTEGER, V_NUMBER, V_TEXT, V_BOOLEAN, V_LIST, V_DICTIONARY = 0, 1, 2, 3, 4, 5, 6, 9

_TYPES = ["None", "Boolean", "Number", "Character", "Range", "Text", "Error", "ErrorWithValue",
          "Iterator", "List", "Logger", "File", "Directory", "TextWriter", "TextReader",
          "Stacktrace", "Mutable", "Dictionary"]
# NameTable.BuiltInPredefinedNames (NameTable.cs:32-102), in order
BUILTIN_NAMES = ([""] + _TYPES + ["Strict/" + t for t in _TYPES]
                 + [t[0].lower() + t[1:] for t in _TYPES if t not in ("None", "ErrorWithValue")]
                 + ["index", "value", "Run", "from", "first", "second", "numbers", "characters",
                    "texts", "NewLine", "Tab", "Strict/List(Number)", "List(Number)",
                    "Strict/List(Text)", "List(Text)"])


class FormatError(Exception):
    def __init__(self, kind: str, message: str):
        super().__init__(f"{kind}: {message}")
        self.kind = kind


# ---- .NET BinaryWriter / BinaryReader -----------------------------------------

def seven_bit(value: int) -> bytes:
    """Write7BitEncodedInt: 7 bits per byte, low first, of the uint32 pattern."""
    v = value & 0xFFFFFFFF
    out = bytearray()
    while v > 0x7F:
        out.append((v & 0x7F) | 0x80)
        v >>= 7
    out.append(v)
    return bytes(out)


class Reader:
    def __init__(self, data: bytes):
        self.data, self.pos = data, 0

    def byte(self) -> int:
        if self.pos >= len(self.data):
            raise FormatError("InvalidFile", "Unable to read beyond the end of the stream.")
        self.pos += 1
        return self.data[self.pos - 1]

    def boolean(self) -> bool:
        return self.byte() != 0

    def i32(self) -> int:
        return struct.unpack("<i", bytes(self.byte() for _ in range(4)))[0]

    def f64(self) -> float:
        return struct.unpack("<d", bytes(self.byte() for _ in range(8)))[0]

    def seven(self) -> int:
        result = 0
        for shift in range(0, 28, 7):
            b = self.byte()
            result |= (b & 0x7F) << shift
            if b <= 0x7F:
                return result - (1 << 32) if result >= 1 << 31 else result
        b = self.byte()
        if b > 0x0F:
            raise FormatError("InvalidFile", "Too many bytes in what should have been a 7-bit "
                                             "encoded integer.")
        result |= b << 28
        return result - (1 << 32) if result >= 1 << 31 else result

    def string(self) -> str:
        n = self.seven()
        raw = bytes(self.byte() for _ in range(n))
        return raw.decode("utf-8")


def write_string(s: str) -> bytes:
    raw = s.encode("utf-8")
    return seven_bit(len(raw)) + raw


# ---- object model ----------------------------------------------------------------

@dataclass
class Value:
    kind: int
    number: float = 0.0
    text: str = ""
    items: List["Value"] = field(default_factory=list)


def number(v: float) -> Value:
    """A Number ValueInstance (the writer picks its stored kind)."""
    return Value(V_NUMBER, float(v))


def text(s: str) -> Value:
    return Value(V_TEXT, text=s)


def boolean(b: bool) -> Value:
    return Value(V_BOOLEAN, 1.0 if b else 0.0)


def none() -> Value:
    return Value(V_NONE)


def number_list(values, type_name: str = "Strict/List(Number)") -> Value:
    return Value(V_LIST, text=type_name, items=[number(v) for v in values])


def dictionary(pairs, type_name: str) -> Value:
    items = []
    for k, v in pairs:
        items += [k, v]
    return Value(V_DICTIONARY, text=type_name, items=items)


@dataclass
class Instr:
    type: int
    regs: Tuple[int, ...] = ()
    name: Optional[str] = None          # identifier / print prefix / invoke method
    value: Optional[Value] = None       # LoadConstant / StoreConstant / Set
    flag: bool = False                  # StoreConstant.IsMember / Print.ValueIsText
    number: int = 0                     # jumps, LoopEnd steps
    has_end: bool = False               # LoopBegin with an end register
    names: Tuple[str, ...] = ()         # LoopBegin custom names / Invoke parameter names
    invoke_type: Optional[str] = None
    invoke_return: Optional[str] = None
    invoke_args: Tuple[int, ...] = ()
    invoke_instance: Optional[int] = None
    print_register: Optional[int] = None
    source_line: int = 0


@dataclass
class Member:
    name: str
    type: str
    initial: Optional[Instr] = None


@dataclass
class Method:
    parameters: List[Member]
    return_type: str
    instructions: List[Instr]


@dataclass
class TypeEntry:
    full_name: str
    members: List[Member]
    groups: Dict[str, List[Method]]


def just_type_name(full: str) -> str:
    return full.split("/")[-1]


# ---- name table ----------------------------------------------------------------------

class NameTable:
    def __init__(self, just: str):
        self.names: List[str] = []
        self.index: Dict[str, int] = {}
        for n in BUILTIN_NAMES:
            self.add(n)
        self.add(just)
        self.prefilled = len(self.names)

    def add(self, n: str) -> "NameTable":
        if n not in self.index:
            self.index[n] = len(self.names)
            self.names.append(n)
        return self

    def at(self, i: int) -> str:
        if not 0 <= i < len(self.names):
            raise FormatError("InvalidFile", f"name index {i} outside the table")
        return self.names[i]

    def collect_value(self, v: Value):
        """CollectValueInstanceStrings (NameTable.cs:137-163)."""
        if v.kind == V_TEXT:
            return self.add(v.text)
        if v.kind in (V_LIST, V_DICTIONARY):
            self.add(v.text)
            for i in v.items:
                self.collect_value(i)
            return self
        if v.kind in (V_SMALL, V_INTEGER, V_NUMBER) and not _is_integer(v.number):
            self.add("Strict/Number")
        return self

    def collect(self, ins: Instr):
        """CollectStrings (NameTable.cs:104-122)."""
        t = ins.type
        if t in (LOAD_VARIABLE, STORE_REGISTER, WRITE_TO_LIST, WRITE_TO_TABLE, REMOVE, LIST_CALL,
                 PRINT):
            self.add(ins.name)
        elif t == STORE_CONSTANT:
            self.add(ins.name).collect_value(ins.value)
        elif t in (SET, LOAD_CONSTANT):
            self.collect_value(ins.value)
        elif t == INVOKE:
            self.add(ins.invoke_type).add(ins.name).add(ins.invoke_return)
            for n in ins.names:
                self.add(n)
        elif t == LOOP_BEGIN:
            for n in ins.names:
                self.add(n)
        return self

    def member(self, m: Member):
        self.add(m.name).add(m.type)
        if m.initial is not None:
            self.collect(m.initial)

    def write(self) -> bytes:
        custom = self.names[self.prefilled:]
        return seven_bit(len(custom)) + b"".join(write_string(n) for n in custom)


def _is_small(v: float) -> bool:
    return 0 <= v <= 255 and v == math.floor(v)


def _is_integer(v: float) -> bool:
    return -2147483648.0 <= v <= 2147483647.0 and v == math.floor(v)


# ---- writer ----------------------------------------------------------------------------

def write_value(v: Value, t: NameTable) -> bytes:
    """WriteValueInstance (BinaryExecutable.cs:208-267)."""
    if v.kind == V_TEXT:
        return bytes([V_TEXT]) + seven_bit(t.index[v.text])
    if v.kind == V_LIST:
        return (bytes([V_LIST]) + seven_bit(t.index[v.text]) + seven_bit(len(v.items))
                + b"".join(write_value(i, t) for i in v.items))
    if v.kind == V_DICTIONARY:
        return (bytes([V_DICTIONARY]) + seven_bit(t.index[v.text]) + seven_bit(len(v.items) // 2)
                + b"".join(write_value(i, t) for i in v.items))
    if v.kind == V_BOOLEAN:
        return bytes([V_BOOLEAN, 1 if v.number else 0])
    if v.kind == V_NONE:
        return bytes([V_NONE])
    if _is_small(v.number):
        return bytes([V_SMALL, int(v.number)])
    if _is_integer(v.number):
        return bytes([V_INTEGER]) + struct.pack("<i", int(v.number))
    return bytes([V_NUMBER]) + struct.pack("<d", v.number)


def write_instruction(ins: Instr, t: NameTable, prev: List[int]) -> bytes:
    """Instruction.WriteCompressed + the type's WritePayload."""
    out = bytearray()
    if ins.source_line != 0 and ins.source_line != prev[0]:
        out.append(ins.type | INCLUDES_SOURCE_LINE)
        out += seven_bit(ins.source_line)
        prev[0] = ins.source_line
    else:
        out.append(ins.type)
    ty = ins.type
    if ty == LOAD_CONSTANT:
        out.append(ins.regs[0])
        out += write_value(ins.value, t)
    elif ty in (LOAD_VARIABLE, STORE_REGISTER, WRITE_TO_LIST, REMOVE):
        out.append(ins.regs[0])
        out += seven_bit(t.index[ins.name])
    elif ty == STORE_CONSTANT:
        out += write_value(ins.value, t) + seven_bit(t.index[ins.name]) + bytes([ins.flag])
    elif ty == SET:
        out += write_value(ins.value, t)
        out.append(ins.regs[0])
    elif ty == INVOKE:
        out.append(ins.regs[0])
        out += seven_bit(t.index[ins.invoke_type]) + seven_bit(t.index[ins.name])
        out += seven_bit(len(ins.names)) + b"".join(seven_bit(t.index[n]) for n in ins.names)
        out += seven_bit(t.index[ins.invoke_return])
        out += seven_bit(len(ins.invoke_args)) + bytes(ins.invoke_args)
        out.append(ins.invoke_instance is not None)
        if ins.invoke_instance is not None:
            out.append(ins.invoke_instance)
    elif ty == RETURN:
        out.append(ins.regs[0])
    elif ty == LOOP_BEGIN:
        out.append(ins.regs[0])
        out.append(ins.has_end)
        if ins.has_end:
            out += seven_bit(ins.regs[1])
        out += seven_bit(len(ins.names)) + b"".join(seven_bit(t.index[n]) for n in ins.names)
    elif ty in (LOOP_END, JUMP, JUMP_IF_TRUE, JUMP_IF_FALSE, JUMP_END, JUMP_TO_ID_IF_FALSE,
                JUMP_TO_ID_IF_TRUE):
        out += seven_bit(ins.number)
    elif ty == JUMP_IF_NOT_ZERO:
        out += seven_bit(ins.number)
        out.append(ins.regs[0])
    elif ty in (WRITE_TO_TABLE, LIST_CALL):
        out += bytes([ins.regs[0], ins.regs[1]]) + seven_bit(t.index[ins.name])
    elif ty == PRINT:
        out += seven_bit(t.index[ins.name])
        out.append(ins.print_register is not None)
        if ins.print_register is not None:
            out += bytes([ins.print_register, ins.flag])
    else:  # binary operators: register count, registers
        out.append(len(ins.regs))
        out += bytes(ins.regs)
    return bytes(out)


def _write_members(members: List[Member], t: NameTable) -> bytes:
    out = bytearray(seven_bit(len(members)))
    for m in members:
        out += seven_bit(t.index[m.name]) + seven_bit(t.index[m.type])
        out.append(m.initial is not None)
        if m.initial is not None:
            out += write_instruction(m.initial, t, [0])
    return bytes(out)


def write_type(entry: TypeEntry) -> bytes:
    """BinaryType.Write (BinaryType.cs:108-122) with CreateNameTable (:88-106)."""
    t = NameTable(just_type_name(entry.full_name))
    for m in entry.members:
        t.member(m)
    for name, methods in entry.groups.items():
        t.add(name)
        for method in methods:
            t.add(method.return_type)
            for p in method.parameters:
                t.member(p)
            for ins in method.instructions:
                t.collect(ins)
    out = bytearray(b"S" + bytes([1]))
    out += t.write()
    out += _write_members(entry.members, t)
    out += seven_bit(len(entry.groups))
    for name, methods in entry.groups.items():
        out += seven_bit(t.index[name]) + seven_bit(len(methods))
        for method in methods:
            out += _write_members(method.parameters, t)
            out += seven_bit(t.index[method.return_type])
            out += seven_bit(len(method.instructions))
            prev = [0]
            for ins in method.instructions:
                out += write_instruction(ins, t, prev)
    return bytes(out)


def write_strictbinary(entries: List[TypeEntry], compression=zipfile.ZIP_DEFLATED) -> bytes:
    """Serialize (BinaryExecutable.cs:144-156): one "<type>.bytecode" entry per type."""
    buf = io.BytesIO()
    with zipfile.ZipFile(buf, "w", compression) as z:
        for e in entries:
            z.writestr(e.full_name + ".bytecode", write_type(e))
    return buf.getvalue()


# ---- reader -------------------------------------------------------------------------------

def read_value(r: Reader, t: NameTable) -> Value:
    """ReadValueInstance (BinaryExecutable.cs:278-292)."""
    kind = r.byte()
    if kind == V_TEXT:
        return Value(V_TEXT, text=t.at(r.seven()))
    if kind == V_NONE:
        return Value(V_NONE)
    if kind == V_BOOLEAN:
        return Value(V_BOOLEAN, 1.0 if r.boolean() else 0.0)
    if kind == V_SMALL:
        return Value(V_SMALL, float(r.byte()))
    if kind == V_INTEGER:
        return Value(V_INTEGER, float(r.i32()))
    if kind == V_NUMBER:
        return Value(V_NUMBER, r.f64())
    if kind == V_LIST:
        name = t.at(r.seven())
        return Value(V_LIST, text=name, items=[read_value(r, t) for _ in range(r.seven())])
    if kind == V_DICTIONARY:
        name = t.at(r.seven())
        items = []
        for _ in range(r.seven()):
            items += [read_value(r, t), read_value(r, t)]
        return Value(V_DICTIONARY, text=name, items=items)
    names = ["None", "SmallNumber", "IntegerNumber", "Number", "Text", "Boolean", "List",
             "Character", "Name", "Dictionary"]
    raise FormatError("InvalidFile", "Unknown ValueKind: " + (names[kind] if kind < 10 else str(kind)))


def read_instruction(r: Reader, t: NameTable, prev: List[int]) -> Instr:
    """ReadInstruction (BinaryExecutable.cs:167-203)."""
    raw = r.byte()
    ty = raw & (INCLUDES_SOURCE_LINE - 1)
    if raw & INCLUDES_SOURCE_LINE:
        prev[0] = r.seven()
    ins = Instr(ty)
    if ty == LOAD_CONSTANT:
        ins.regs = (r.byte(),)
        ins.value = read_value(r, t)
    elif ty in (LOAD_VARIABLE, STORE_REGISTER, WRITE_TO_LIST, REMOVE):
        ins.regs = (r.byte(),)
        ins.name = t.at(r.seven())
    elif ty == STORE_CONSTANT:
        ins.value = read_value(r, t)
        ins.name = t.at(r.seven())
        ins.flag = r.boolean()
    elif ty == SET:
        ins.value = read_value(r, t)
        ins.regs = (r.byte(),)
    elif ty == INVOKE:
        ins.regs = (r.byte(),)
        ins.invoke_type = t.at(r.seven())
        ins.name = t.at(r.seven())
        ins.names = tuple(t.at(r.seven()) for _ in range(r.seven()))
        ins.invoke_return = t.at(r.seven())
        ins.invoke_args = tuple(r.byte() for _ in range(r.seven()))
        ins.invoke_instance = r.byte() if r.boolean() else None
    elif ty == RETURN:
        ins.regs = (r.byte(),)
    elif ty == LOOP_BEGIN:
        regs = [r.byte()]
        if r.boolean():
            ins.has_end = True
            regs.append(r.seven())
        ins.regs = tuple(regs)
        ins.names = tuple(t.at(r.seven()) for _ in range(r.seven()))
    elif ty in (LOOP_END, JUMP, JUMP_IF_TRUE, JUMP_IF_FALSE, JUMP_END, JUMP_TO_ID_IF_FALSE,
                JUMP_TO_ID_IF_TRUE):
        ins.number = r.seven()
    elif ty == JUMP_IF_NOT_ZERO:
        ins.number = r.seven()
        ins.regs = (r.byte(),)
    elif ty in (WRITE_TO_TABLE, LIST_CALL):
        ins.regs = (r.byte(), r.byte())
        ins.name = t.at(r.seven())
    elif ty == PRINT:
        ins.name = t.at(r.seven())
        if r.boolean():
            ins.print_register = r.byte()
            ins.flag = r.boolean()
    elif 10 < ty < 30:
        ins.regs = tuple(r.byte() for _ in range(r.byte()))
    else:
        raise FormatError("InvalidFile", f"Unknown instruction type: {ty}")
    ins.source_line = prev[0]
    return ins


def _read_members(r: Reader, t: NameTable) -> List[Member]:
    out = []
    for _ in range(r.seven()):
        name, ty = t.at(r.seven()), t.at(r.seven())
        out.append(Member(name, ty, read_instruction(r, t, [0]) if r.boolean() else None))
    return out


def read_type(data: bytes, full_name: str) -> TypeEntry:
    """BinaryType(BinaryReader, ...) (BinaryType.cs:11-28, :43-62)."""
    r = Reader(data)
    if r.byte() != ord("S"):
        raise FormatError("InvalidBytecodeEntry", "Entry does not start with compact 'S' magic byte")
    version = second = r.byte()
    if second == ord("t"):
        if bytes(r.byte() for _ in range(4)) != b"rict":
            raise FormatError("InvalidBytecodeEntry", "Entry does not start with supported magic bytes")
        version = r.byte()
    if version == 0 or version > 1:
        raise FormatError("InvalidVersion",
                          f"File version: {version}, this runtime only supports up to version 1")
    t = NameTable(just_type_name(full_name))
    for _ in range(r.seven()):
        t.add(r.string())
    members = _read_members(r, t)
    groups: Dict[str, List[Method]] = {}
    for _ in range(r.seven()):
        name = t.at(r.seven())
        methods = []
        for _ in range(r.seven()):
            params = _read_members(r, t)
            ret = t.at(r.seven())
            prev = [0]
            methods.append(Method(params, ret, [read_instruction(r, t, prev) for _ in range(r.seven())]))
        groups[name] = methods
    return TypeEntry(full_name, members, groups)


def read_strictbinary(data: bytes) -> List[TypeEntry]:
    """BinaryExecutable(filePath) (BinaryExecutable.cs:40-61), entries in archive order."""
    try:
        z = zipfile.ZipFile(io.BytesIO(data))
    except zipfile.BadZipFile as e:
        raise FormatError("InvalidFile", str(e)) from None
    out = []
    for info in z.infolist():
        if info.filename.lower().endswith(".bytecode"):
            name = info.filename.replace("\\", "/")
            dot = name.rfind(".")
            out.append(read_type(z.read(info), name[:dot] if dot > 0 else name))
    return out
