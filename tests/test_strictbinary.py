""".strictbinary loading (sh_strictbinary_*, strict_amd.strictbinary) against
the format restated in oracle/strictbinary.py, on the CPU.

The reference is C# and cannot run here; its own tests
(Strict.Bytecode.Tests/BinaryExecutableTests.cs, BinaryTypeTests.cs) are
mirrored case by case below. The oracle itself is pinned by .NET
BinaryWriter's published encodings (7-bit integers, length-prefixed UTF-8),
the facts the reference's tests assert about headers and name tables, a
byte-level known answer derived by hand from the format, and Python's own
zipfile reading what the product writes.
"""
import io
import struct
import zipfile

import numpy as np
import pytest

import oracle.strictbinary as osb
from strict_amd import codegen as cg
from strict_amd import strictbinary as sb

R0, R1, R2, R3 = 0, 1, 2, 3


def entry(full_name="Number", members=(), groups=None):
    return osb.TypeEntry(full_name, list(members), groups or {})


def run_type(instructions, full_name="Number"):
    return entry(full_name, groups={"Run": [osb.Method([], "None", list(instructions))]})


def load(*entries, compression=zipfile.ZIP_DEFLATED):
    return sb.BinaryExecutable(data=osb.write_strictbinary(list(entries), compression))


def zip_with(name, payload: bytes) -> bytes:
    buf = io.BytesIO()
    with zipfile.ZipFile(buf, "w") as z:
        z.writestr(name, payload)
    return buf.getvalue()


def header(names=()):
    # WriteHeader of BinaryExecutableTests.cs:134-141
    out = b"S" + bytes([1]) + osb.seven_bit(len(names))
    for n in names:
        out += osb.write_string(n)
    return out


# ---- pinning the oracle ------------------------------------------------------

@pytest.mark.parametrize("value,encoded", [
    (0, "00"), (1, "01"), (127, "7f"), (128, "8001"), (300, "ac02"), (16383, "ff7f"),
    (16384, "808001"), (2**31 - 1, "ffffffff07"), (-1, "ffffffff0f"), (-2**31, "8080808008"),
])
def test_seven_bit_encoding_known_answers(value, encoded):
    # .NET BinaryWriter.Write7BitEncodedInt: the uint32 pattern, 7 bits a byte, low first
    assert osb.seven_bit(value).hex() == encoded
    assert osb.Reader(bytes.fromhex(encoded)).seven() == value


def test_seven_bit_rejects_a_sixth_group():
    with pytest.raises(osb.FormatError, match="7-bit"):
        osb.Reader(bytes.fromhex("ffffffff1f")).seven()


def test_strings_are_utf8_with_a_byte_length():
    assert osb.write_string("Value = ") == b"\x08Value = "
    assert osb.write_string("ü") == b"\x02\xc3\xbc"
    assert osb.Reader(b"\x02\xc3\xbc").string() == "ü"


def test_builtin_name_table_layout():
    names = osb.BUILTIN_NAMES
    assert len(names) == 68 and len(set(names)) == 68
    assert names[:4] == ["", "None", "Boolean", "Number"]
    assert names[19] == "Strict/None" and names[36] == "Strict/Dictionary"
    assert names[37:40] == ["boolean", "number", "character"]
    assert "none" not in names and "errorWithValue" not in names
    assert names[53:57] == ["index", "value", "Run", "from"]
    assert names[-4:] == ["Strict/List(Number)", "List(Number)", "Strict/List(Text)", "List(Text)"]


def test_name_table_writes_only_custom_names():
    # NameTableWritesOnlyCustomNamesAndPrefillsBaseTypes (BinaryExecutableTests.cs:323-339)
    t = osb.NameTable("Number").add("CustomIdentifier")
    r = osb.Reader(t.write())
    assert r.seven() == 1 and r.string() == "CustomIdentifier"
    # NameTablePrefillsRequestedCommonNames (:365-387)
    t = osb.NameTable("Number")
    for n in ["index", "value", "first", "second", "from", "Run", "characters", "NewLine", "Tab",
              "textWriter"]:
        t.add(n)
    assert osb.Reader(t.write()).seven() == 0


def test_known_answer_bytes_of_a_small_type():
    # Hand-derived from the format: type "Add" (its just-name joins the table at
    # index 68), member `value Number` (built-in names 54 and 3), group "Run"
    # (55) with one overload: no parameters, returns None (1), instructions
    # LoadConstant R0 5 (type 0, register 0, SmallNumber kind 1, byte 5) and
    # Return R0 (type 32 = 0x20, register 0). No custom names.
    e = entry("Add", [osb.Member("value", "Number")],
              {"Run": [osb.Method([], "None", [osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number(5)),
                                               osb.Instr(osb.RETURN, (R0,))])]})
    expected = bytes.fromhex("53 01 00" "01 36 03 00" "01 37 01 00 01 02" "00 00 01 05" "20 00")
    assert osb.write_type(e) == expected
    back = osb.read_type(expected, "Add")
    assert back.members[0].name == "value" and back.groups["Run"][0].instructions[0].value.number == 5
    # the product reads the same bytes
    b = sb.BinaryExecutable(data=zip_with("Add.bytecode", expected))
    run = b.methods_per_type["Add"].method_groups["Run"][0]
    assert [(int(i.type), i.registers, i.number) for i in run.instructions] == [(0, (0,), 5.0), (32, (0,), 0.0)]


def test_number_kinds_follow_their_value():
    t = osb.NameTable("Number")
    assert osb.write_value(osb.number(255), t) == b"\x01\xff"
    assert osb.write_value(osb.number(256), t) == b"\x02" + struct.pack("<i", 256)
    assert osb.write_value(osb.number(-1), t) == b"\x02" + struct.pack("<i", -1)
    assert osb.write_value(osb.number(2.5), t) == b"\x03" + struct.pack("<d", 2.5)
    assert osb.write_value(osb.number(2.0**31), t) == b"\x03" + struct.pack("<d", 2.0**31)
    assert osb.write_value(osb.number(-0.0), t) == b"\x01\x00"  # IsSmallNumber(-0.0) holds


# ---- the reference's BinaryExecutableTests / BinaryTypeTests ------------------

def test_serialize_and_load_preserves_method_instructions():
    b = load(run_type([osb.Instr(osb.RETURN, (R0,))]))
    assert len(b.methods_per_type["Number"].method_groups["Run"][0].instructions) == 1


def test_serialize_and_load_preserves_member_metadata():
    b = load(entry("Number", [osb.Member("value", "Number")],
                   {"Run": [osb.Method([], "None", [osb.Instr(osb.RETURN, (R0,))])]}))
    assert b.methods_per_type["Number"].members[0].name == "value"


def test_find_instructions_returns_matching_overload():
    b = load(entry("Number", groups={"Compute": [
        osb.Method([], "None", [osb.Instr(osb.RETURN, (R0,))]),
        osb.Method([osb.Member("value", "Number")], "Number", [osb.Instr(osb.RETURN, (R1,))])]}))
    found = b.find_instructions("Number", "Compute", 1, "Number")
    assert int(found[0].type) == osb.RETURN and found[0].registers == (R1,)
    assert b.find_instructions("Number", "Compute", 1, "Strict/Number") is not None
    assert b.find_instructions("Number", "Compute", 0)[0].registers == (R0,)
    assert b.find_instructions("Number", "Compute", 2) is None
    assert b.find_instructions("Text", "Compute", 1) is None


def test_write_and_read_preserves_method_instructions():
    # BinaryTypeTests.WriteAndReadPreservesMethodInstructions (:9-32)
    e = entry("BinaryTypeTests", [osb.Member("value", "Number")], {"Compute": [osb.Method(
        [osb.Member("input", "Number")], "Number",
        [osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number(5)), osb.Instr(osb.RETURN, (R0,))])]})
    b = load(e)
    compute = b.methods_per_type["BinaryTypeTests"].method_groups["Compute"][0]
    assert len(compute.instructions) == 2
    assert sb.BinaryType.reconstruct_method_name("Compute", compute) == "Compute(input Number) Number"


@pytest.mark.parametrize("raw,name", [(105, "105"), (46, "FieldLoad"), (6, "6")])
def test_unknown_instruction_type_is_invalid_file(raw, name):
    payload = header() + bytes.fromhex("00" "01 37 01 00 01 01") + bytes([raw])
    with pytest.raises(sb.InvalidFile, match=f"Unknown instruction type: {name}$"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", payload))
    with pytest.raises(osb.FormatError, match="Unknown instruction type"):
        osb.read_type(payload, "Number")


def test_invalid_zip_is_invalid_file():
    with pytest.raises(sb.InvalidFile):
        sb.BinaryExecutable(data=bytes([0x42, 0x00, 0x10]))


def test_zip_without_bytecode_entries_is_empty():
    b = sb.BinaryExecutable(data=zip_with("dummy.txt", b""))
    assert b.methods_per_type == {}
    with pytest.raises(LookupError, match="No Run entry point"):
        b.entry_point


def test_bad_magic_bytes():
    with pytest.raises(sb.InvalidBytecodeEntry, match="magic byte"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", bytes([0xBA, 0x01])))
    with pytest.raises(sb.InvalidBytecodeEntry, match="magic byte"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", bytes([0x01, 1])))
    with pytest.raises(sb.InvalidBytecodeEntry, match="supported magic bytes"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", b"Stroct\x01"))


@pytest.mark.parametrize("version", [0, 2, 255])
def test_unsupported_version(version):
    with pytest.raises(sb.InvalidVersion, match=f"File version: {version}, this runtime only "
                                                "supports up to version 1"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", b"S" + bytes([version])))


def test_legacy_magic_loads():
    body = osb.write_type(run_type([osb.Instr(osb.RETURN, (R2,))]))
    legacy = b"Strict" + body[1:]  # "S" "trict" then the version byte
    b = sb.BinaryExecutable(data=zip_with("Number.bytecode", legacy))
    assert b.entry_point.instructions[0].registers == (R2,)


def test_unknown_value_kind():
    # UnknownValueKindThrows (BinaryExecutableTests.cs:114-132), byte for byte
    payload = header(["member", "Number"])
    payload += osb.seven_bit(1) + osb.seven_bit(0) + osb.seven_bit(1) + b"\x01"
    payload += bytes([osb.LOAD_CONSTANT, R0, 0xFF]) + osb.seven_bit(0) + osb.seven_bit(0)
    with pytest.raises(sb.InvalidFile, match="Unknown ValueKind: 255"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", payload))
    char_kind = payload.replace(bytes([osb.LOAD_CONSTANT, R0, 0xFF]), bytes([osb.LOAD_CONSTANT, R0, 7]))
    with pytest.raises(sb.InvalidFile, match="Unknown ValueKind: Character"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", char_kind))


def test_header_is_one_magic_byte_and_the_version():
    data = osb.write_strictbinary([run_type([osb.Instr(osb.RETURN, (R0,))], "Add")])
    b = sb.BinaryExecutable(data=data)
    out = zipfile.ZipFile(io.BytesIO(b.to_bytes()))
    body = out.read("Add.bytecode")
    assert body[:2] == b"S\x01"


def test_entry_name_table_holds_no_base_names_or_type_name():
    # EntryNameTableDoesNotStoreBaseFullNamesOrEntryTypeName (:341-363)
    e = entry("Add", [osb.Member("First", "Strict/Number"), osb.Member("Second", "Strict/Number")],
              {"Calculate": [osb.Method([], "Strict/Number", [
                  osb.Instr(osb.LOAD_VARIABLE, (R0,), name="First"),
                  osb.Instr(osb.LOAD_VARIABLE, (R1,), name="Second"),
                  osb.Instr(osb.ADD, (R0, R1, R2)), osb.Instr(osb.RETURN, (R2,))])]})
    body = zipfile.ZipFile(io.BytesIO(load(e).to_bytes())).read("Add.bytecode")
    r = osb.Reader(body[2:])
    custom = [r.string() for _ in range(r.seven())]
    assert custom == ["First", "Second", "Calculate"]


# ---- round trips ------------------------------------------------------------------

ALL_KINDS = [
    osb.Instr(osb.SET, (R0,), value=osb.number(42)),
    osb.Instr(osb.STORE_REGISTER, (R1,), name="result"),
    *[osb.Instr(op, (R0, R1)) for op in (osb.ADD, osb.SUBTRACT, osb.MULTIPLY, osb.DIVIDE,
                                         osb.MODULO, osb.EQUAL, osb.NOT_EQUAL, osb.LESS_THAN,
                                         osb.GREATER_THAN)],
    osb.Instr(osb.ADD, (R0, R1, R3)),
    osb.Instr(osb.JUMP, number=3), osb.Instr(osb.JUMP_IF_TRUE, number=2),
    osb.Instr(osb.JUMP_IF_FALSE, number=1), osb.Instr(osb.JUMP_IF_NOT_ZERO, (R0,), number=5),
    osb.Instr(osb.JUMP_END, number=10), osb.Instr(osb.JUMP_TO_ID_IF_FALSE, number=20),
    osb.Instr(osb.JUMP_TO_ID_IF_TRUE, number=30),
    osb.Instr(osb.WRITE_TO_LIST, (R0,), name="myList"),
    osb.Instr(osb.WRITE_TO_TABLE, (R0, R1), name="myTable"),
    osb.Instr(osb.REMOVE, (R2,), name="myList"),
    osb.Instr(osb.LIST_CALL, (R0, R1), name="myList"),
    osb.Instr(osb.PRINT, name="Value = ", print_register=R2),
    osb.Instr(osb.PRINT, name="Name: ", print_register=R1, flag=True),
    osb.Instr(osb.PRINT, name="done"),
    osb.Instr(osb.LOOP_BEGIN, (R0,), names=("element",)),
    osb.Instr(osb.LOOP_END, number=4),
    osb.Instr(osb.LOOP_BEGIN, (R1, 200), has_end=True),
    osb.Instr(osb.LOOP_END, number=1),
    osb.Instr(osb.INVOKE, (R3,), name="Calculate", invoke_type="Strict/Add", names=("first", "second"),
              invoke_return="Strict/Number", invoke_args=(R0, R1), invoke_instance=R2),
    osb.Instr(osb.INVOKE, (R0,), name="from", invoke_type="Strict/Color", invoke_return="Strict/Color"),
    osb.Instr(osb.STORE_CONSTANT, value=osb.text("héllo"), name="greeting", flag=True),
    osb.Instr(osb.STORE_CONSTANT, value=osb.none(), name="nothing"),
    osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.boolean(True)),
    osb.Instr(osb.LOAD_CONSTANT, (R1,), value=osb.dictionary(
        [(osb.number(1), osb.number(10)), (osb.number(2), osb.number(20))],
        "Strict/Dictionary(Number, Number)")),
    osb.Instr(osb.LOAD_CONSTANT, (R2,), value=osb.number_list([1.5, -3, 1e300, 70000])),
    osb.Instr(osb.RETURN, (R0,)),
]


def with_lines(instructions, lines):
    out = []
    for ins, line in zip(instructions, lines):
        c = osb.Instr(**{**ins.__dict__})
        c.source_line = line
        out.append(c)
    return out


def test_every_instruction_kind_round_trips_byte_for_byte():
    instructions = with_lines(ALL_KINDS, [0, 3, 3, 3, 7] + [7] * (len(ALL_KINDS) - 6) + [90])
    e = entry("Strict/ImageProcessing/Color", [osb.Member("Red", "Number",
                                                          osb.Instr(osb.SET, (R0,), value=osb.number(0.25)))],
              {"Run": [osb.Method([], "None", instructions)],
               "Mix": [osb.Method([osb.Member("other", "Strict/ImageProcessing/Color")], "Number",
                                  [osb.Instr(osb.RETURN, (R1,))])]})
    original = osb.write_type(e)
    b = load(e)
    out = zipfile.ZipFile(io.BytesIO(b.to_bytes()))
    assert out.namelist() == ["Strict/ImageProcessing/Color.bytecode"]
    assert out.read("Strict/ImageProcessing/Color.bytecode") == original
    # the oracle reads the product's output back to the same structure
    assert osb.read_type(out.read(out.namelist()[0]), e.full_name) == osb.read_type(original, e.full_name)
    # the product's flattened view agrees with the instructions
    run = b.methods_per_type[e.full_name].method_groups["Run"][0]
    assert [int(i.type) for i in run.instructions] == [i.type for i in instructions]
    for got, want in zip(run.instructions, instructions):
        regs = want.regs if want.print_register is None else (want.print_register,)
        assert got.registers == tuple(regs[:3]), want
        if want.type in (osb.LOAD_VARIABLE, osb.STORE_REGISTER, osb.WRITE_TO_LIST, osb.WRITE_TO_TABLE,
                         osb.REMOVE, osb.LIST_CALL, osb.PRINT, osb.INVOKE, osb.STORE_CONSTANT):
            assert got.identifier == want.name
        if want.type in (osb.JUMP, osb.JUMP_IF_TRUE, osb.JUMP_IF_FALSE, osb.JUMP_IF_NOT_ZERO,
                         osb.JUMP_END, osb.JUMP_TO_ID_IF_FALSE, osb.JUMP_TO_ID_IF_TRUE, osb.LOOP_END):
            assert got.number == want.number
    member = b.methods_per_type[e.full_name].members[0]
    assert (member.name, member.full_type_name, member.has_initial_value) == ("Red", "Number", True)
    mix = b.methods_per_type[e.full_name].method_groups["Mix"][0]
    assert [str(p) for p in mix.parameters] == ["other Color"]


def test_source_lines_are_stored_only_where_they_change():
    ins = with_lines([osb.Instr(osb.RETURN, (R0,))] * 4, [3, 3, 0, 5])
    body = osb.write_type(run_type(ins))
    flagged = [b for b in body if b & osb.INCLUDES_SOURCE_LINE]
    assert flagged == [osb.RETURN | 128, osb.RETURN | 128]
    # reading gives 3, 3, 3 (inherited), 5; writing that back stores the same two lines
    back = osb.read_type(body, "Number").groups["Run"][0].instructions
    assert [i.source_line for i in back] == [3, 3, 3, 5]
    b = sb.BinaryExecutable(data=zip_with("Number.bytecode", body))
    assert zipfile.ZipFile(io.BytesIO(b.to_bytes())).read("Number.bytecode") == body


def test_load_serialize_load_is_the_identity():
    types = [run_type(ALL_KINDS[:5], "Strict/Number"),
             entry("Strict/Text", [osb.Member("characters", "List(Character)")], {})]
    first = load(*types)
    data = first.to_bytes()
    second = sb.BinaryExecutable(data=data)
    assert second.to_bytes() == data
    assert list(second.methods_per_type) == ["Strict/Number", "Strict/Text"]
    # Python's zipfile reads the image (CRC-32 checked on read)
    z = zipfile.ZipFile(io.BytesIO(data))
    assert z.testzip() is None
    assert [i.compress_type for i in z.infolist()] == [zipfile.ZIP_DEFLATED] * 2


def test_stored_entries_and_windows_separators():
    data = osb.write_strictbinary([run_type([osb.Instr(osb.RETURN, (R1,))], "Strict/Number")],
                                  zipfile.ZIP_STORED)
    assert sb.BinaryExecutable(data=data).entry_point.instructions[0].registers == (R1,)
    body = osb.write_type(run_type([osb.Instr(osb.RETURN, (R3,))], "Strict/Number"))
    b = sb.BinaryExecutable(data=zip_with("Strict\\Number.BYTECODE", body))
    assert list(b.methods_per_type) == ["Strict/Number"]


def test_corrupt_entry_crc_is_invalid_file():
    data = bytearray(osb.write_strictbinary([run_type([osb.Instr(osb.RETURN, (R0,))])],
                                            zipfile.ZIP_STORED))
    at = data.index(b"Number.bytecode") + len(b"Number.bytecode")  # the local header's name
    assert data[at:at + 2] == b"S\x01"
    data[at + 3] ^= 0xFF  # a payload byte; the CRC in the headers no longer matches
    with pytest.raises(sb.InvalidFile, match="CRC-32"):
        sb.BinaryExecutable(data=bytes(data))


def test_truncated_entry_is_invalid_file():
    body = osb.write_type(run_type([osb.Instr(osb.RETURN, (R0,))]))
    with pytest.raises(sb.InvalidFile, match="end of the stream"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", body[:-1]))


def _nested_list(depth):
    v = osb.number_list([1.0])
    for _ in range(depth - 1):
        v = osb.Value(osb.V_LIST, text="Strict/List(Number)", items=[v])
    return v


def test_deeply_nested_values_are_invalid_file():
    # values nest one reader level per List; past 256 levels the file is
    # rejected (a deflated entry of a few KB could otherwise nest deep
    # enough to exhaust the stack)
    def binary(depth):
        return osb.write_strictbinary([run_type([
            osb.Instr(osb.LOAD_CONSTANT, (R0,), value=_nested_list(depth)),
            osb.Instr(osb.RETURN, (R0,))])])
    assert len(sb.BinaryExecutable(data=binary(200)).entry_point.instructions) == 2
    with pytest.raises(sb.InvalidFile, match="nested deeper than 256"):
        sb.BinaryExecutable(data=binary(300))


def test_declared_size_beyond_deflate_ratio_is_invalid_file():
    # a central directory entry that declares ~4 GiB for a few compressed
    # bytes is rejected before anything is allocated for it
    body = osb.write_type(run_type([osb.Instr(osb.RETURN, (R0,))]))
    buf = io.BytesIO()
    with zipfile.ZipFile(buf, "w", zipfile.ZIP_DEFLATED) as z:
        z.writestr("Number.bytecode", body)
    data = bytearray(buf.getvalue())
    cd = data.index(b"PK\x01\x02")
    assert struct.unpack_from("<H", data, cd + 10)[0] == 8  # deflated
    struct.pack_into("<I", data, cd + 24, 0xFFFFFFF0)
    with pytest.raises(sb.InvalidFile, match="declares 4294967280 bytes"):
        sb.BinaryExecutable(data=bytes(data))


def test_list_longer_than_its_entry_is_invalid_file():
    # a List declaring 2^31 - 1 items in an entry that ends after the count
    body = osb.write_type(run_type([
        osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number_list([7.0] * 3)),
        osb.Instr(osb.RETURN, (R0,))]))
    count = osb.seven_bit(3) + bytes([osb.V_SMALL, 7])
    at = body.index(count)
    cut = body[:at] + osb.seven_bit(2**31 - 1)
    with pytest.raises(sb.InvalidFile, match="end of the stream"):
        sb.BinaryExecutable(data=zip_with("Number.bytecode", cut))


def test_duplicate_type_entries_are_rejected():
    buf = io.BytesIO()
    body = osb.write_type(run_type([osb.Instr(osb.RETURN, (R0,))]))
    with zipfile.ZipFile(buf, "w") as z:
        z.writestr("Number.bytecode", body)
        z.writestr("Number.BYTECODE", body)
    with pytest.raises(sb.InvalidFile, match="same key"):
        sb.BinaryExecutable(data=buf.getvalue())


def test_entry_point_is_the_first_run_overload_in_archive_order():
    a = entry("A", groups={"Helper": [osb.Method([], "None", [osb.Instr(osb.RETURN, (R0,))])]})
    b = entry("B", groups={"Run": [osb.Method([], "None", [osb.Instr(osb.RETURN, (R1,))]),
                                   osb.Method([osb.Member("x", "Number")], "None",
                                              [osb.Instr(osb.RETURN, (R2,))])]})
    c = run_type([osb.Instr(osb.RETURN, (R3,))], "C")
    x = load(a, b, c)
    assert x.entry_point.instructions[0].registers == (R1,)
    assert [m.instructions[0].registers for m in x.get_run_methods()] == [(R1,), (R2,), (R3,)]
    assert x.to_instructions()[0].registers == (R1,)


def test_repeated_group_name_replaces_in_place():
    # MethodGroups[name] = overloads: the later group wins, the first keeps its slot
    t = osb.NameTable("T")
    body = b"S\x01" + osb.seven_bit(1) + osb.write_string("Helper") + osb.seven_bit(0)
    body += osb.seven_bit(3)
    for name, reg in [("Helper", R0), ("Run", R1), ("Helper", R2)]:
        body += osb.seven_bit(68 + 1 if name == "Helper" else t.index["Run"]) + osb.seven_bit(1)
        body += osb.seven_bit(0) + osb.seven_bit(t.index["None"]) + osb.seven_bit(1)
        body += bytes([osb.RETURN, reg])
    x = sb.BinaryExecutable(data=zip_with("T.bytecode", body))
    groups = x.methods_per_type["T"].method_groups
    assert list(groups) == ["Helper", "Run"]
    assert groups["Helper"][0].instructions[0].registers == (R2,)


# ---- constants as kernel inputs -------------------------------------------------

def constants_type():
    values = [1.5, 2, 300, -7, 1e10, 0.1, -0.0, 255, 256]
    run = [
        osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number_list(values)),
        osb.Instr(osb.STORE_CONSTANT, value=osb.number_list([4, 5, 6], "List(Number)"), name="first"),
        osb.Instr(osb.SET, (R1,), value=osb.number(42)),
        osb.Instr(osb.LOAD_CONSTANT, (R2,), value=osb.text("label")),
        osb.Instr(osb.LOAD_CONSTANT, (R3,), value=osb.number_list([])),
        osb.Instr(osb.LOAD_CONSTANT, (R3,), value=osb.Value(osb.V_LIST, text="List(Text)",
                                                          items=[osb.text("a")])),
        osb.Instr(osb.RETURN, (R0,)),
    ]
    members = [osb.Member("numbers", "List(Number)",
                          osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number_list([9, 8]))),
               osb.Member("plain", "Number")]
    return values, entry("Strict/Vectors", members, {"Run": [osb.Method([], "None", run)]})


def test_constants_of_the_entry_point():
    values, e = constants_type()
    b = load(e)
    cs = b.constants()
    assert [(c.instruction, c.instruction_type, c.kind, c.register, c.identifier, c.count) for c in cs] == [
        (0, osb.LOAD_CONSTANT, osb.V_LIST, R0, None, len(values)),
        (1, osb.STORE_CONSTANT, osb.V_LIST, -1, "first", 3),
        (2, osb.SET, osb.V_SMALL, R1, None, 1),
        (3, osb.LOAD_CONSTANT, osb.V_TEXT, R2, None, 0),
        (4, osb.LOAD_CONSTANT, osb.V_LIST, R3, None, 0),
        (5, osb.LOAD_CONSTANT, osb.V_LIST, R3, None, 0),
    ]
    got = b.constant_values(cs[0])
    assert got.dtype == np.float64 and np.array_equal(got, values)
    assert not np.signbit(got[6])  # -0.0 is stored as SmallNumber 0 (IsSmallNumber holds)
    assert b.constant_values(cs[2]).tolist() == [42.0]
    assert b.constant_values(cs[4]).size == 0
    with pytest.raises(Exception, match="Text, not a Number"):
        b.constant_values(cs[3])
    members = b.constants(type_full_name="Strict/Vectors")
    assert [(c.instruction, c.identifier, c.count) for c in members] == [(0, "numbers", 2)]
    assert b.constant_values(members[0], type_full_name="Strict/Vectors").tolist() == [9.0, 8.0]


def test_compile_binary_takes_a_loaded_binary():
    ins = [osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number(2.5)),
           osb.Instr(osb.LOAD_CONSTANT, (R1,), value=osb.number(4)),
           osb.Instr(osb.MULTIPLY, (R0, R1, R2)), osb.Instr(osb.RETURN, (R2,))]
    b = load(run_type(ins, "Strict/Scale"))
    gen = cg.InstructionsToHip()
    direct = gen.compile_binary([cg.load_constant(0, 2.5), cg.load_constant(1, 4),
                                 cg.binary(cg.InstructionType.Multiply, 0, 1, 2), cg.return_register(2)])
    assert gen.compile_binary(b) == direct
    assert "2.5f * 4.0f" in direct or "2.5" in direct


def test_a_loaded_method_compiles_with_its_parameters():
    add = osb.Method([osb.Member("first", "Number"), osb.Member("second", "Number")], "Number",
                     [osb.Instr(osb.LOAD_VARIABLE, (R0,), name="first"),
                      osb.Instr(osb.LOAD_VARIABLE, (R1,), name="second"),
                      osb.Instr(osb.ADD, (R0, R1, R2)), osb.Instr(osb.RETURN, (R2,))])
    b = load(entry("Strict/Vectors", groups={"Add": [add]}))
    method = b.find_method("Strict/Vectors", "Add", 2, "Number")
    src = cg.InstructionsToHip().compile(method.as_codegen_method())
    expected = cg.InstructionsToHip().compile(cg.Method.parse(["Add(first Number, second Number) Number",
                                                               "\tfirst + second"]))
    assert src == expected
