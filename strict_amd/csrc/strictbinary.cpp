// .strictbinary loading: the native counterpart of BinaryExecutable's ZIP
// loader (Strict.Bytecode/BinaryExecutable.cs:40-61) and of the BinaryType /
// BinaryMethod / instruction readers it drives, plus Serialize
// (BinaryExecutable.cs:144-156) for round trips. Host code only: a loaded
// binary hands its method instructions to sh_instructions_to_hip and its
// Number / List(Number) constants to device buffers as kernel inputs.
//
// Format (BinaryType.cs:11-28, :108-122): a ZIP archive whose entries
// "<type full name>.bytecode" each hold one type:
//   'S' version(1)            (legacy: "Strict" then the version)
//   name table                custom names after the built-in ones
//   members                   name, type, optional initial-value instruction
//   method groups             name, overloads: parameters, return type,
//                             instructions
// Integers in the stream are .NET BinaryWriter's: 7-bit encoded (LEB128 of
// the uint32 bit pattern, at most 5 bytes), little-endian int32 / double,
// booleans as one byte, strings as a 7-bit byte length and UTF-8 bytes.
#include <zlib.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.h"

struct sh_strictbinary;

namespace sh {
namespace {

// InstructionType values (Strict.Bytecode/InstructionType.cs:9-47)
enum : int {
  kLoadConstant = 0, kLoadVariable = 1, kStoreConstant = 2, kStoreRegister = 3, kSet = 4,
  kListCall = 5, kStoreSeparator = 10, kBinaryOperatorsSeparator = 30, kInvoke = 31,
  kReturn = 32, kLoopBegin = 33, kLoopEnd = 34, kJump = 35, kJumpIfTrue = 36,
  kJumpIfFalse = 37, kJumpIfNotZero = 38, kJumpEnd = 39, kJumpToIdIfFalse = 40,
  kJumpToIdIfTrue = 41, kWriteToList = 42, kWriteToTable = 43, kRemove = 44, kPrint = 45,
  kIncludesSourceLine = 128
};

// Names of the defined InstructionType values, for "Unknown instruction type"
// messages (an undefined value prints as its number, as a C# enum does).
const char *instruction_type_name(int t) {
  static const std::map<int, const char *> names = {
      {0, "LoadConstantToRegister"}, {1, "LoadVariableToRegister"}, {2, "StoreConstantToVariable"},
      {3, "StoreRegisterToVariable"}, {4, "Set"}, {5, "ListCall"}, {10, "StoreSeparator"},
      {11, "Add"}, {12, "Subtract"}, {13, "Multiply"}, {14, "Divide"}, {15, "Modulo"},
      {20, "ArithmeticSeparator"}, {21, "Equal"}, {22, "NotEqual"}, {23, "LessThan"},
      {24, "GreaterThan"}, {30, "BinaryOperatorsSeparator"}, {31, "Invoke"}, {32, "Return"},
      {33, "LoopBegin"}, {34, "LoopEnd"}, {35, "Jump"}, {36, "JumpIfTrue"}, {37, "JumpIfFalse"},
      {38, "JumpIfNotZero"}, {39, "JumpEnd"}, {40, "JumpToIdIfFalse"}, {41, "JumpToIdIfTrue"},
      {42, "InvokeWriteToList"}, {43, "InvokeWriteToTable"}, {44, "InvokeRemove"},
      {45, "Print"}, {46, "FieldLoad"}, {47, "ConstructValueType"}};
  auto it = names.find(t);
  return it == names.end() ? nullptr : it->second;
}

// ValueKind values (Strict.Bytecode/Serialization/ValueKind.cs)
enum : int {
  kValueNone = 0, kValueSmallNumber = 1, kValueIntegerNumber = 2, kValueNumber = 3,
  kValueText = 4, kValueBoolean = 5, kValueList = 6, kValueCharacter = 7, kValueName = 8,
  kValueDictionary = 9
};

const char *value_kind_name(int k) {
  static const char *names[] = {"None", "SmallNumber", "IntegerNumber", "Number", "Text",
                                "Boolean", "List", "Character", "Name", "Dictionary"};
  return k >= 0 && k < 10 ? names[k] : nullptr;
}

// The exceptions the reference's loader throws, as error kinds.
enum ErrorKind { kInvalidFile, kInvalidBytecodeEntry, kInvalidVersion };

struct FormatError {
  ErrorKind kind;
  std::string message;
};

[[noreturn]] void throw_format(ErrorKind kind, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
void throw_format(ErrorKind kind, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw FormatError{kind, buf};
}

// ---- object model --------------------------------------------------------

struct Value {
  int kind = kValueNone;      // as stored
  double number = 0.0;        // SmallNumber / IntegerNumber / Number; Boolean as 0 / 1
  std::string text;           // Text; List / Dictionary: the collection's type name
  std::vector<Value> items;   // List items; Dictionary: key, value, key, value, ...
};

// One instruction; which fields a type uses follows its reader
// (Strict.Bytecode/Instructions/*.cs).
struct Instr {
  int type = 0;
  int source_line = 0;
  std::vector<int> regs;          // register operands in payload order
  std::string name;               // identifier / Print text prefix / Invoke method name
  bool flag = false;              // StoreConstantToVariable.IsMember, Print.ValueIsText
  bool has_value = false;         // LoadConstant / StoreConstant / Set
  Value value;
  int number = 0;                 // Jump skip, JumpToId id, LoopEnd steps
  bool has_end = false;           // LoopBegin with an end register (regs[1])
  bool has_print_register = false;
  std::vector<std::string> names; // LoopBegin custom names / Invoke parameter names
  std::string invoke_type, invoke_return;
  std::vector<int> invoke_args;
  int invoke_instance = -1;       // -1: no instance register
};

struct Member {
  std::string name, type;
  bool has_initial = false;
  Instr initial;
};

struct MethodData {
  std::string name;
  std::vector<Member> parameters;
  std::string return_type;
  std::vector<Instr> instructions;
  std::vector<sh_bc_instruction> flat;  // sh_strictbinary_instructions' view
};

struct TypeData {
  std::string full_name;
  std::vector<std::string> names;       // the name table, built-in names first
  std::vector<Member> members;
  std::vector<MethodData> methods;      // overloads of every group, groups in file order
  std::vector<std::string> group_order; // group names in file order
};

// ---- the name table (NameTable.cs:13-26, :32-102) ----------------------------

const std::vector<std::string> &builtin_names() {
  static const std::vector<std::string> names = [] {
    const char *types[] = {"None", "Boolean", "Number", "Character", "Range", "Text",
                           "Error", "ErrorWithValue", "Iterator", "List", "Logger", "File",
                           "Directory", "TextWriter", "TextReader", "Stacktrace", "Mutable",
                           "Dictionary"};
    std::vector<std::string> v = {""};
    for (const char *t : types) v.push_back(t);
    for (const char *t : types) v.push_back(std::string("Strict/") + t);
    for (const char *t : types) {  // first letter lowercased, but for None and ErrorWithValue
      if (std::strcmp(t, "None") == 0 || std::strcmp(t, "ErrorWithValue") == 0) continue;
      std::string s = t;
      s[0] = (char)(s[0] - 'A' + 'a');
      v.push_back(s);
    }
    for (const char *s : {"index", "value", "Run", "from", "first", "second", "numbers",
                          "characters", "texts", "NewLine", "Tab", "Strict/List(Number)",
                          "List(Number)", "Strict/List(Text)", "List(Text)"})
      v.push_back(s);
    return v;
  }();
  return names;
}

struct NameTable {
  std::vector<std::string> names;
  std::map<std::string, int> index;
  size_t prefilled = 0;

  explicit NameTable(const std::string &just_type_name) {
    for (const std::string &n : builtin_names()) add(n);
    add(just_type_name);
    prefilled = names.size();
  }
  void add(const std::string &n) {
    if (index.count(n)) return;
    index[n] = (int)names.size();
    names.push_back(n);
  }
  const std::string &at(int i) const {
    if (i < 0 || (size_t)i >= names.size())
      throw_format(kInvalidFile, "Name index %d outside the name table (%zu names)", i,
                   names.size());
    return names[(size_t)i];
  }
  int operator[](const std::string &n) const { return index.at(n); }
};

std::string just_type_name(const std::string &full) {
  const size_t p = full.rfind('/');
  return p == std::string::npos ? full : full.substr(p + 1);
}

// ---- .NET BinaryReader --------------------------------------------------------

struct Reader {
  const uint8_t *p, *end;

  uint8_t byte() {
    if (p >= end) throw_format(kInvalidFile, "Unable to read beyond the end of the stream.");
    return *p++;
  }
  bool boolean() { return byte() != 0; }
  int32_t i32() {
    uint32_t v = 0;
    for (int i = 0; i < 4; i++) v |= (uint32_t)byte() << (8 * i);
    return (int32_t)v;
  }
  double f64() {
    uint64_t v = 0;
    for (int i = 0; i < 8; i++) v |= (uint64_t)byte() << (8 * i);
    double d;
    std::memcpy(&d, &v, 8);
    return d;
  }
  // Read7BitEncodedInt: four 7-bit groups, then a fifth byte of at most 4 bits
  int32_t seven() {
    uint32_t r = 0;
    for (int shift = 0; shift < 28; shift += 7) {
      const uint8_t b = byte();
      r |= (uint32_t)(b & 0x7f) << shift;
      if (b <= 0x7f) return (int32_t)r;
    }
    const uint8_t b = byte();
    if (b > 0x0f) throw_format(kInvalidFile, "Too many bytes in what should have been a 7-bit encoded integer.");
    return (int32_t)(r | (uint32_t)b << 28);
  }
  std::string str() {
    const int32_t n = seven();
    if (n < 0) throw_format(kInvalidFile, "BinaryReader encountered an invalid string length of %d characters.", n);
    if (end - p < n) throw_format(kInvalidFile, "Unable to read beyond the end of the stream.");
    std::string s(reinterpret_cast<const char *>(p), (size_t)n);
    p += n;
    return s;
  }
};

// ---- readers (BinaryExecutable.cs:167-200, :278-292; BinaryType.cs:11-28,
//      :43-62; BinaryMember.cs:9-13; BinaryMethod.cs:49-59) -----------------

// Values nest (a List of Lists ...); the reader recurses once per level, so
// the depth is bounded and a deeper file is rejected rather than allowed to
// exhaust the stack.
constexpr int kMaxValueDepth = 256;

Value read_value(Reader &r, const NameTable &t, int depth = 0) {
  if (depth >= kMaxValueDepth)
    throw_format(kInvalidFile, "Values nested deeper than %d levels", kMaxValueDepth);
  Value v;
  v.kind = r.byte();
  switch (v.kind) {
    case kValueText: v.text = t.at(r.seven()); break;
    case kValueNone: break;
    case kValueBoolean: v.number = r.boolean() ? 1.0 : 0.0; break;
    case kValueSmallNumber: v.number = r.byte(); break;
    case kValueIntegerNumber: v.number = r.i32(); break;
    case kValueNumber: v.number = r.f64(); break;
    case kValueList: {
      v.text = t.at(r.seven());
      const int32_t n = r.seven();
      if (n < 0) throw_format(kInvalidFile, "Negative list length %d", n);
      for (int32_t i = 0; i < n; i++) v.items.push_back(read_value(r, t, depth + 1));
      break;
    }
    case kValueDictionary: {
      v.text = t.at(r.seven());
      const int32_t n = r.seven();
      if (n < 0) throw_format(kInvalidFile, "Negative dictionary length %d", n);
      for (int32_t i = 0; i < n; i++) {
        v.items.push_back(read_value(r, t, depth + 1));
        v.items.push_back(read_value(r, t, depth + 1));
      }
      break;
    }
    default: {
      const char *name = value_kind_name(v.kind);
      if (name)
        throw_format(kInvalidFile, "Unknown ValueKind: %s", name);
      throw_format(kInvalidFile, "Unknown ValueKind: %d", v.kind);
    }
  }
  return v;
}

bool is_binary_op(int type) { return type > kStoreSeparator && type < kBinaryOperatorsSeparator; }

Instr read_instruction(Reader &r, const NameTable &t, int &prev_line) {
  Instr in;
  const uint8_t raw = r.byte();
  in.type = raw & (kIncludesSourceLine - 1);
  if (raw & kIncludesSourceLine) prev_line = r.seven();
  switch (in.type) {
    case kLoadConstant:
      in.regs = {r.byte()};
      in.has_value = true;
      in.value = read_value(r, t);
      break;
    case kLoadVariable:
    case kStoreRegister:
    case kWriteToList:
    case kRemove:
      in.regs = {r.byte()};
      in.name = t.at(r.seven());
      break;
    case kStoreConstant:
      in.has_value = true;
      in.value = read_value(r, t);
      in.name = t.at(r.seven());
      in.flag = r.boolean();
      break;
    case kSet:
      in.has_value = true;
      in.value = read_value(r, t);
      in.regs = {r.byte()};
      break;
    case kInvoke: {
      in.regs = {r.byte()};
      in.invoke_type = t.at(r.seven());
      in.name = t.at(r.seven());
      const int32_t np = r.seven();
      if (np < 0) throw_format(kInvalidFile, "Negative parameter count %d", np);
      for (int32_t i = 0; i < np; i++) in.names.push_back(t.at(r.seven()));
      in.invoke_return = t.at(r.seven());
      const int32_t na = r.seven();
      if (na < 0) throw_format(kInvalidFile, "Negative argument count %d", na);
      for (int32_t i = 0; i < na; i++) in.invoke_args.push_back(r.byte());
      if (r.boolean()) in.invoke_instance = r.byte();
      break;
    }
    case kReturn: in.regs = {r.byte()}; break;
    case kLoopBegin: {
      in.regs = {r.byte()};
      if (r.boolean()) {
        in.has_end = true;
        in.regs.push_back(r.seven());
      }
      const int32_t n = r.seven();
      if (n < 0) throw_format(kInvalidFile, "Negative custom variable count %d", n);
      for (int32_t i = 0; i < n; i++) in.names.push_back(t.at(r.seven()));
      break;
    }
    case kLoopEnd:
    case kJump:
    case kJumpIfTrue:
    case kJumpIfFalse:
    case kJumpEnd:
    case kJumpToIdIfFalse:
    case kJumpToIdIfTrue: in.number = r.seven(); break;
    case kJumpIfNotZero:
      in.number = r.seven();
      in.regs = {r.byte()};
      break;
    case kWriteToTable:
      in.regs = {r.byte(), r.byte()};
      in.name = t.at(r.seven());
      break;
    case kListCall:
      in.regs = {r.byte(), r.byte()};
      in.name = t.at(r.seven());
      break;
    case kPrint:
      in.name = t.at(r.seven());
      if (r.boolean()) {
        in.has_print_register = true;
        in.regs = {r.byte()};
        in.flag = r.boolean();
      }
      break;
    default:
      if (is_binary_op(in.type)) {
        const int n = r.byte();
        for (int i = 0; i < n; i++) in.regs.push_back(r.byte());
        break;
      }
      if (const char *name = instruction_type_name(in.type))
        throw_format(kInvalidFile, "Unknown instruction type: %s", name);
      throw_format(kInvalidFile, "Unknown instruction type: %d", in.type);
  }
  in.source_line = prev_line;
  return in;
}

Member read_member(Reader &r, const NameTable &t) {
  Member m;
  m.name = t.at(r.seven());
  m.type = t.at(r.seven());
  if (r.boolean()) {
    int prev = 0;
    m.has_initial = true;
    m.initial = read_instruction(r, t, prev);
  }
  return m;
}

std::vector<Member> read_members(Reader &r, const NameTable &t) {
  const int32_t n = r.seven();
  if (n < 0) throw_format(kInvalidFile, "Negative member count %d", n);
  std::vector<Member> v;
  for (int32_t i = 0; i < n; i++) v.push_back(read_member(r, t));
  return v;
}

void flatten(MethodData &m) {
  m.flat.clear();
  for (const Instr &in : m.instructions) {
    sh_bc_instruction f{};
    f.type = in.type;
    f.register_count = (int)in.regs.size();
    for (size_t j = 0; j < in.regs.size() && j < 3; j++) f.registers[j] = in.regs[j];
    f.identifier = in.name.empty() && in.type != kPrint ? nullptr : in.name.c_str();
    if (in.has_value)
      f.number = (in.value.kind == kValueSmallNumber || in.value.kind == kValueIntegerNumber ||
                  in.value.kind == kValueNumber)
                     ? in.value.number
                     : std::nan("");
    else
      f.number = in.number;
    m.flat.push_back(f);
  }
}

TypeData read_type(const uint8_t *data, size_t size, const std::string &full_name) {
  Reader r{data, data + size};
  // ValidateMagicAndVersion (BinaryType.cs:43-62)
  if (r.byte() != 'S')
    throw_format(kInvalidBytecodeEntry, "Entry does not start with compact 'S' magic byte");
  const uint8_t second = r.byte();
  uint8_t version = second;
  if (second == 't') {
    const char tail[4] = {'r', 'i', 'c', 't'};
    for (char c : tail)
      if (r.p >= r.end || r.byte() != (uint8_t)c)
        throw_format(kInvalidBytecodeEntry, "Entry does not start with supported magic bytes");
    version = r.byte();
  }
  if (version == 0 || version > 1)
    throw_format(kInvalidVersion, "File version: %d, this runtime only supports up to version 1",
                 version);
  TypeData t;
  t.full_name = full_name;
  NameTable table(just_type_name(full_name));
  const int32_t custom = r.seven();
  if (custom < 0) throw_format(kInvalidFile, "Negative name count %d", custom);
  for (int32_t i = 0; i < custom; i++) table.add(r.str());
  t.members = read_members(r, table);
  const int32_t groups = r.seven();
  if (groups < 0) throw_format(kInvalidFile, "Negative method group count %d", groups);
  std::vector<std::vector<MethodData>> overloads_of;  // per entry of group_order
  for (int32_t g = 0; g < groups; g++) {
    const std::string name = table.at(r.seven());
    const int32_t overloads = r.seven();
    if (overloads < 0) throw_format(kInvalidFile, "Negative overload count %d", overloads);
    std::vector<MethodData> group;
    for (int32_t o = 0; o < overloads; o++) {
      MethodData m;
      m.name = name;
      m.parameters = read_members(r, table);
      m.return_type = table.at(r.seven());
      const int32_t count = r.seven();
      if (count < 0) throw_format(kInvalidFile, "Negative instruction count %d", count);
      int prev = 0;
      for (int32_t i = 0; i < count; i++) m.instructions.push_back(read_instruction(r, table, prev));
      group.push_back(std::move(m));
    }
    // MethodGroups[name] = overloads: a repeated name replaces the earlier
    // group's overloads and keeps its place in the dictionary's order
    const auto at = std::find(t.group_order.begin(), t.group_order.end(), name);
    if (at == t.group_order.end()) {
      t.group_order.push_back(name);
      overloads_of.push_back(std::move(group));
    } else {
      overloads_of[(size_t)(at - t.group_order.begin())] = std::move(group);
    }
  }
  for (std::vector<MethodData> &group : overloads_of)
    for (MethodData &m : group) t.methods.push_back(std::move(m));
  t.names = table.names;
  return t;
}

// ---- writers (BinaryType.cs:108-137, BinaryMember.cs:22-28,
//      BinaryMethod.cs:81-89, Instruction.cs, BinaryExecutable.cs:208-267) ---

struct Writer {
  std::vector<uint8_t> out;
  void byte(uint8_t b) { out.push_back(b); }
  void boolean(bool b) { byte(b ? 1 : 0); }
  void i32(int32_t v) {
    for (int i = 0; i < 4; i++) byte((uint8_t)((uint32_t)v >> (8 * i)));
  }
  void f64(double d) {
    uint64_t v;
    std::memcpy(&v, &d, 8);
    for (int i = 0; i < 8; i++) byte((uint8_t)(v >> (8 * i)));
  }
  void seven(int32_t value) {
    uint32_t v = (uint32_t)value;
    while (v > 0x7f) {
      byte((uint8_t)(v | 0x80));
      v >>= 7;
    }
    byte((uint8_t)v);
  }
  void str(const std::string &s) {
    seven((int32_t)s.size());
    out.insert(out.end(), s.begin(), s.end());
  }
};

// The name table a writer builds (BinaryType.CreateNameTable, :88-106;
// NameTable.CollectStrings, :104-163) from the type's contents.
struct TableBuilder {
  NameTable t;
  explicit TableBuilder(const std::string &just) : t(just) {}

  void value(const Value &v) {
    if (v.kind == kValueText) return t.add(v.text);
    if (v.kind == kValueList || v.kind == kValueDictionary) {
      t.add(v.text);
      for (const Value &i : v.items) value(i);
    }
    // Numbers, booleans and None add no name when integral (NameTable.cs:158-161);
    // a fractional Number adds its type's full name
    if ((v.kind == kValueSmallNumber || v.kind == kValueIntegerNumber || v.kind == kValueNumber) &&
        !(v.number >= -2147483648.0 && v.number <= 2147483647.0 && v.number == std::floor(v.number)))
      t.add("Strict/Number");
  }
  void instruction(const Instr &in) {
    switch (in.type) {
      case kLoadVariable:
      case kStoreRegister:
      case kWriteToList:
      case kWriteToTable:
      case kRemove:
      case kListCall:
      case kPrint: t.add(in.name); break;
      case kStoreConstant:
        t.add(in.name);
        value(in.value);
        break;
      case kSet:
      case kLoadConstant: value(in.value); break;
      case kInvoke:
        t.add(in.invoke_type);
        t.add(in.name);
        t.add(in.invoke_return);
        for (const std::string &n : in.names) t.add(n);
        break;
      case kLoopBegin:
        for (const std::string &n : in.names) t.add(n);
        break;
      default: break;
    }
  }
  void member(const Member &m) {
    t.add(m.name);
    t.add(m.type);
    if (m.has_initial) instruction(m.initial);
  }
};

bool is_small_number(double v) { return v >= 0 && v <= 255 && v == std::floor(v); }
bool is_integer_number(double v) {
  return v >= -2147483648.0 && v <= 2147483647.0 && v == std::floor(v);
}

void write_value(Writer &w, const Value &v, const NameTable &t) {
  switch (v.kind) {
    case kValueText:
      w.byte(kValueText);
      w.seven(t[v.text]);
      return;
    case kValueList:
    case kValueDictionary:
      w.byte((uint8_t)v.kind);
      w.seven(t[v.text]);
      w.seven((int32_t)(v.kind == kValueList ? v.items.size() : v.items.size() / 2));
      for (const Value &i : v.items) write_value(w, i, t);
      return;
    case kValueBoolean:
      w.byte(kValueBoolean);
      w.boolean(v.number != 0.0);
      return;
    case kValueNone: w.byte(kValueNone); return;
    default:  // a Number, in the smallest form that holds it
      if (is_small_number(v.number)) {
        w.byte(kValueSmallNumber);
        w.byte((uint8_t)(int)v.number);
      } else if (is_integer_number(v.number)) {
        w.byte(kValueIntegerNumber);
        w.i32((int32_t)v.number);
      } else {
        w.byte(kValueNumber);
        w.f64(v.number);
      }
  }
}

void write_instruction(Writer &w, const Instr &in, const NameTable &t, int &prev_line) {
  if (in.source_line != 0 && in.source_line != prev_line) {
    w.byte((uint8_t)(in.type | kIncludesSourceLine));
    w.seven(in.source_line);
    prev_line = in.source_line;
  } else {
    w.byte((uint8_t)in.type);
  }
  switch (in.type) {
    case kLoadConstant:
      w.byte((uint8_t)in.regs[0]);
      write_value(w, in.value, t);
      break;
    case kLoadVariable:
    case kStoreRegister:
    case kWriteToList:
    case kRemove:
      w.byte((uint8_t)in.regs[0]);
      w.seven(t[in.name]);
      break;
    case kStoreConstant:
      write_value(w, in.value, t);
      w.seven(t[in.name]);
      w.boolean(in.flag);
      break;
    case kSet:
      write_value(w, in.value, t);
      w.byte((uint8_t)in.regs[0]);
      break;
    case kInvoke:
      w.byte((uint8_t)in.regs[0]);
      w.seven(t[in.invoke_type]);
      w.seven(t[in.name]);
      w.seven((int32_t)in.names.size());
      for (const std::string &n : in.names) w.seven(t[n]);
      w.seven(t[in.invoke_return]);
      w.seven((int32_t)in.invoke_args.size());
      for (int a : in.invoke_args) w.byte((uint8_t)a);
      w.boolean(in.invoke_instance >= 0);
      if (in.invoke_instance >= 0) w.byte((uint8_t)in.invoke_instance);
      break;
    case kReturn: w.byte((uint8_t)in.regs[0]); break;
    case kLoopBegin:
      w.byte((uint8_t)in.regs[0]);
      w.boolean(in.has_end);
      if (in.has_end) w.seven(in.regs[1]);
      w.seven((int32_t)in.names.size());
      for (const std::string &n : in.names) w.seven(t[n]);
      break;
    case kLoopEnd:
    case kJump:
    case kJumpIfTrue:
    case kJumpIfFalse:
    case kJumpEnd:
    case kJumpToIdIfFalse:
    case kJumpToIdIfTrue: w.seven(in.number); break;
    case kJumpIfNotZero:
      w.seven(in.number);
      w.byte((uint8_t)in.regs[0]);
      break;
    case kWriteToTable:
    case kListCall:
      w.byte((uint8_t)in.regs[0]);
      w.byte((uint8_t)in.regs[1]);
      w.seven(t[in.name]);
      break;
    case kPrint:
      w.seven(t[in.name]);
      w.boolean(in.has_print_register);
      if (in.has_print_register) {
        w.byte((uint8_t)in.regs[0]);
        w.boolean(in.flag);
      }
      break;
    default:  // binary operators
      w.byte((uint8_t)in.regs.size());
      for (int reg : in.regs) w.byte((uint8_t)reg);
  }
}

void write_members(Writer &w, const std::vector<Member> &members, const NameTable &t) {
  w.seven((int32_t)members.size());
  for (const Member &m : members) {
    w.seven(t[m.name]);
    w.seven(t[m.type]);
    w.boolean(m.has_initial);
    if (m.has_initial) {
      int prev = 0;
      write_instruction(w, m.initial, t, prev);
    }
  }
}

std::vector<uint8_t> write_type(const TypeData &type) {
  TableBuilder b(just_type_name(type.full_name));
  for (const Member &m : type.members) b.member(m);
  for (const std::string &g : type.group_order) {
    b.t.add(g);
    for (const MethodData &m : type.methods) {
      if (m.name != g) continue;
      b.t.add(m.return_type);
      for (const Member &p : m.parameters) b.member(p);
      for (const Instr &in : m.instructions) b.instruction(in);
    }
  }
  const NameTable &t = b.t;
  Writer w;
  w.byte('S');
  w.byte(1);
  w.seven((int32_t)(t.names.size() - t.prefilled));
  for (size_t i = t.prefilled; i < t.names.size(); i++) w.str(t.names[i]);
  write_members(w, type.members, t);
  w.seven((int32_t)type.group_order.size());
  for (const std::string &g : type.group_order) {
    w.seven(t[g]);
    int32_t overloads = 0;
    for (const MethodData &m : type.methods) overloads += m.name == g;
    w.seven(overloads);
    for (const MethodData &m : type.methods) {
      if (m.name != g) continue;
      write_members(w, m.parameters, t);
      w.seven(t[m.return_type]);
      w.seven((int32_t)m.instructions.size());
      int prev = 0;
      for (const Instr &in : m.instructions) write_instruction(w, in, t, prev);
    }
  }
  return w.out;
}

// ---- ZIP (PKWARE APPNOTE: local headers, central directory, end record) ----

uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }
uint32_t le32(const uint8_t *p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

struct ZipEntry {
  std::string name;
  std::vector<uint8_t> data;
};

std::vector<ZipEntry> read_zip(const uint8_t *d, size_t n) {
  // end of central directory: signature 0x06054b50, 22 bytes plus a comment
  size_t eocd = (size_t)-1;
  if (n >= 22)
    for (size_t i = n - 22 + 1; i-- > 0 && n - i <= 22 + 65535;)
      if (le32(d + i) == 0x06054b50u && i + 22 + le16(d + i + 20) == n) {
        eocd = i;
        break;
      }
  if (eocd == (size_t)-1)
    throw_format(kInvalidFile, "End of Central Directory record could not be found.");
  const uint32_t count = le16(d + eocd + 10);
  const uint32_t cd_size = le32(d + eocd + 12), cd_off = le32(d + eocd + 16);
  if (cd_off == 0xffffffffu || count == 0xffffu)
    throw_format(kInvalidFile, "ZIP64 archives are not supported");
  if ((size_t)cd_off + cd_size > eocd)
    throw_format(kInvalidFile, "Central directory outside the archive");
  std::vector<ZipEntry> entries;
  size_t p = cd_off;
  for (uint32_t e = 0; e < count; e++) {
    if (p + 46 > eocd || le32(d + p) != 0x02014b50u)
      throw_format(kInvalidFile, "Central directory corrupt");
    const uint16_t flags = le16(d + p + 8), method = le16(d + p + 10);
    const uint32_t crc = le32(d + p + 16), csize = le32(d + p + 20), usize = le32(d + p + 24);
    const uint16_t nlen = le16(d + p + 28), xlen = le16(d + p + 30), clen = le16(d + p + 32);
    const uint32_t local = le32(d + p + 42);
    if (p + 46 + nlen > eocd) throw_format(kInvalidFile, "Central directory corrupt");
    ZipEntry z;
    z.name.assign(reinterpret_cast<const char *>(d + p + 46), nlen);
    p += 46 + (size_t)nlen + xlen + clen;
    if (flags & 1) throw_format(kInvalidFile, "Encrypted entry %s", z.name.c_str());
    if ((size_t)local + 30 > n || le32(d + local) != 0x04034b50u)
      throw_format(kInvalidFile, "Local file header corrupt");
    const size_t data_off = (size_t)local + 30 + le16(d + local + 26) + le16(d + local + 28);
    if (data_off + csize > n) throw_format(kInvalidFile, "Entry %s outside the archive", z.name.c_str());
    if (method == 0) {
      if (csize != usize) throw_format(kInvalidFile, "Stored entry %s has inconsistent sizes", z.name.c_str());
      z.data.assign(d + data_off, d + data_off + csize);
    } else if (method == 8) {
      // deflate expands at most ~1032:1, so a larger declared size is a
      // corrupt (or hostile) header; it is rejected before anything is
      // allocated for it
      if ((uint64_t)usize > (uint64_t)csize * 1032 + 64)
        throw_format(kInvalidFile, "Entry %s declares %u bytes from %u compressed", z.name.c_str(),
                     usize, csize);
      z.data.resize(usize);
      z_stream zs{};
      if (inflateInit2(&zs, -MAX_WBITS) != Z_OK) throw_format(kInvalidFile, "inflateInit2 failed");
      zs.next_in = const_cast<Bytef *>(d + data_off);
      zs.avail_in = csize;
      zs.next_out = z.data.data();
      zs.avail_out = usize;
      uint8_t spare;
      if (usize == 0) {  // an empty entry still holds a deflate end block
        zs.next_out = &spare;
        zs.avail_out = 1;
      }
      const int rc = inflate(&zs, Z_FINISH);
      const size_t produced = usize == 0 ? 1 - zs.avail_out : usize - zs.avail_out;
      inflateEnd(&zs);
      if (rc != Z_STREAM_END || produced != usize)
        throw_format(kInvalidFile, "Entry %s: the deflate stream is corrupt", z.name.c_str());
    } else {
      throw_format(kInvalidFile, "Entry %s: unsupported compression method %d", z.name.c_str(), method);
    }
    if ((uint32_t)crc32(0L, z.data.data(), (uInt)z.data.size()) != crc)
      throw_format(kInvalidFile, "Entry %s: CRC-32 mismatch", z.name.c_str());
    entries.push_back(std::move(z));
  }
  return entries;
}

void put16(std::vector<uint8_t> &o, uint32_t v) {
  o.push_back((uint8_t)v);
  o.push_back((uint8_t)(v >> 8));
}
void put32(std::vector<uint8_t> &o, uint32_t v) {
  put16(o, v & 0xffff);
  put16(o, v >> 16);
}

std::vector<uint8_t> write_zip(const std::vector<ZipEntry> &entries) {
  std::vector<uint8_t> out, cd;
  for (const ZipEntry &e : entries) {
    // raw deflate at the default level (the reference asks for Optimal)
    z_stream zs{};
    if (deflateInit2(&zs, Z_DEFAULT_COMPRESSION, Z_DEFLATED, -MAX_WBITS, 8, Z_DEFAULT_STRATEGY) != Z_OK)
      throw_format(kInvalidFile, "deflateInit2 failed");
    std::vector<uint8_t> comp(deflateBound(&zs, (uLong)e.data.size()) + 16);
    zs.next_in = const_cast<Bytef *>(e.data.data());
    zs.avail_in = (uInt)e.data.size();
    zs.next_out = comp.data();
    zs.avail_out = (uInt)comp.size();
    const int rc = deflate(&zs, Z_FINISH);
    comp.resize(comp.size() - zs.avail_out);
    deflateEnd(&zs);
    if (rc != Z_STREAM_END) throw_format(kInvalidFile, "deflate failed");
    const uint32_t crc = (uint32_t)crc32(0L, e.data.data(), (uInt)e.data.size());
    bool utf8 = false;
    for (unsigned char c : e.name) utf8 |= c >= 0x80;
    const uint16_t flags = utf8 ? 0x0800 : 0;
    const uint32_t local = (uint32_t)out.size();
    put32(out, 0x04034b50u);
    put16(out, 20); put16(out, flags); put16(out, 8); put16(out, 0); put16(out, 0x21);
    put32(out, crc); put32(out, (uint32_t)comp.size()); put32(out, (uint32_t)e.data.size());
    put16(out, (uint32_t)e.name.size()); put16(out, 0);
    out.insert(out.end(), e.name.begin(), e.name.end());
    out.insert(out.end(), comp.begin(), comp.end());
    put32(cd, 0x02014b50u);
    put16(cd, 20); put16(cd, 20); put16(cd, flags); put16(cd, 8); put16(cd, 0); put16(cd, 0x21);
    put32(cd, crc); put32(cd, (uint32_t)comp.size()); put32(cd, (uint32_t)e.data.size());
    put16(cd, (uint32_t)e.name.size()); put16(cd, 0); put16(cd, 0); put16(cd, 0); put16(cd, 0);
    put32(cd, 0); put32(cd, local);
    cd.insert(cd.end(), e.name.begin(), e.name.end());
  }
  const uint32_t cd_off = (uint32_t)out.size();
  out.insert(out.end(), cd.begin(), cd.end());
  put32(out, 0x06054b50u);
  put16(out, 0); put16(out, 0);
  put16(out, (uint32_t)entries.size()); put16(out, (uint32_t)entries.size());
  put32(out, (uint32_t)cd.size()); put32(out, cd_off);
  put16(out, 0);
  return out;
}

bool ends_with_bytecode(const std::string &name) {
  static const char ext[] = ".bytecode";
  const size_t n = sizeof ext - 1;
  if (name.size() < n) return false;
  for (size_t i = 0; i < n; i++)
    if (std::tolower((unsigned char)name[name.size() - n + i]) != ext[i]) return false;
  return true;
}

// GetEntryNameWithoutExtension (BinaryExecutable.cs:86-93)
std::string entry_type_name(const std::string &entry) {
  std::string s = entry;
  std::replace(s.begin(), s.end(), '\\', '/');
  const size_t dot = s.rfind('.');
  return dot != std::string::npos && dot > 0 ? s.substr(0, dot) : s;
}

int report(const FormatError &e) {
  static const char *kinds[] = {"InvalidFile", "InvalidBytecodeEntry", "InvalidVersion"};
  return fail(SH_ERR_INVALID_FILE, "%s: %s", kinds[e.kind], e.message.c_str());
}

bool numeric(const Value &v) {
  return v.kind == kValueSmallNumber || v.kind == kValueIntegerNumber || v.kind == kValueNumber;
}

// Numbers a constant holds: 1 for a Number, the items of a List whose items
// are all Numbers, 0 for anything else.
size_t numbers_in(const Value &v) {
  if (numeric(v)) return 1;
  if (v.kind != kValueList) return 0;
  for (const Value &i : v.items)
    if (!numeric(i)) return 0;
  return v.items.size();
}

}  // namespace
}  // namespace sh

struct sh_strictbinary {
  std::vector<sh::TypeData> types;
  std::vector<uint8_t> serialized;  // cached sh_strictbinary_serialize output
  // constants listed per (type, method), cached for the pointers handed out
  std::map<std::pair<int, int>, std::vector<std::pair<const sh::Value *, sh_strictbinary_constant>>> constants;
};

namespace sh {
namespace {

int check_type(const sh_strictbinary *b, int type) {
  if (!b) return fail(SH_ERR_INVALID_ARGUMENT, "binary is NULL");
  if (type < 0 || (size_t)type >= b->types.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "type index %d outside 0..%zu", type, b->types.size());
  return SH_OK;
}

int check_method(const sh_strictbinary *b, int type, int method) {
  int rc = check_type(b, type);
  if (rc != SH_OK) return rc;
  if (method < 0 || (size_t)method >= b->types[(size_t)type].methods.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "method index %d outside 0..%zu", method,
                b->types[(size_t)type].methods.size());
  return SH_OK;
}

// The value-carrying instructions of a method (method >= 0) or the members'
// initial values (method == -1), listed once and kept in the handle.
int list_constants(sh_strictbinary *b, int type, int method,
                   const std::vector<std::pair<const Value *, sh_strictbinary_constant>> **out) {
  int rc = method == -1 ? check_type(b, type) : check_method(b, type, method);
  if (rc != SH_OK) return rc;
  auto key = std::make_pair(type, method);
  auto it = b->constants.find(key);
  if (it == b->constants.end()) {
    std::vector<std::pair<const Value *, sh_strictbinary_constant>> v;
    const TypeData &t = b->types[(size_t)type];
    auto add = [&](const Instr &in, int index, const char *member) {
      if (!in.has_value) return;
      sh_strictbinary_constant c{};
      c.instruction = index;
      c.instruction_type = in.type;
      c.kind = in.value.kind;
      c.register_id = in.regs.empty() ? -1 : in.regs[0];
      c.identifier = member ? member : (in.type == kStoreConstant ? in.name.c_str() : nullptr);
      c.count = numbers_in(in.value);
      v.emplace_back(&in.value, c);
    };
    if (method == -1) {
      for (size_t i = 0; i < t.members.size(); i++)
        if (t.members[i].has_initial) add(t.members[i].initial, (int)i, t.members[i].name.c_str());
    } else {
      const MethodData &m = t.methods[(size_t)method];
      for (size_t i = 0; i < m.instructions.size(); i++) add(m.instructions[i], (int)i, nullptr);
    }
    it = b->constants.emplace(key, std::move(v)).first;
  }
  *out = &it->second;
  return SH_OK;
}

int constant_numbers(sh_strictbinary *b, int type, int method, int index, std::vector<double> &vals) {
  const std::vector<std::pair<const Value *, sh_strictbinary_constant>> *list;
  int rc = list_constants(b, type, method, &list);
  if (rc != SH_OK) return rc;
  if (index < 0 || (size_t)index >= list->size())
    return fail(SH_ERR_INVALID_ARGUMENT, "constant index %d outside 0..%zu", index, list->size());
  const Value &v = *(*list)[(size_t)index].first;
  if ((*list)[(size_t)index].second.count == 0 && !(v.kind == kValueList && v.items.empty()))
    return fail(SH_ERR_INVALID_ARGUMENT, "constant %d is a %s, not a Number or a List of Numbers",
                index, value_kind_name(v.kind) ? value_kind_name(v.kind) : "value");
  vals.clear();
  if (numeric(v)) {
    vals.push_back(v.number);
  } else {
    for (const Value &i : v.items) vals.push_back(i.number);
  }
  return SH_OK;
}

}  // namespace
}  // namespace sh

using namespace sh;

extern "C" {

SH_API int sh_strictbinary_load(const void *data, size_t bytes, sh_strictbinary **binary) {
  if (!binary || (!data && bytes)) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  *binary = nullptr;
  auto *b = new sh_strictbinary();
  try {
    const auto entries = read_zip(static_cast<const uint8_t *>(data), bytes);
    for (const ZipEntry &e : entries) {
      if (!ends_with_bytecode(e.name)) continue;
      const std::string name = entry_type_name(e.name);
      for (const TypeData &t : b->types)
        if (t.full_name == name)
          throw_format(kInvalidFile, "An item with the same key has already been added. Key: %s",
                       name.c_str());
      b->types.push_back(read_type(e.data.data(), e.data.size(), name));
    }
  } catch (const FormatError &e) {
    delete b;
    return report(e);
  } catch (const std::bad_alloc &) {
    delete b;
    return fail(SH_ERR_OUT_OF_MEMORY, "out of host memory reading the file");
  } catch (const std::exception &e) {
    delete b;
    return fail(SH_ERR_INVALID_FILE, "InvalidFile: %s", e.what());
  }
  // the flat views point into the instructions' strings: built once the
  // types have their final place
  for (TypeData &t : b->types)
    for (MethodData &m : t.methods) flatten(m);
  *binary = b;
  return SH_OK;
}

SH_API int sh_strictbinary_free(sh_strictbinary *binary) {
  delete binary;
  return SH_OK;
}

SH_API int sh_strictbinary_type_count(const sh_strictbinary *binary, int *count) {
  if (!binary || !count) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  *count = (int)binary->types.size();
  return SH_OK;
}

SH_API int sh_strictbinary_type(const sh_strictbinary *binary, int type_index,
                                const char **full_name, int *member_count, int *method_count) {
  int rc = check_type(binary, type_index);
  if (rc != SH_OK) return rc;
  const TypeData &t = binary->types[(size_t)type_index];
  if (full_name) *full_name = t.full_name.c_str();
  if (member_count) *member_count = (int)t.members.size();
  if (method_count) *method_count = (int)t.methods.size();
  return SH_OK;
}

SH_API int sh_strictbinary_member(const sh_strictbinary *binary, int type_index, int method_index,
                                  int member_index, const char **name, const char **full_type_name,
                                  int *has_initial_value) {
  int rc = method_index == -1 ? check_type(binary, type_index)
                              : check_method(binary, type_index, method_index);
  if (rc != SH_OK) return rc;
  const TypeData &t = binary->types[(size_t)type_index];
  const std::vector<Member> &ms =
      method_index == -1 ? t.members : t.methods[(size_t)method_index].parameters;
  if (member_index < 0 || (size_t)member_index >= ms.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "member index %d outside 0..%zu", member_index, ms.size());
  const Member &m = ms[(size_t)member_index];
  if (name) *name = m.name.c_str();
  if (full_type_name) *full_type_name = m.type.c_str();
  if (has_initial_value) *has_initial_value = m.has_initial ? 1 : 0;
  return SH_OK;
}

SH_API int sh_strictbinary_method(const sh_strictbinary *binary, int type_index, int method_index,
                                  const char **name, int *parameter_count,
                                  const char **return_type, int *instruction_count) {
  int rc = check_method(binary, type_index, method_index);
  if (rc != SH_OK) return rc;
  const MethodData &m = binary->types[(size_t)type_index].methods[(size_t)method_index];
  if (name) *name = m.name.c_str();
  if (parameter_count) *parameter_count = (int)m.parameters.size();
  if (return_type) *return_type = m.return_type.c_str();
  if (instruction_count) *instruction_count = (int)m.instructions.size();
  return SH_OK;
}

SH_API int sh_strictbinary_entry_point(const sh_strictbinary *binary, int *type_index,
                                       int *method_index) {
  if (!binary || !type_index || !method_index) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  for (size_t t = 0; t < binary->types.size(); t++)
    for (size_t m = 0; m < binary->types[t].methods.size(); m++)
      if (binary->types[t].methods[m].name == "Run") {
        *type_index = (int)t;
        *method_index = (int)m;
        return SH_OK;
      }
  return fail(SH_ERR_NOT_FOUND, "No Run entry point found in binary executable");
}

SH_API int sh_strictbinary_find(const sh_strictbinary *binary, const char *type_full_name,
                                const char *method_name, int parameter_count,
                                const char *return_type, int *type_index, int *method_index) {
  if (!binary || !type_full_name || !method_name || !type_index || !method_index)
    return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  const std::string expected = return_type ? return_type : "";
  auto ends_with = [](const std::string &s, const std::string &tail) {
    return s.size() >= tail.size() && s.compare(s.size() - tail.size(), tail.size(), tail) == 0;
  };
  for (size_t t = 0; t < binary->types.size(); t++) {
    if (binary->types[t].full_name != type_full_name) continue;
    for (size_t m = 0; m < binary->types[t].methods.size(); m++) {
      const MethodData &md = binary->types[t].methods[m];
      if (md.name != method_name || (int)md.parameters.size() != parameter_count) continue;
      const std::string &stored = md.return_type;
      // DoesReturnTypeMatch (BinaryExecutable.cs:133-138)
      if (expected.empty() || stored == expected || ends_with(stored, "/" + expected) ||
          ends_with(expected, "/" + stored)) {
        *type_index = (int)t;
        *method_index = (int)m;
        return SH_OK;
      }
    }
  }
  return fail(SH_ERR_NOT_FOUND, "no %s.%s with %d parameters returning '%s'", type_full_name,
              method_name, parameter_count, expected.c_str());
}

SH_API int sh_strictbinary_instructions(const sh_strictbinary *binary, int type_index,
                                        int method_index, sh_bc_instruction *instructions,
                                        int capacity, int *count) {
  int rc = check_method(binary, type_index, method_index);
  if (rc != SH_OK) return rc;
  if (!count) return fail(SH_ERR_INVALID_ARGUMENT, "count is NULL");
  const MethodData &m = binary->types[(size_t)type_index].methods[(size_t)method_index];
  *count = (int)m.flat.size();
  if (!instructions) return SH_OK;
  if (capacity < (int)m.flat.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "capacity %d < %zu instructions", capacity, m.flat.size());
  std::copy(m.flat.begin(), m.flat.end(), instructions);
  return SH_OK;
}

SH_API int sh_strictbinary_constants(sh_strictbinary *binary, int type_index, int method_index,
                                     sh_strictbinary_constant *constants, int capacity, int *count) {
  if (!count) return fail(SH_ERR_INVALID_ARGUMENT, "count is NULL");
  const std::vector<std::pair<const Value *, sh_strictbinary_constant>> *list;
  int rc = list_constants(binary, type_index, method_index, &list);
  if (rc != SH_OK) return rc;
  *count = (int)list->size();
  if (!constants) return SH_OK;
  if (capacity < (int)list->size())
    return fail(SH_ERR_INVALID_ARGUMENT, "capacity %d < %zu constants", capacity, list->size());
  for (size_t i = 0; i < list->size(); i++) constants[i] = (*list)[i].second;
  return SH_OK;
}

SH_API int sh_strictbinary_constant_values(sh_strictbinary *binary, int type_index,
                                           int method_index, int constant_index, double *values,
                                           size_t capacity) {
  std::vector<double> v;
  int rc = constant_numbers(binary, type_index, method_index, constant_index, v);
  if (rc != SH_OK) return rc;
  if (!values && !v.empty()) return fail(SH_ERR_INVALID_ARGUMENT, "values is NULL");
  if (capacity < v.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "capacity %zu < %zu numbers", capacity, v.size());
  std::copy(v.begin(), v.end(), values);
  return SH_OK;
}

SH_API int sh_strictbinary_upload_f32(sh_ctx *ctx, sh_strictbinary *binary, int type_index,
                                      int method_index, int constant_index, float *device_dst,
                                      size_t capacity) {
  int rc = enter(ctx);
  if (rc != SH_OK) return rc;
  std::vector<double> v;
  if ((rc = constant_numbers(binary, type_index, method_index, constant_index, v)) != SH_OK)
    return rc;
  if (capacity < v.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "capacity %zu < %zu numbers", capacity, v.size());
  if (v.empty()) return SH_OK;
  if ((rc = check_range(ctx, device_dst, v.size() * sizeof(float), "device_dst")) != SH_OK) return rc;
  std::vector<float> f(v.size());
  for (size_t i = 0; i < v.size(); i++) f[i] = (float)v[i];  // round to nearest even
  hipStream_t s = stream_of(ctx);
  SH_HIP_TRY(hipMemcpyAsync(device_dst, f.data(), f.size() * sizeof(float), hipMemcpyHostToDevice, s));
  SH_HIP_TRY(hipStreamSynchronize(s));  // `f` is a local buffer
  return SH_OK;
}

SH_API int sh_strictbinary_serialize(sh_strictbinary *binary, void *data, size_t capacity,
                                     size_t *bytes) {
  if (!binary || !bytes) return fail(SH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (binary->serialized.empty()) {
    try {
      std::vector<ZipEntry> entries;
      for (const TypeData &t : binary->types) entries.push_back({t.full_name + ".bytecode", write_type(t)});
      binary->serialized = write_zip(entries);
    } catch (const FormatError &e) {
      return report(e);
    } catch (const std::out_of_range &) {
      return fail(SH_ERR_INVALID_ARGUMENT, "a name is missing from the name table");
    } catch (const std::bad_alloc &) {
      return fail(SH_ERR_OUT_OF_MEMORY, "out of host memory serializing");
    } catch (const std::exception &e) {
      return fail(SH_ERR_INVALID_ARGUMENT, "serializing: %s", e.what());
    }
  }
  *bytes = binary->serialized.size();
  if (!data) return SH_OK;
  if (capacity < binary->serialized.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "capacity %zu < %zu bytes", capacity, binary->serialized.size());
  std::memcpy(data, binary->serialized.data(), binary->serialized.size());
  return SH_OK;
}

}  // extern "C"
