// Elementwise kernel source generation from Strict bytecode: the native
// counterpart of InstructionsToCuda.BuildCudaKernel
// (Strict.Compiler.Cuda/InstructionsToCuda.cs:19-74). Host code only; the
// text it writes is compiled for gfx950 by sh_compile (hipRTC).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common.h"

namespace sh {
namespace {

// One folded register value: its C text and how tightly it binds
// (kAtom for names, constants and "0"; then multiplicative, additive).
enum Binding { kAdditive = 1, kMultiplicative = 2, kAtom = 3 };
struct Expr {
  std::string text;
  int binding = kAtom;
};

// double.ToString(CultureInfo.InvariantCulture) of .NET Core 3.0 and later,
// which InstructionsToCuda.cs:41-42 uses for constants: the shortest digit
// string that reads back to the same double, in fixed notation for decimal
// exponents -4 .. 14 (0.0001, 123456789012345) and as d[.ddd]E+XX / E-XX
// (at least two exponent digits: 1E-05, 1E+15) outside that range; "NaN",
// "Infinity", "-Infinity" for the special values.
std::string dotnet_double(double v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "Infinity" : "-Infinity";
  const bool negative = std::signbit(v);
  if (v == 0.0) return negative ? "-0" : "0";
  char buf[64];
  for (int p = 0; p <= 16; p++) {  // %.{p}e has p + 1 significant digits
    std::snprintf(buf, sizeof buf, "%.*e", p, std::fabs(v));
    if (std::strtod(buf, nullptr) == std::fabs(v)) break;
  }
  // buf = d[.ddd]e[+-]XX
  std::string digits;
  const char *c = buf;
  for (; *c && *c != 'e'; c++)
    if (*c >= '0' && *c <= '9') digits += *c;
  const int exp10 = std::atoi(c + 1);
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  std::string out = negative ? "-" : "";
  if (exp10 >= 15 || exp10 < -4) {
    out += digits[0];
    if (digits.size() > 1) out += "." + digits.substr(1);
    char e[16];
    std::snprintf(e, sizeof e, "E%c%02d", exp10 < 0 ? '-' : '+', std::abs(exp10));
    return out + e;
  }
  if (exp10 < 0) return out + "0." + std::string(-exp10 - 1, '0') + digits;
  const size_t int_digits = (size_t)exp10 + 1;
  if (digits.size() <= int_digits) return out + digits + std::string(int_digits - digits.size(), '0');
  return out + digits.substr(0, int_digits) + "." + digits.substr(int_digits);
}

// InstructionsToCuda.cs:92-96: width and height are int scalars,
// initialDepth a float scalar; every other Number parameter is an array.
bool is_scalar_name(const std::string &n) {
  return n == "width" || n == "height" || n == "initialDepth";
}

// InstructionsToCuda.cs:101-109
const char *operator_symbol(int type) {
  switch (type) {
    case SH_BC_ADD: return "+";
    case SH_BC_SUBTRACT: return "-";
    case SH_BC_MULTIPLY: return "*";
    case SH_BC_DIVIDE: return "/";
    default: return nullptr;
  }
}

const char *instruction_name(int type) {
  switch (type) {
    case SH_BC_MODULO: return "Modulo";
    default: return "binary instruction";
  }
}

}  // namespace
}  // namespace sh

using namespace sh;

extern "C" SH_API int sh_instructions_to_hip(const char *method_name,
                                             const char *const *parameters, int parameter_count,
                                             int add_count_parameter,
                                             const sh_bc_instruction *instructions,
                                             int instruction_count, char *source,
                                             size_t capacity, size_t *length) {
  if (!length) return fail(SH_ERR_INVALID_ARGUMENT, "length out-pointer is NULL");
  *length = 0;
  if (!method_name || !*method_name) return fail(SH_ERR_INVALID_ARGUMENT, "empty method name");
  if (parameter_count < 0 || (parameter_count > 0 && !parameters))
    return fail(SH_ERR_INVALID_ARGUMENT, "bad parameter array");
  if (instruction_count < 0 || (instruction_count > 0 && !instructions))
    return fail(SH_ERR_INVALID_ARGUMENT, "bad instruction array");
  std::vector<std::string> params;
  for (int i = 0; i < parameter_count; i++) {
    if (!parameters[i] || !*parameters[i])
      return fail(SH_ERR_INVALID_ARGUMENT, "parameter %d has no name", i);
    params.emplace_back(parameters[i]);
  }
  auto has_param = [&](const char *n) {
    for (const auto &p : params)
      if (p == n) return true;
    return false;
  };

  // Fold the registers into one C expression (InstructionsToCuda.cs:29-54).
  std::map<int, Expr> regs;
  std::string output = "0.0f";
  auto operand = [&](int r) {
    const auto it = regs.find(r);
    return it == regs.end() ? Expr{"0", kAtom} : it->second;
  };
  for (int i = 0; i < instruction_count; i++) {
    const sh_bc_instruction &in = instructions[i];
    if (in.register_count < 0 || in.register_count > 3)
      return fail(SH_ERR_INVALID_ARGUMENT, "instruction %d: register_count %d", i,
                  in.register_count);
    const bool loads = in.type == SH_BC_LOAD_VARIABLE || in.type == SH_BC_LOAD_CONSTANT ||
                       in.type == SH_BC_RETURN;
    if (loads && in.register_count < 1)
      return fail(SH_ERR_INVALID_ARGUMENT, "instruction %d has no register", i);
    if (in.type == SH_BC_LOAD_VARIABLE) {
      if (!in.identifier || !*in.identifier)
        return fail(SH_ERR_INVALID_ARGUMENT, "instruction %d: variable without a name", i);
      const std::string name = in.identifier;
      const bool scalar = has_param(name.c_str()) && is_scalar_name(name);
      regs[in.registers[0]] = Expr{scalar ? name : name + "[idx]", kAtom};
    } else if (in.type == SH_BC_LOAD_CONSTANT) {
      regs[in.registers[0]] = Expr{dotnet_double(in.number), kAtom};
    } else if (in.type > 10 && in.type < 20) {  // arithmetic BinaryInstruction
      if (in.register_count <= 2) continue;
      const char *op = operator_symbol(in.type);
      if (!op)
        return fail(SH_ERR_UNSUPPORTED, "%s (instruction type %d) has no kernel operator",
                    instruction_name(in.type), in.type);
      const int binding =
          (in.type == SH_BC_ADD || in.type == SH_BC_SUBTRACT) ? kAdditive : kMultiplicative;
      const Expr l = operand(in.registers[0]), r = operand(in.registers[1]);
      // C groups left to right: a left operand keeps its grouping unless it
      // binds more loosely; a right operand needs parentheses unless it binds
      // more tightly (a - (b - c), a * (b + c), and the same for + and *,
      // whose floating-point evaluation order matters too)
      const std::string lt = l.binding < binding ? "(" + l.text + ")" : l.text;
      const std::string rt = r.binding <= binding ? "(" + r.text + ")" : r.text;
      regs[in.registers[2]] = Expr{lt + " " + op + " " + rt, binding};
    } else if (in.type == SH_BC_RETURN) {
      const auto it = regs.find(in.registers[0]);
      if (it != regs.end()) output = it->second.text;
    }
    // conditional binaries (21..24) and all other instructions: skipped
  }

  // Signature and bounds check (InstructionsToCuda.cs:55-99).
  std::string signature;
  for (const auto &p : params) {
    if (!signature.empty()) signature += ", ";
    if (p == "width" || p == "height")
      signature += "const int " + p;
    else if (p == "initialDepth")
      signature += "const float " + p;
    else
      signature += "const float *" + p;
  }
  signature += signature.empty() ? "float *output" : ", float *output";
  if (add_count_parameter) signature += ", const int count";
  const bool by_count = add_count_parameter || !has_param("width") || !has_param("height");
  const std::string index =
      by_count ? "y * gridDim.x * blockDim.x + x" : "y * width + x";
  const std::string check = by_count ? "idx >= count" : "x >= width || y >= height";

  std::string text;
  text += "extern \"C\" __global__ void " + std::string(method_name) + "(" + signature + ")\n";
  text += "{\n";
  text += "\tint x = blockIdx.x * blockDim.x + threadIdx.x;\n";
  text += "\tint y = blockIdx.y * blockDim.y + threadIdx.y;\n";
  text += "\tint idx = " + index + ";\n";
  text += "\tif (" + check + ") return;\n";
  text += "\toutput[idx] = " + output + ";\n";
  text += "}\n";

  *length = text.size();
  if (!source || capacity <= text.size())
    return fail(SH_ERR_INVALID_ARGUMENT, "source buffer of %zu bytes, %zu needed", capacity,
                text.size() + 1);
  std::memcpy(source, text.c_str(), text.size() + 1);
  return SH_OK;
}

// InstructionsToMlir.cs:397-408: complexity = iterations * max(body, 1),
// compared strictly against the two thresholds. The product saturates.
extern "C" SH_API int sh_range_loop_target(long long iterations, int body_instructions) {
  const long long n = iterations > 0 ? iterations : 0;
  const long long body = body_instructions > 1 ? body_instructions : 1;
  const long long complexity = n > INT64_MAX / body ? INT64_MAX : n * body;
  if (complexity > SH_GPU_COMPLEXITY_THRESHOLD) return SH_LOOP_GPU;
  if (complexity > SH_PARALLEL_COMPLEXITY_THRESHOLD) return SH_LOOP_PARALLEL;
  return SH_LOOP_SERIAL;
}
