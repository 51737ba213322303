"""Kernel source generation on the CPU: InstructionsToHip and
CSharpToHipTranspiler against the strings and errors the reference's own tests
pin (Strict.Compiler.Cuda.Tests/InstructionsToCudaTests.cs:13-51,
CSharpToCudaTranspilerTests.cs:19-44), and hipRTC compiles of what they emit
(hipRTC needs no GPU). Launching the generated kernels is tests/test_gpu_codegen.py.

Two deliberate differences from the reference's text are asserted here as
such: the element index is the true row-major one, and nested binary operands
are parenthesised where C would regroup them."""
import pytest

import strict_amd
from strict_amd import codegen as cg

C_SHARP_INPUTS = {
    # One-method C# files in the shapes CSharpType's line parser reads
    # (CSharpToCudaTranspiler.cs:46-98): lines holding the type name, braces,
    # `using`/`namespace`, `this.`, `\tprivate ` or `\t\tfor ` are skipped; a
    # line starting `\t\treturn` or `\t\t\t` is the body; any other line is
    # the method line, `<access> float|void Name(float a, ...)`.
    "AddNumbers": "using System.Numerics;\n\nnamespace KernelSamples.Arithmetic;\n\n"
                  "internal sealed class AddNumbers\n{\n\tinternal float Add(float left, float right)"
                  "\n\t{\n\t\treturn left + right;\n\t}\n}\n",
    # block-scoped namespace: the method line is indented twice and the body
    # is a `\t\t\treturn` line
    "SubtractNumbers": "namespace KernelSamples.Arithmetic\n{\n\tpublic record SubtractNumbers\n\t{\n"
                       "\t\tpublic float Subtract(float minuend, float subtrahend)\n\t\t{\n"
                       "\t\t\treturn minuend - subtrahend;\n\t\t}\n\t}\n}\n",
    "MultiplyNumbers": "public struct MultiplyNumbers\n{\n\tpublic float Multiply(float factor, "
                       "float multiplier)\n\t{\n\t\treturn factor * multiplier;\n\t}\n}\n",
    # DepthImage expands to (input, width, height, initialDepth); the body is
    # the right-hand side of the `\t\t\t... = value;` line
    "InitializeDepths": "using System;\n\nnamespace DepthTools;\n\n"
                        "public sealed class InitializeDepths(float initialDepth)\n{\n"
                        "\tprivate float Start => initialDepth;\n\n"
                        "\tpublic void Process(DepthImage image)\n\t{\n"
                        "\t\tfor (var row = 0; row < image.Height; row++)\n"
                        "\t\tfor (var column = 0; column < image.Width; column++)\n"
                        "\t\t\timage.Depths[row * image.Width + column] = initialDepth;\n\t}\n}\n",
    # an expression statement is not a return: no body line is found
    "MissingReturnStatement": "public class MissingReturnStatement\n{\n\tpublic float Half(float value)"
                              "\n\t{\n\t\tvalue / 2;\n\t}\n}\n",
    "TakesInts": "public class TakesInts\n{\n\tpublic float Twice(int value)\n\t{\n\t\treturn value + value;\n\t}\n}\n",
}


def write_input(tmp_path, name):
    path = tmp_path / f"{name}.cs"
    path.write_text("﻿" + C_SHARP_INPUTS[name], encoding="utf-8")  # BOM, as the C# files carry
    return str(path)


def single_method(*lines):
    return cg.Method.parse(list(lines))


@pytest.mark.parametrize("name,op", [("Add", "+"), ("Subtract", "-"), ("Multiply", "*"),
                                     ("Divide", "/")])
def test_generate_array_operation_kernel(name, op):
    # InstructionsToCudaTests.GenerateArrayOperationKernel (cs:13-27)
    method = single_method(f"{name}(first Number, second Number) Number", f"\tfirst {op} second")
    hip = cg.InstructionsToHip().compile(method)
    assert (f"void {name}(const float *first, const float *second, float *output, "
            "const int count)") in hip
    assert f"output[idx] = first[idx] {op} second[idx]" in hip


def test_generate_scalar_output_kernel():
    # InstructionsToCudaTests.GenerateScalarOutputKernel (cs:29-40)
    method = single_method("Process(input Number, width Number, height Number, initialDepth Number) Number",
                           "\tinitialDepth")
    hip = cg.InstructionsToHip().compile(method)
    assert ("void Process(const float *input, const int width, const int height, "
            "const float initialDepth, float *output)") in hip
    assert "output[idx] = initialDepth" in hip
    assert "if (x >= width || y >= height) return;" in hip
    assert "int idx = y * width + x;" in hip


def test_kernel_contains_thread_indexing():
    # InstructionsToCudaTests.KernelContainsCudaThreadIndexing (cs:42-51); the
    # index line is the row-major one instead of the reference's aliasing
    # `y * blockDim.x + x`
    hip = cg.InstructionsToHip().compile(single_method("Add(first Number, second Number) Number",
                                                       "\tfirst + second"))
    assert "blockIdx.x * blockDim.x + threadIdx.x" in hip
    assert "blockIdx.y * blockDim.y + threadIdx.y" in hip
    assert "int idx = y * gridDim.x * blockDim.x + x;" in hip
    assert "if (idx >= count) return;" in hip


def test_instruction_list_matches_binary_generator_order():
    m = single_method("Add(first Number, second Number) Number", "\tfirst + second")
    assert [str(i) for i in m.instructions] == [
        "LoadVariableToRegister first R0", "LoadVariableToRegister second R1", "Add R0 R1 R2",
        "Return R2"]


def test_modulo_has_no_operator():
    # GetOperatorSymbol throws NotSupportedException (InstructionsToCuda.cs:101-109)
    m = single_method("Rest(first Number, second Number) Number", "\tfirst % second")
    with pytest.raises(NotImplementedError, match="Modulo"):
        cg.InstructionsToHip().compile(m)


@pytest.mark.parametrize("body,expected", [
    ("(first + second) * third", "(first[idx] + second[idx]) * third[idx]"),
    ("first - (second - third)", "first[idx] - (second[idx] - third[idx])"),
    ("first + (second + third)", "first[idx] + (second[idx] + third[idx])"),
    ("first * second + third", "first[idx] * second[idx] + third[idx]"),
    ("first + second * third", "first[idx] + second[idx] * third[idx]"),
    ("first + second - third", "first[idx] + second[idx] - third[idx]"),
    ("first / (second * third)", "first[idx] / (second[idx] * third[idx])"),
    ("(first - second) / 2", "(first[idx] - second[idx]) / 2"),
])
def test_nested_binaries_keep_their_grouping(body, expected):
    m = single_method("Mix(first Number, second Number, third Number) Number", "\t" + body)
    assert f"output[idx] = {expected};" in cg.InstructionsToHip().compile(m)


@pytest.mark.parametrize("value,text", [
    (5.0, "5"), (0.5, "0.5"), (0.1, "0.1"), (-2.25, "-2.25"), (1e15, "1E+15"), (1e14, "100000000000000"),
    (123456789012345.0, "123456789012345"), (1234567890123456.0, "1.234567890123456E+15"),
    (0.0001, "0.0001"), (0.00001, "1E-05"), (1.5e-7, "1.5E-07"), (1.5e300, "1.5E+300"),
    (1 / 3, "0.3333333333333333"), (0.0, "0"), (-0.0, "-0"), (float("nan"), "NaN"),
    (float("inf"), "Infinity"), (float("-inf"), "-Infinity"), (5e-324, "5E-324"),
    (1.7976931348623157e308, "1.7976931348623157E+308"),
])
def test_constants_print_as_dotnet_invariant(value, text):
    # constant.Number.ToString(CultureInfo.InvariantCulture) (InstructionsToCuda.cs:41-42)
    hip = cg.InstructionsToHip().compile_binary([cg.load_constant(0, value), cg.return_register(0)])
    assert f"output[idx] = {text};" in hip


def test_compile_binary_entry_point_has_only_output_and_count():
    # Compile(BinaryExecutable, Platform) (InstructionsToCuda.cs:14-15)
    hip = cg.InstructionsToHip().compile_binary([cg.load_constant(3, 7.0), cg.return_register(3)])
    assert "void Run(float *output, const int count)" in hip
    assert "output[idx] = 7;" in hip
    assert cg.InstructionsToHip.extension == ".hip"


def test_register_quirks_follow_the_reference():
    I = cg.InstructionType
    gen = cg.InstructionsToHip()
    # a Return of a register never written keeps "0.0f" (cs:31, :52-54)
    assert "output[idx] = 0.0f;" in gen.compile_binary([cg.return_register(5)])
    # a missing operand folds as "0" (cs:47-51)
    hip = gen.compile_binary([cg.load_constant(0, 2.0), cg.binary(I.Add, 0, 9, 1),
                              cg.return_register(1)])
    assert "output[idx] = 2 + 0;" in hip
    # conditional binaries are skipped (cs:46 `!binary.IsConditional()`)
    hip = gen.compile_binary([cg.load_constant(0, 2.0), cg.load_constant(1, 3.0),
                              cg.binary(I.Equal, 0, 1, 0), cg.return_register(0)])
    assert "output[idx] = 2;" in hip
    # a name that is not a scalar parameter is indexed (cs:37-39)
    hip = gen.compile_binary([cg.load_variable(0, "width"), cg.return_register(0)])
    assert "output[idx] = width[idx];" in hip
    # registers wrap after R15 (Registry.cs:18-24)
    body = " + ".join(f"v{i}" for i in range(12))
    m = single_method("Sum(" + ", ".join(f"v{i} Number" for i in range(12)) + ") Number", "\t" + body)
    assert max(max(i.registers) for i in m.instructions) == 15
    assert "output[idx] = " + " + ".join(f"v{i}[idx]" for i in range(12)) + ";" in gen.compile(m)


def test_source_buffer_contract():
    import ctypes
    from strict_amd import _lib
    lib = _lib.load()
    arr, keep = cg._flatten([cg.load_constant(0, 1.0), cg.return_register(0)])
    n = ctypes.c_size_t(0)
    args = (b"Run", None, 0, 1, ctypes.cast(arr, ctypes.c_void_p), 2)
    assert lib.sh_instructions_to_hip(*args, None, 0, ctypes.byref(n)) == _lib.SH_ERR_INVALID_ARGUMENT
    assert n.value > 0 and b"needed" in lib.sh_last_error()
    buf = ctypes.create_string_buffer(n.value)  # one byte short of the NUL
    assert lib.sh_instructions_to_hip(*args, buf, n.value, ctypes.byref(n)) == _lib.SH_ERR_INVALID_ARGUMENT
    buf = ctypes.create_string_buffer(n.value + 1)
    assert lib.sh_instructions_to_hip(*args, buf, n.value + 1, ctypes.byref(n)) == _lib.SH_OK
    assert len(buf.value) == n.value
    assert lib.sh_instructions_to_hip(b"", None, 0, 1, None, 0, buf, 10, ctypes.byref(n)) == \
        _lib.SH_ERR_INVALID_ARGUMENT


# ---- CSharpToCudaTranspiler ---------------------------------------------------

def test_empty_input_will_not_work():
    with pytest.raises(cg.CSharpToHipTranspiler.InvalidCode):
        cg.CSharpToHipTranspiler().convert("")


def test_missing_return_statement(tmp_path):
    with pytest.raises(cg.CSharpType.MissingReturnStatement):
        cg.CSharpToHipTranspiler().parse_csharp(write_input(tmp_path, "MissingReturnStatement"))


def test_parse_add_numbers(tmp_path):
    # CSharpToCudaTranspilerTests.ParseAddNumbers (cs:31-42)
    t = cg.CSharpToHipTranspiler().parse_csharp(write_input(tmp_path, "AddNumbers"))
    assert t.name == "AddNumbers"
    assert len(t.methods) == 1
    m = t.methods[0]
    assert m.name == "Add"
    assert m.parameters[1].type == "Number" and m.return_type == "Number"
    assert m.body_text() == "left + right"


def test_parse_depth_image_expands_to_four_parameters(tmp_path):
    t = cg.CSharpToHipTranspiler().parse_csharp(write_input(tmp_path, "InitializeDepths"))
    m = t.methods[0]
    assert m.name == "Process" and m.return_type is None
    assert [p.name for p in m.parameters] == ["input", "width", "height", "initialDepth"]
    assert m.body_text() == "initialDepth"


def test_non_float_parameter_is_not_supported(tmp_path):
    with pytest.raises(NotImplementedError, match="value"):
        cg.CSharpToHipTranspiler().parse_csharp(write_input(tmp_path, "TakesInts"))


@pytest.mark.parametrize("name", ["AddNumbers", "SubtractNumbers", "MultiplyNumbers",
                                  "InitializeDepths"])
def test_generated_sources_compile_for_gfx950(tmp_path, name):
    # ParseGenerateCudaAndExecute up to CompileKernelAndSaveAsPtxFile (cs:44-53, :100-109)
    tr = cg.CSharpToHipTranspiler()
    t = tr.parse_csharp(write_input(tmp_path, name))
    hip = tr.generate_hip(t)
    with strict_amd.RuntimeCompiler(hip, t.name) as rtc:
        rtc.compile()
        assert len(rtc.get_code()) > 1000  # a gfx950 code object
