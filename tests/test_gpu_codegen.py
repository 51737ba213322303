"""Generated kernels on the GPU: C# input -> Strict method -> HIP source
(sh_instructions_to_hip) -> hipRTC gfx950 code object -> sh_module_load ->
sh_launch, as CSharpToCudaTranspilerTests.ParseGenerateCudaAndExecute does
through ManagedCuda (CSharpToCudaTranspilerTests.cs:44-98), plus the launch
shapes of the reference's Output/*.cu fixtures and large 2-D grids.

Checkers: the reference's known answers (tests/golden), oracle.binary_f32 /
oracle.fill_f32 for the single operations (bit-exact: IEEE float add,
subtract and multiply are correctly rounded on both sides), and numpy
evaluating nested expressions under C's conversions (float op float in
float, a double constant promotes to double). Tolerance: exact (HIP's float
and double division are correctly rounded too), except a * b + c, which
hipRTC may contract into one fused multiply-add: either rounding is accepted
there."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
import strict_amd
from strict_amd import codegen as cg

from test_codegen import write_input

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
OPS = {"Add": oracle.ADD, "Subtract": oracle.SUBTRACT, "Multiply": oracle.MULTIPLY}


def load_generated(ctx, hip, type_name, method_name):
    with strict_amd.RuntimeCompiler(hip, type_name) as rtc:
        rtc.compile()
        return ctx.load_kernel(rtc.get_code(), method_name)


@pytest.mark.parametrize("name,expected", [("AddNumbers", 3), ("SubtractNumbers", -1),
                                           ("MultiplyNumbers", 2), ("InitializeDepths", 5)])
def test_parse_generate_hip_and_execute(ctx, tmp_path, name, expected):
    # ParseGenerateCudaAndExecute (CSharpToCudaTranspilerTests.cs:44-98): count 1,
    # default grid and block of 1
    tr = cg.CSharpToHipTranspiler()
    t = tr.parse_csharp(write_input(tmp_path, name))
    kernel = load_generated(ctx, tr.generate_hip(t), t.name, t.methods[0].name)
    output = ctx.empty(1, np.float32)
    if t.methods[0].name == "Process":
        kernel.run(ctx.upload(np.ones(1, np.float32)), 1, 1, 5.0, output)
    else:
        kernel.run(ctx.upload(np.array([1.0], np.float32)), ctx.upload(np.array([2.0], np.float32)),
                   output, 1)
    assert output.to_host()[0] == expected
    kernel.module.unload()


def test_fixture_launch_shapes(ctx):
    # Output/*.cu: N = 10 blocks of one thread each, every element checked
    gen = cg.InstructionsToHip()
    for case in GOLDEN["binary_f32"]:
        m = cg.Method.parse([f"{case['op']}(first Number, second Number) Number",
                             f"\tfirst {dict(Add='+', Subtract='-', Multiply='*')[case['op']]} second"])
        k = load_generated(ctx, gen.compile(m), case["op"] + "Numbers", case["op"])
        n = case["count"]
        out = ctx.upload(np.full(n + 4, np.nan, np.float32))
        k.grid_dimensions = n
        k.block_dimensions = 1
        k.run(ctx.upload(np.full(n, case["first"], np.float32)),
              ctx.upload(np.full(n, case["second"], np.float32)), out, n)
        host = out.to_host()
        assert np.all(host[:n] == case["expected"]), case
        assert np.all(np.isnan(host[n:]))  # nothing past count
        k.module.unload()
    for case in GOLDEN["initialize_depths"]:
        m = cg.Method.parse(["Process(input Number, width Number, height Number, initialDepth Number)",
                             "\tinitialDepth"])
        k = load_generated(ctx, gen.compile(m), "InitializeDepths", "Process")
        n = case["count"]
        out = ctx.upload(np.full(n, np.nan, np.float32))
        k.grid_dimensions = (n, 1, 1)
        k.run(ctx.upload(np.ones(n, np.float32)), n, 1, float(case["initial_depth"]), out)
        assert np.all(out.to_host() == case["expected"]), case
        k.module.unload()


@pytest.mark.parametrize("op", ["Add", "Subtract", "Multiply"])
def test_binary_kernels_on_a_2d_grid_match_the_oracle(ctx, op):
    # 2^20 + 3 elements over a 64-wide 2-D grid: every element is written once,
    # which the reference's `y * blockDim.x + x` index would not do
    n = (1 << 20) + 3
    rng = np.random.default_rng(7)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    sym = {"Add": "+", "Subtract": "-", "Multiply": "*"}[op]
    m = cg.Method.parse([f"{op}(first Number, second Number) Number", f"\tfirst {sym} second"])
    k = load_generated(ctx, cg.InstructionsToHip().compile(m), op, op)
    out = ctx.upload(np.full(n + 64, np.nan, np.float32))
    k.block_dimensions = 256
    k.grid_dimensions = (64, -(-n // (64 * 256)), 1)
    k.run(ctx.upload(a), ctx.upload(b), out, n)
    host = out.to_host()
    assert np.array_equal(host[:n], oracle.binary_f32(OPS[op], a, b))
    assert np.all(np.isnan(host[n:]))
    k.module.unload()


def test_process_kernel_fills_width_by_height(ctx):
    w, h = 37, 19
    m = cg.Method.parse(["Process(input Number, width Number, height Number, initialDepth Number)",
                         "\tinitialDepth"])
    k = load_generated(ctx, cg.InstructionsToHip().compile(m), "InitializeDepths", "Process")
    out = ctx.upload(np.full(w * h + 64, np.nan, np.float32))
    k.block_dimensions = (8, 8, 1)
    k.grid_dimensions = (-(-w // 8), -(-h // 8), 1)
    k.run(ctx.upload(np.ones(w * h, np.float32)), w, h, 0.75, out)
    host = out.to_host()
    assert np.array_equal(host[:w * h], oracle.fill_f32(0.75, w * h))
    assert np.all(np.isnan(host[w * h:]))
    k.module.unload()


def _c_eval(node, env):
    """numpy value of an expression tree under C's usual conversions."""
    kind = node[0]
    if kind == "name":
        return env[node[1]]
    if kind == "number":
        v = node[1]
        return np.int32(v) if float(v).is_integer() else np.float64(v)
    op, l, r = node
    a, b = _c_eval(l, env), _c_eval(r, env)
    wide = np.float64 if (np.asarray(a).dtype == np.float64 or np.asarray(b).dtype == np.float64) \
        else np.float32
    a, b = np.asarray(a).astype(wide), np.asarray(b).astype(wide)
    return {"+": np.add, "-": np.subtract, "*": np.multiply, "/": np.divide}[op](a, b)


def _ulp_diff(x, y):
    xi = x.view(np.int32).astype(np.int64)
    yi = y.view(np.int32).astype(np.int64)
    xi = np.where(xi < 0, -(xi & 0x7FFFFFFF), xi)
    yi = np.where(yi < 0, -(yi & 0x7FFFFFFF), yi)
    return np.abs(xi - yi)


@pytest.mark.parametrize("body,max_ulp", [
    ("(first + second) * third", 0),
    ("first - (second - third)", 0),
    ("first + (second + third)", 0),
    ("(first - second) / 2.5 + 2", 0),
    ("first / second", 0),
    ("first * second + third", None),  # contracted or not
])
def test_nested_expressions_match_c_semantics(ctx, body, max_ulp):
    n = 100_003
    rng = np.random.default_rng(11)
    env = {k: rng.uniform(-4, 4, n).astype(np.float32) for k in ("first", "second", "third")}
    env["second"][np.abs(env["second"]) < 1e-3] = 0.5
    m = cg.Method.parse(["Mix(first Number, second Number, third Number) Number", "\t" + body])
    k = load_generated(ctx, cg.InstructionsToHip().compile(m), "Mix", "Mix")
    out = ctx.empty(n, np.float32)
    k.block_dimensions = 256
    k.grid_dimensions = -(-n // 256)
    k.run(ctx.upload(env["first"]), ctx.upload(env["second"]), ctx.upload(env["third"]), out, n)
    got = out.to_host()
    tree = cg._parse_expression(body)
    want = np.asarray(_c_eval(tree, env)).astype(np.float32)
    if max_ulp is None:
        a, b, c = (env[k].astype(np.float64) for k in ("first", "second", "third"))
        fused = (a * b + c).astype(np.float32)  # a*b is exact in double
        assert np.all((got == want) | (got == fused))
    else:
        d = _ulp_diff(got, want)
        print(f"[codegen] {body}: max ulp {int(d.max())}")
        assert d.max() <= max_ulp
    k.module.unload()


@pytest.mark.parametrize("count", [1, 1000, 1 << 20])
def test_compile_binary_entry_point_runs(ctx, count):
    # Compile(BinaryExecutable, Platform) (InstructionsToCuda.cs:14-15): the
    # entry point with no parameters plus `count`, launched over count
    # elements with a partial last block; every element holds the entry
    # point's value (2.5 * 4 - 1.25 = 8.75, exact in float)
    I = cg.InstructionType
    hip = cg.InstructionsToHip().compile_binary([
        cg.load_constant(0, 2.5), cg.load_constant(1, 4.0), cg.binary(I.Multiply, 0, 1, 2),
        cg.load_constant(3, 1.25), cg.binary(I.Subtract, 2, 3, 4), cg.return_register(4)])
    kernel = load_generated(ctx, hip, "Run", cg.InstructionsToHip.run_method)
    sentinel = np.full(count + 64, -7.0, np.float32)
    out = ctx.upload(sentinel)
    kernel.grid_dimensions = ((count + 255) // 256, 1, 1)
    kernel.block_dimensions = (256, 1, 1)
    kernel.run(out, count)
    got = out.to_host()
    assert np.all(got[:count] == np.float32(8.75))
    assert np.all(got[count:] == np.float32(-7.0))  # the bounds check held
    out.free()
    kernel.module.unload()
