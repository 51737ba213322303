"""A .strictbinary's constants as kernel inputs on the GPU: load the file
(sh_strictbinary_load), upload its List(Number) constants to device buffers
(sh_strictbinary_upload_f32), generate the kernel of one of its methods from
the loaded instructions (sh_instructions_to_hip), compile it with hipRTC and
run it. Bar: bit-exact against numpy's float32 arithmetic on the same
constants (IEEE float add and multiply are correctly rounded on both sides,
and the double -> float conversion rounds to nearest even on both)."""
import numpy as np
import pytest

import oracle.strictbinary as osb
import strict_amd
from strict_amd import codegen as cg
from strict_amd import strictbinary as sb

pytestmark = pytest.mark.gpu

R0, R1, R2 = 0, 1, 2


def vectors_binary(first, second):
    run = [osb.Instr(osb.STORE_CONSTANT, value=osb.number_list(first), name="first"),
           osb.Instr(osb.STORE_CONSTANT, value=osb.number_list(second), name="second"),
           osb.Instr(osb.RETURN, (R0,))]
    methods = {"Run": [osb.Method([], "None", run)]}
    for name, op in [("Add", osb.ADD), ("Multiply", osb.MULTIPLY)]:
        methods[name] = [osb.Method([osb.Member("first", "Number"), osb.Member("second", "Number")],
                                    "Number", [osb.Instr(osb.LOAD_VARIABLE, (R0,), name="first"),
                                               osb.Instr(osb.LOAD_VARIABLE, (R1,), name="second"),
                                               osb.Instr(op, (R0, R1, R2)), osb.Instr(osb.RETURN, (R2,))])]
    members = [osb.Member("scale", "List(Number)",
                          osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number_list([0.5, 3.0, -2.0])))]
    data = osb.write_strictbinary([osb.TypeEntry("Strict/Vectors", members, methods)])
    return sb.BinaryExecutable(data=data)


@pytest.mark.parametrize("op", ["Add", "Multiply"])
def test_list_constants_feed_a_generated_kernel(ctx, op):
    n = 4099  # a partial last block
    rng = np.random.default_rng(17)
    first = rng.normal(0, 100, n)
    second = np.concatenate([rng.integers(-300, 300, n - 3), [0.1, 1e10, 255]]).astype(np.float64)
    b = vectors_binary(first, second)
    print(f"[strictbinary] {op} n={n}", flush=True)
    consts = {c.identifier: c for c in b.constants() if c.identifier}
    assert consts["first"].count == n and consts["second"].count == n
    bufs = {name: ctx.empty(n, np.float32) for name in ("first", "second")}
    for name, buf in bufs.items():
        b.upload_f32(ctx, consts[name], buf)
    method = b.find_method("Strict/Vectors", op, 2, "Number")
    src = cg.InstructionsToHip().compile(method.as_codegen_method())
    with strict_amd.RuntimeCompiler(src, "Vectors") as rtc:
        rtc.compile()
        kernel = ctx.load_kernel(rtc.get_code(), op)
    out = ctx.upload(np.full(n + 8, np.nan, np.float32))
    kernel.block_dimensions = 256
    kernel.grid_dimensions = (n + 255) // 256
    kernel.run(bufs["first"], bufs["second"], out, n)
    got = out.to_host()
    f32 = (first.astype(np.float32), second.astype(np.float32))
    want = f32[0] + f32[1] if op == "Add" else f32[0] * f32[1]
    assert np.array_equal(got[:n], want)
    assert np.all(np.isnan(got[n:]))  # nothing past count
    assert np.array_equal(bufs["first"].to_host(), f32[0])
    kernel.module.unload()
    for buf in list(bufs.values()) + [out]:
        buf.free()


def test_member_constant_upload_and_capacity_check(ctx):
    b = vectors_binary([1.0], [2.0])
    (scale,) = b.constants(type_full_name="Strict/Vectors")
    buf = ctx.upload(np.full(4, 7.0, np.float32))
    b.upload_f32(ctx, scale, buf, type_full_name="Strict/Vectors")
    assert buf.to_host().tolist() == [0.5, 3.0, -2.0, 7.0]
    small = buf.view(0, 8, np.float32)  # room for two of the three numbers
    with pytest.raises(strict_amd.StrictHipError, match="capacity"):
        b.upload_f32(ctx, scale, small, type_full_name="Strict/Vectors")
    buf.free()
