"""The MLIR backend's GPU path retargeted to ROCDL (strict_amd.mlir), string level.

The reference pins its MLIR emitter only at string level
(Strict.Compiler.Assembly.Tests/InstructionsToMlirTests.cs:670-938); those
cases are mirrored here, with the NVVM / CUDA expectations of its pipeline
tests (:956-966 and MlirLinker.cs:60-76) replaced by their ROCDL / HIP
counterparts. The image has no mlir-opt, so nothing is lowered or run; a
structural check (every SSA value defined before its use, regions balanced)
covers what a parser would reject first.
"""
import re
import zipfile

import pytest

import oracle.strictbinary as osb
from strict_amd import _lib, codegen as cg, mlir
from strict_amd import strictbinary as sb

I = cg.InstructionType
R0, R1, R2, R3, R4 = range(5)


def loop_program(end, body_count, body=None):
    """R0 = 0, R1 = end, R2 = 1, R3 = 2; a range loop R0..R1 over body_count
    copies of `body` (default: R4 = R2 + R3); return R2."""
    body = body or cg.binary(I.Add, R2, R3, R4)
    ins = [cg.load_constant(R0, 0.0), cg.load_constant(R1, end), cg.load_constant(R2, 1.0),
           cg.load_constant(R3, 2.0), cg.Instruction(I.LoopBegin, (R0, R1))]
    ins += [body] * body_count
    ins += [cg.Instruction(I.LoopEnd, (), number=body_count), cg.return_register(R2)]
    return ins


REGION_ARGS = {"%bx", "%by", "%bz", "%tx", "%ty", "%tz", "%grid_x", "%grid_y", "%grid_z",
               "%block_x", "%block_y", "%block_z"}


def assert_well_formed(text):
    """Braces balance; every %value is defined (left of `=`, a region or
    function argument, or a loop induction variable) before it is used."""
    assert text.count("{") == text.count("}")
    defined = set(REGION_ARGS)
    for line in text.splitlines():
        line = line.strip()
        defined |= set(re.findall(r"(%param\d+):", line))
        m = re.match(r"((?:%[\w.]+\s*,\s*)*%[\w.]+)\s*=\s*(.*)", line)
        rhs = line
        if m:
            rhs = m.group(2)
        for iv in re.findall(r"scf\.for (%\w+) =|scf\.parallel \((%\w+)\)", line):
            defined |= {v for v in iv if v}
            rhs = rhs.split("=", 1)[1]
        used = set(re.findall(r"%[\w.]+", rhs)) - REGION_ARGS
        missing = used - defined
        assert not missing, (missing, line)
        if m:
            defined |= set(re.findall(r"%[\w.]+", m.group(1)))


def compile_fn(name, ins):
    text = mlir.InstructionsToMlir().compile_instructions(name, ins)
    assert_well_formed(text)
    return text


def test_high_complexity_loop_emits_gpu_launch():
    # HighComplexityLoopEmitsGpuLaunch (:709-732): 921,600 iterations x 20
    # body instructions = 18.4 M > 10 M
    text = compile_fn("GpuLaunchTest", loop_program(921600.0, 20))
    assert "gpu.launch blocks" in text


def test_gpu_launch_uses_block_times_block_size_plus_thread():
    # GpuLaunchUsesCorrectGlobalIdComputation (:734-757): 8,294,400 x 30
    text = compile_fn("GpuGridTest", loop_program(8294400.0, 30))
    assert "arith.muli %bx, %block_x : index" in text
    gid = re.search(r"(%\w+) = arith\.addi (%\w+), %tx : index", text)
    assert gid, "global id = blockIdx * blockDim + threadIdx"
    assert re.search(rf"{gid.group(2)} = arith\.muli %bx, %block_x", text)


def test_gpu_launch_has_bounds_check_and_terminator():
    # GpuLaunchHasBoundsCheckAndTerminator (:759-784)
    text = compile_fn("GpuBoundsTest", loop_program(8294400.0, 30))
    n = re.search(r"(%\w+) = arith\.subi", text).group(1)
    assert re.search(rf"arith\.cmpi ult, %\w+, {n} : index", text)
    assert "scf.if" in text and "gpu.terminator" in text
    assert f"%block_x = %bs" in text and "arith.constant 256 : index" in text


def test_gpu_launch_includes_memory_management():
    # GpuLaunchIncludesMemoryManagement (:786-819), plus what the build adds:
    # the device buffer receives each iteration's value and comes back to the host
    text = compile_fn("GpuMemoryTest", loop_program(8294400.0, 30))
    for op in ("memref.alloc", "gpu.alloc async", "gpu.memcpy async", "gpu.dealloc async",
               "memref.dealloc"):
        assert op in text, op
    dev = re.search(r"(%dev\d+), %\w+ = gpu\.alloc", text).group(1)
    host = re.search(r"(%host\d+) = memref\.alloc", text).group(1)
    assert re.search(rf"memref\.store %v\d+, {dev}\[%gid\d+\]", text)
    launch, after = text.index("gpu.launch"), text.index("gpu.terminator")
    assert text.index(f"gpu.memcpy async [%t", after) > after  # results copied back after the launch
    assert re.search(rf"gpu\.memcpy async \[%t\d+\] {host}, {dev}", text[after:])
    assert re.search(rf"gpu\.memcpy async \[%t\d+\] {dev}, {host}", text[:launch])


def test_gpu_launch_uses_region_arguments():
    # GpuLaunchUsesProperRegionArguments (:821-848)
    text = compile_fn("GpuRegionTest", loop_program(8294400.0, 30))
    assert "blocks(%bx, %by, %bz) in (%grid_x =" in text
    assert "threads(%tx, %ty, %tz) in (%block_x =" in text
    assert "gpu.block_id" not in text and "gpu.thread_id" not in text


def test_medium_complexity_stays_scf_parallel():
    # MediumComplexityStaysScfParallelNotGpu (:850-873): 100 K x 2 = 200 K
    text = compile_fn("MediumComplexityTest", loop_program(100000.0, 2))
    assert "scf.parallel" in text and "gpu.launch" not in text


def test_parallel_above_the_cpu_threshold():
    # 10 K iterations x 20 body instructions = 200 K > 100 K (:650-673)
    text = compile_fn("ParallelTest", loop_program(10000.0, 20))
    assert "scf.parallel" in text and "scf.for" not in text


def test_simple_body_below_threshold_stays_sequential():
    # SimpleBodyWithManyIterationsDoesNotParallelize... (:675-695): 50 K x 1
    ins = [cg.load_constant(R0, 0.0), cg.load_constant(R1, 50000.0),
           cg.Instruction(I.LoopBegin, (R0, R1)), cg.load_constant(R2, 1.0),
           cg.Instruction(I.LoopEnd, (), number=1), cg.return_register(R2)]
    text = compile_fn("SimpleBodyTest", ins)
    assert "scf.for" in text and "scf.parallel" not in text


def test_thresholds_are_the_dispatch_hooks():
    # GpuThresholdConstantIsExposed (:875-884); the same rule as
    # sh_range_loop_target, which the VM's dispatch hook uses
    assert mlir.GPU_COMPLEXITY_THRESHOLD == 10_000_000
    assert mlir.PARALLEL_COMPLEXITY_THRESHOLD == 100_000
    header = (_lib.LIB_PATH.parent.parent / "include" / "strict_hip.h").read_text()
    assert "SH_GPU_COMPLEXITY_THRESHOLD 10000000LL" in header
    assert "SH_PARALLEL_COMPLEXITY_THRESHOLD 100000LL" in header
    assert mlir.loop_target(921600, 20) == 2
    assert mlir.loop_target(100000, 2) == 1
    assert mlir.loop_target(50000, 1) == 0
    assert mlir.loop_target(10_000_000, 1) == 1  # not above the GPU threshold


def test_mlir_opt_arguments_target_rocdl_gfx950():
    # MlirOptArgsIncludeGpuPasses (:886-899), the NVVM passes replaced
    args = mlir.mlir_opt_args_with_gpu("in.mlir", "out.mlir")
    for p in ("--gpu-kernel-outlining", '--rocdl-attach-target="chip=gfx950"',
              "--convert-gpu-to-rocdl", "--gpu-module-to-binary", "--gpu-to-llvm",
              "--convert-memref-to-llvm", "--reconcile-unrealized-casts"):
        assert p in args, p
    assert "nvvm" not in args
    # outlining before the target is attached, the target before serializing
    assert (args.index("--gpu-kernel-outlining") < args.index("--rocdl-attach-target")
            < args.index("--convert-gpu-to-rocdl") < args.index("--gpu-module-to-binary")
            < args.index("--gpu-to-llvm"))
    cpu = mlir.mlir_opt_args("in.mlir", "out.mlir")
    assert "gpu" not in cpu and "--convert-func-to-llvm" in cpu


def test_gpu_link_line_uses_hip():
    args = mlir.gpu_link_args("a.ll", "a.out")
    assert "-lamdhip64" in args and "-lmlir_rocm_runtime" in args
    assert "cuda" not in args


def test_gpu_module_has_container_attribute():
    # GpuCompileForPlatformAddsContainerModuleAttribute (:901-923)
    text = mlir.InstructionsToMlir().compile_module("Run", loop_program(921600.0, 20))
    assert text.startswith("module attributes {gpu.container_module} {")
    assert "func.func @main() -> i32" in text and "func.call @Run()" in text
    assert_well_formed(text)


def test_cpu_module_is_plain():
    # NonGpuCompileForPlatformHasPlainModule (:925-938)
    text = mlir.InstructionsToMlir().compile_module("Run", [cg.load_constant(R0, 5.0),
                                                            cg.return_register(R0)])
    assert text.startswith("module {") and "gpu.container_module" not in text
    assert "%c1 = arith.constant 5.0 : f64" in text and "return %c1 : f64" in text
    assert_well_formed(text)


def test_arithmetic_and_parameters():
    ins = [cg.load_variable(R0, "first"), cg.load_variable(R1, "second"),
           cg.binary(I.Multiply, R0, R1, R2), cg.load_constant(R3, 0.5),
           cg.binary(I.Subtract, R2, R3, R4), cg.return_register(R4)]
    text = mlir.InstructionsToMlir().compile_instructions("Scale", ins, ["first", "second"])
    assert "func.func @Scale(%param0: f64, %param1: f64) -> f64" in text
    assert re.search(r"(%v\d+) = arith\.mulf %param0, %param1 : f64", text)
    assert re.search(r"= arith\.subf %v\d+, %c\d+ : f64", text)
    assert_well_formed(text)


def test_loop_body_reads_the_iteration_index():
    # a body reading the loop's index computes from start + global id
    body = cg.Instruction(I.LoadVariableToRegister, (R2,), identifier="index")
    ins = [cg.load_constant(R0, 0.0), cg.load_constant(R1, 4_000_000.0),
           cg.load_constant(R3, 2.0), cg.Instruction(I.LoopBegin, (R0, R1)), body]
    ins += [cg.binary(I.Multiply, R2, R3, R4)] * 3
    ins += [cg.Instruction(I.LoopEnd, (), number=4), cg.return_register(R3)]
    text = compile_fn("Indexed", ins)
    assert "gpu.launch" in text  # 4 M x 4 = 16 M
    it = re.search(r"(%it\d+) = arith\.addi (%lo\d+), (%gid\d+) : index", text)
    x = re.search(rf"(%i\d+) = arith\.index_cast {it.group(1)}", text)
    assert re.search(rf"= arith\.sitofp {x.group(1)} : i64 to f64", text)


def test_nested_loop_in_a_launch_is_a_thread_loop():
    inner = [cg.load_constant(5, 0.0), cg.load_constant(6, 8.0), cg.Instruction(I.LoopBegin, (5, 6)),
             cg.binary(I.Add, R2, R3, R4), cg.Instruction(I.LoopEnd, (), number=1)]
    ins = [cg.load_constant(R0, 0.0), cg.load_constant(R1, 2_000_000.0),
           cg.load_constant(R2, 1.0), cg.load_constant(R3, 2.0),
           cg.Instruction(I.LoopBegin, (R0, R1))] + inner * 2
    ins += [cg.Instruction(I.LoopEnd, (), number=len(inner) * 2), cg.return_register(R2)]
    text = compile_fn("Nested", ins)  # 2 M x 10 = 20 M
    assert text.count("gpu.launch") == 1 and text.count("scf.for") == 2
    assert text.index("scf.for") > text.index("gpu.launch")


def test_unsupported_instruction_is_rejected():
    # InstructionsToMlir.cs:163-168 throws NotSupportedException
    with pytest.raises(NotImplementedError):
        mlir.InstructionsToMlir().compile_instructions(
            "Bad", [cg.Instruction(I.Invoke, (R0,)), cg.return_register(R0)])


def test_compile_a_loaded_binarys_entry_point():
    # Compile(BinaryExecutable, Platform) (InstructionsToMlir.cs:14-20): the
    # entry point of a .strictbinary whose Run holds a range loop
    run = [osb.Instr(osb.LOAD_CONSTANT, (R0,), value=osb.number(0)),
           osb.Instr(osb.LOAD_CONSTANT, (R1,), value=osb.number(921600)),
           osb.Instr(osb.LOAD_CONSTANT, (R2,), value=osb.number(1)),
           osb.Instr(osb.LOAD_CONSTANT, (R3,), value=osb.number(2)),
           osb.Instr(osb.LOOP_BEGIN, (R0, R1), has_end=True)]
    run += [osb.Instr(osb.ADD, (R2, R3, R4))] * 20
    run += [osb.Instr(osb.LOOP_END, number=20), osb.Instr(osb.RETURN, (R2,))]
    entry = osb.TypeEntry("Strict/Loops", [], {"Run": [osb.Method([], "None", run)]})
    binary = sb.BinaryExecutable(data=osb.write_strictbinary([entry], zipfile.ZIP_DEFLATED))
    ins = binary.entry_point.instructions
    assert [i.type for i in ins[4:5]] == [I.LoopBegin] and ins[4].registers[:2] == (R0, R1)
    text = mlir.InstructionsToMlir().compile_module("Run", ins)
    assert "gpu.launch blocks" in text and text.startswith("module attributes {gpu.container_module}")
    assert_well_formed(text)


def test_the_structure_check_catches_planted_mistakes():
    good = mlir.InstructionsToMlir().compile_instructions("G", loop_program(921600.0, 20))
    assert_well_formed(good)
    # a value used before its definition, and an unbalanced region
    swapped = good.replace("%gid", "%gidX", 1)
    with pytest.raises(AssertionError):
        assert_well_formed(swapped)
    with pytest.raises(AssertionError):
        assert_well_formed(good.replace("gpu.terminator\n    }", "gpu.terminator", 1))
