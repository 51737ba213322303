"""Strict bytecode -> MLIR text whose heavy range loops run on the GPU through
`gpu.launch`, lowered for ROCm / gfx950.

The reference's MLIR backend (Strict.Compiler.Assembly/InstructionsToMlir.cs)
emits arith / func / scf / cf text and picks, per range loop, a serial
`scf.for`, a CPU-parallel `scf.parallel` or a `gpu.launch` by complexity =
iterations x body instructions (:397-418); MlirLinker.cs:60-76 then lowers GPU
modules through NVVM and links against the CUDA driver. This module keeps the
emission rule and the launch shape and retargets the lowering: the pass
pipeline attaches a `#rocdl.target<chip = "gfx950">` to the outlined
`gpu.module`, converts it with `convert-gpu-to-rocdl`, serializes it to a
gfx950 code object (`gpu-module-to-binary`) and links the host side against
`amdhip64` through MLIR's ROCm runtime wrappers. The loop thresholds are the
ones libstrict_hip's `sh_range_loop_target` applies (include/strict_hip.h), so
the VM's dispatch hook and this backend agree on which loops go to the GPU.

Differences from the reference's text, on purpose:
  - the launch's device buffer is used: every thread stores the loop body's
    last value at its iteration's index, the results are copied back to the
    host buffer after the launch, and both buffers are freed; the reference
    copies host -> device and never reads or writes either buffer;
  - allocation, copies and frees are ordered with async tokens
    (`gpu.wait async`, `gpu.alloc async [...]`), the form `gpu-to-llvm` lowers
    to HIP stream calls;
  - iterations are end - start when both bounds are constants (the reference
    counts the end alone);
  - a loop inside a launched loop stays a `scf.for` inside the kernel.

The image has no `mlir-opt` / `mlir-translate`, so this is text generation
only; tests/test_mlir.py pins it with the reference's own string tests
(InstructionsToMlirTests.cs:709-938, adapted to ROCDL) and a structural check
that every SSA value is defined before its use.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

from . import _lib
from .codegen import Instruction, InstructionType

__all__ = ["InstructionsToMlir", "GPU_COMPLEXITY_THRESHOLD", "PARALLEL_COMPLEXITY_THRESHOLD",
           "BLOCK_SIZE", "ROCM_CHIP", "mlir_opt_args", "mlir_opt_args_with_gpu", "gpu_link_args"]

# include/strict_hip.h: SH_GPU_COMPLEXITY_THRESHOLD / SH_PARALLEL_COMPLEXITY_THRESHOLD
# (InstructionsToMlir.cs:414, :418)
GPU_COMPLEXITY_THRESHOLD = 10_000_000
PARALLEL_COMPLEXITY_THRESHOLD = 100_000
BLOCK_SIZE = 256  # threads per workgroup: four 64-lane waves, one per SIMD of a CU
ROCM_CHIP = "gfx950"

_SERIAL, _PARALLEL, _GPU = 0, 1, 2
_ARITH = {InstructionType.Add: "arith.addf", InstructionType.Subtract: "arith.subf",
          InstructionType.Multiply: "arith.mulf", InstructionType.Divide: "arith.divf",
          InstructionType.Modulo: "arith.remf"}
_COMPARE = {InstructionType.Equal: "oeq", InstructionType.NotEqual: "one",
            InstructionType.LessThan: "olt", InstructionType.GreaterThan: "ogt"}


def _number(v: float) -> str:
    """An f64 literal MLIR accepts: always a decimal point or an exponent."""
    text = repr(float(v))
    return text if any(c in text for c in ".eEn") else text + ".0"


def loop_target(iterations: int, body_instructions: int) -> int:
    """sh_range_loop_target: 0 serial, 1 CPU-parallel, 2 GPU."""
    return int(_lib.load().sh_range_loop_target(ctypes.c_longlong(max(iterations, 0)),
                                                ctypes.c_int(max(body_instructions, 0))))


@dataclass
class _Loop:
    kind: int                    # _SERIAL / _PARALLEL / _GPU
    index_f64: str               # the iteration's value as f64 (start + index)
    last: Optional[str] = None   # the body's last computed value
    host: Optional[str] = None   # a launch's host and device result buffers
    device: Optional[str] = None
    gid: Optional[str] = None    # a launch's thread index within the loop


@dataclass
class _Function:
    name: str
    params: Sequence[str]
    lines: List[str] = field(default_factory=list)
    regs: Dict[int, str] = field(default_factory=dict)
    consts: Dict[int, float] = field(default_factory=dict)
    variables: Dict[str, str] = field(default_factory=dict)
    loops: List[_Loop] = field(default_factory=list)
    counter: int = 0
    indent: int = 2
    uses_gpu: bool = False
    text: str = ""

    def temp(self, hint: str = "v") -> str:
        self.counter += 1
        return f"%{hint}{self.counter}"

    def emit(self, text: str) -> None:
        self.lines.append("  " * self.indent + text)

    def open(self, text: str) -> None:
        self.emit(text)
        self.indent += 1

    def close(self, text: str = "}") -> None:
        self.indent -= 1
        self.emit(text)

    def value(self, register: int) -> str:
        """The SSA value a register holds (0.0 for one never written)."""
        if register not in self.regs:
            t = self.temp("zero")
            self.emit(f"{t} = arith.constant 0.0 : f64")
            self.regs[register] = t
        return self.regs[register]

    def as_f64(self, index: str) -> str:
        i64, f = self.temp("i"), self.temp("x")
        self.emit(f"{i64} = arith.index_cast {index} : index to i64")
        self.emit(f"{f} = arith.sitofp {i64} : i64 to f64")
        return f


class InstructionsToMlir:
    """Bytecode instructions -> an MLIR `func.func` (compile_instructions) or a
    whole module with a `main` that calls it (compile_module)."""

    extension = ".mlir"

    def compile_instructions(self, method_name: str, instructions: Sequence[Instruction],
                             parameters: Sequence[str] = ()) -> str:
        return self._function(method_name, list(instructions), parameters).text

    def compile_module(self, method_name: str, instructions: Sequence[Instruction],
                       parameters: Sequence[str] = ()) -> str:
        """The function plus `main` (exit code 0) calling it with zeros; the
        module carries `gpu.container_module` when a loop was launched."""
        fn = self._function(method_name, list(instructions), parameters)
        head = "module attributes {gpu.container_module} {" if fn.uses_gpu else "module {"
        zero = "    %arg0 = arith.constant 0.0 : f64\n" if parameters else ""
        args = ", ".join("%arg0" for _ in parameters)
        types = ", ".join("f64" for _ in parameters)
        main = ("  func.func @main() -> i32 {\n" + zero +
                f"    %result = func.call @{method_name}({args}) : ({types}) -> f64\n"
                "    %exit = arith.constant 0 : i32\n"
                "    return %exit : i32\n"
                "  }")
        return f"{head}\n{fn.text}\n{main}\n}}\n"

    # ---- one function ---------------------------------------------------------

    def _function(self, name: str, instructions: List[Instruction], parameters) -> _Function:
        fn = _Function(name, list(parameters))
        for i, p in enumerate(parameters):
            fn.variables[p] = f"%param{i}"
        signature = ", ".join(f"%param{i}: f64" for i in range(len(parameters)))
        returned = False
        for i, ins in enumerate(instructions):
            returned |= self._instruction(fn, instructions, i, ins)
        if fn.loops:
            raise ValueError(f"{name}: LoopBegin without its LoopEnd")
        if not returned:
            fn.emit(f"return {fn.value(-1)} : f64")
        fn.text = "\n".join([f"  func.func @{name}({signature}) -> f64 {{"] + fn.lines + ["  }"])
        return fn

    def _instruction(self, fn: _Function, instructions, index: int, ins: Instruction) -> bool:
        t = ins.type
        if t == InstructionType.LoadConstantToRegister:
            v = fn.temp("c")
            fn.emit(f"{v} = arith.constant {_number(ins.number)} : f64")
            fn.regs[ins.registers[0]] = v
            fn.consts[ins.registers[0]] = float(ins.number)
        elif t == InstructionType.LoadVariableToRegister:
            if ins.identifier not in fn.variables:
                raise NotImplementedError(f"variable {ins.identifier} is not known to the MLIR backend")
            fn.regs[ins.registers[0]] = fn.variables[ins.identifier]
            fn.consts.pop(ins.registers[0], None)
        elif t in _ARITH:
            left, right = fn.value(ins.registers[0]), fn.value(ins.registers[1])
            v = fn.temp()
            fn.emit(f"{v} = {_ARITH[t]} {left}, {right} : f64")
            out = ins.registers[2] if len(ins.registers) > 2 else ins.registers[0]
            fn.regs[out] = v
            fn.consts.pop(out, None)
            if fn.loops:
                fn.loops[-1].last = v
        elif t in _COMPARE:
            left, right = fn.value(ins.registers[0]), fn.value(ins.registers[1])
            fn.emit(f"{fn.temp('cmp')} = arith.cmpf {_COMPARE[t]}, {left}, {right} : f64")
        elif t == InstructionType.LoopBegin:
            self._loop_begin(fn, instructions, index, ins)
        elif t == InstructionType.LoopEnd:
            self._loop_end(fn)
        elif t == InstructionType.Return:
            if fn.loops:
                raise NotImplementedError("Return inside a loop body")
            fn.emit(f"return {fn.value(ins.registers[0])} : f64")
            return True
        else:
            # InstructionsToMlir.cs:163-168: anything else is not supported
            raise NotImplementedError(f"MLIR compilation does not support instruction {t!r}")
        return False

    # ---- range loops ------------------------------------------------------------

    @staticmethod
    def _body_count(instructions, index: int) -> int:
        """Instructions between a LoopBegin and its own LoopEnd (nested loops counted)."""
        depth = 0
        for k in range(index + 1, len(instructions)):
            t = instructions[k].type
            if t == InstructionType.LoopBegin:
                depth += 1
            elif t == InstructionType.LoopEnd:
                if depth == 0:
                    return k - index - 1
                depth -= 1
        raise ValueError("LoopBegin without its LoopEnd")

    def _loop_begin(self, fn: _Function, instructions, index: int, ins: Instruction) -> None:
        if len(ins.registers) < 2:
            raise NotImplementedError("only range loops (LoopBegin with an end register)")
        start_reg, end_reg = ins.registers[0], ins.registers[1]
        start, end = fn.value(start_reg), fn.value(end_reg)
        iterations = 0
        if start_reg in fn.consts and end_reg in fn.consts:
            iterations = int(fn.consts[end_reg] - fn.consts[start_reg])
        kind = loop_target(iterations, max(self._body_count(instructions, index), 1))
        if any(l.kind == _GPU for l in fn.loops):
            kind = _SERIAL  # no launch inside a launch: a plain loop of the thread
        lo, hi, one = fn.temp("lo"), fn.temp("hi"), fn.temp("one")
        fn.emit(f"{lo} = arith.fptosi {start} : f64 to index")
        fn.emit(f"{hi} = arith.fptosi {end} : f64 to index")
        fn.emit(f"{one} = arith.constant 1 : index")
        if kind == _GPU:
            loop = self._gpu_launch(fn, lo, hi, one)
        else:
            iv = fn.temp("iv")
            if kind == _PARALLEL:
                fn.open(f"scf.parallel ({iv}) = ({lo}) to ({hi}) step ({one}) {{")
            else:
                fn.open(f"scf.for {iv} = {lo} to {hi} step {one} {{")
            loop = _Loop(kind, fn.as_f64(iv))
        fn.loops.append(loop)
        for name in ("index", "value"):  # the names a Strict range loop's body reads
            fn.variables[name] = loop.index_f64

    @staticmethod
    def _gpu_launch(fn: _Function, lo: str, hi: str, one: str) -> _Loop:
        """gpu.launch over [lo, hi): BLOCK_SIZE threads per block, global id
        blockIdx * blockDim + threadIdx, bounds check against the count; host
        and device result buffers around it."""
        fn.uses_gpu = True
        n, host, dev = fn.temp("n"), fn.temp("host"), fn.temp("dev")
        t0, t1, t2 = fn.temp("t"), fn.temp("t"), fn.temp("t")
        bs, grid = fn.temp("bs"), fn.temp("grid")
        fn.emit(f"{n} = arith.subi {hi}, {lo} : index")
        fn.emit(f"{host} = memref.alloc({n}) : memref<?xf64>")
        fn.emit(f"{t0} = gpu.wait async")
        fn.emit(f"{dev}, {t1} = gpu.alloc async [{t0}] ({n}) : memref<?xf64>")
        fn.emit(f"{t2} = gpu.memcpy async [{t1}] {dev}, {host} : memref<?xf64>, memref<?xf64>")
        fn.emit(f"gpu.wait [{t2}]")
        fn.emit(f"{bs} = arith.constant {BLOCK_SIZE} : index")
        fn.emit(f"{grid} = arith.ceildivui {n}, {bs} : index")
        fn.emit(f"gpu.launch blocks(%bx, %by, %bz) in (%grid_x = {grid}, %grid_y = {one}, "
                f"%grid_z = {one})")
        fn.open(f"           threads(%tx, %ty, %tz) in (%block_x = {bs}, %block_y = {one}, "
                f"%block_z = {one}) {{")
        off, gid, ok, it = fn.temp("off"), fn.temp("gid"), fn.temp("in"), fn.temp("it")
        fn.emit(f"{off} = arith.muli %bx, %block_x : index")
        fn.emit(f"{gid} = arith.addi {off}, %tx : index")
        fn.emit(f"{ok} = arith.cmpi ult, {gid}, {n} : index")
        fn.open(f"scf.if {ok} {{")
        fn.emit(f"{it} = arith.addi {lo}, {gid} : index")
        x = fn.as_f64(it)
        return _Loop(_GPU, x, last=x, host=host, device=dev, gid=gid)

    def _loop_end(self, fn: _Function) -> None:
        if not fn.loops:
            raise ValueError("LoopEnd without a LoopBegin")
        loop = fn.loops.pop()
        outer = fn.loops[-1] if fn.loops else None
        for name in ("index", "value"):  # the enclosing loop's index, if any, is visible again
            if outer:
                fn.variables[name] = outer.index_f64
            else:
                fn.variables.pop(name, None)
        if loop.kind != _GPU:
            fn.close()
            return
        fn.emit(f"memref.store {loop.last}, {loop.device}[{loop.gid}] : memref<?xf64>")
        fn.close()
        fn.emit("gpu.terminator")
        fn.close()
        t0, t1, t2 = fn.temp("t"), fn.temp("t"), fn.temp("t")
        fn.emit(f"{t0} = gpu.wait async")
        fn.emit(f"{t1} = gpu.memcpy async [{t0}] {loop.host}, {loop.device} : "
                f"memref<?xf64>, memref<?xf64>")
        fn.emit(f"{t2} = gpu.dealloc async [{t1}] {loop.device} : memref<?xf64>")
        fn.emit(f"gpu.wait [{t2}]")
        fn.emit(f"memref.dealloc {loop.host} : memref<?xf64>")


# ---- the lowering pipeline (MlirLinker.cs:60-76, retargeted) -------------------

def mlir_opt_args(input_path: str, output_path: str) -> str:
    """mlir-opt arguments of a module without GPU work (the reference's CPU pipeline)."""
    return (f'"{input_path}" --canonicalize --cse --symbol-dce --convert-scf-to-cf '
            "--convert-arith-to-llvm --convert-func-to-llvm --convert-cf-to-llvm "
            f'--reconcile-unrealized-casts -o "{output_path}"')


def mlir_opt_args_with_gpu(input_path: str, output_path: str, chip: str = ROCM_CHIP) -> str:
    """mlir-opt arguments of a module with gpu.launch: outline the launches into
    a gpu.module, attach #rocdl.target<chip = gfx950> to it, lower its body to
    the ROCDL dialect (the flag nests on gpu.module), serialize it to a gfx950
    code object embedded in the host module, then lower the host side's
    launches, allocations and copies to runtime calls."""
    return (f'"{input_path}" --canonicalize --cse --symbol-dce --gpu-kernel-outlining '
            f'--rocdl-attach-target="chip={chip}" --convert-scf-to-cf '
            f'--convert-gpu-to-rocdl="chipset={chip} index-bitwidth=64" '
            "--gpu-module-to-binary --gpu-to-llvm --convert-memref-to-llvm "
            "--convert-arith-to-llvm --convert-func-to-llvm --convert-cf-to-llvm "
            f'--reconcile-unrealized-casts -o "{output_path}"')


def gpu_link_args(llvm_ir_path: str, output_path: str) -> str:
    """clang arguments for the lowered host module: the GPU runtime calls that
    gpu-to-llvm emits come from MLIR's ROCm runtime wrappers over HIP."""
    return (f'"{llvm_ir_path}" -o "{output_path}" -O2 -L/opt/rocm/lib -lmlir_rocm_runtime '
            "-lamdhip64 -Wl,-rpath,/opt/rocm/lib")
