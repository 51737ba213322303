"""Range-loop dispatch hook: runs the body of a Strict range loop as a
generated GPU kernel when the loop is complex enough.

The reference's VM runs range loops on the CPU (VirtualMachine.Loops.cs:111+);
its MLIR backend chooses between a serial loop, a CPU-parallel loop and a GPU
launch by complexity = iterations x max(body instructions, 1) against
ComplexityThreshold = 100,000 and GpuComplexityThreshold = 10,000,000
(InstructionsToMlir.cs:397-418). `range_loop_target` is that rule (through
the C ABI, sh_range_loop_target). `RangeLoopDispatcher.run` is the hook a VM
calls for a range loop whose body is an elementwise method: at the GPU target
it generates the method's HIP kernel (sh_instructions_to_hip), compiles it
for gfx950 with hipRTC once per method, launches it over the loop's
iterations and returns SH_LOOP_GPU; at the other targets it launches nothing
and returns the target, and the caller runs the loop itself, as the
reference's VM does for every loop."""
from typing import Dict, Optional

from . import _lib, codegen as cg

SH_LOOP_SERIAL, SH_LOOP_PARALLEL, SH_LOOP_GPU = 0, 1, 2
GPU_COMPLEXITY_THRESHOLD = 10_000_000  # InstructionsToMlir.cs:418
PARALLEL_COMPLEXITY_THRESHOLD = 100_000  # InstructionsToMlir.cs:414

_GRID_X = 64  # generated kernels index y * (64 * block) + x over a 2-D grid
_BLOCK = 256


def range_loop_target(iterations: int, body_instructions: int) -> int:
    """SH_LOOP_SERIAL, SH_LOOP_PARALLEL or SH_LOOP_GPU for a range loop of
    `iterations` with `body_instructions` between its begin and end
    (InstructionsToMlir.cs:397-408, CountLoopBodyInstructions :420-432)."""
    return _lib.load().sh_range_loop_target(int(iterations), int(body_instructions))


class RangeLoopDispatcher:
    """Hook for a VM's range loops over elementwise bodies: one per context,
    caching each body's compiled kernel."""

    def __init__(self, ctx):
        self.ctx = ctx
        self._kernels: Dict[str, object] = {}

    def kernel(self, method: cg.Method):
        """The method's generated kernel, compiled for gfx950 on first use."""
        source = cg.InstructionsToHip().compile(method)
        k = self._kernels.get(source)
        if k is None:
            from . import RuntimeCompiler
            with RuntimeCompiler(source, method.name) as rtc:
                rtc.compile()
                k = self.ctx.load_kernel(rtc.get_code(), method.name)
            self._kernels[source] = k
        return k

    def run(self, method: cg.Method, iterations: int, *buffers,
            body_instructions: Optional[int] = None) -> int:
        """Runs `output[i] = method(inputs[i]...)` for i < iterations on the
        GPU when the loop's complexity is over the GPU threshold. `buffers`
        are the device arrays of the method's parameters, then the output.
        body_instructions defaults to the method's instruction count.
        Returns the target; only SH_LOOP_GPU launched anything."""
        body = len(method.instructions) if body_instructions is None else body_instructions
        target = range_loop_target(iterations, body)
        if target != SH_LOOP_GPU:
            return target
        if len(buffers) != len(method.parameters) + 1:
            raise ValueError(f"{method.name} takes {len(method.parameters)} inputs and one output")
        k = self.kernel(method)
        k.block_dimensions = _BLOCK
        k.grid_dimensions = (_GRID_X, -(-iterations // (_GRID_X * _BLOCK)), 1)
        k.run(*buffers, iterations)
        return target

    def close(self) -> None:
        for k in self._kernels.values():
            k.module.unload()
        self._kernels.clear()
