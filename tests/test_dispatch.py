"""Range-loop dispatch rule (sh_range_loop_target) against the reference's
own cases: InstructionsToMlir's serial / parallel / GPU choice by
iterations x body instructions (InstructionsToMlir.cs:397-418), as its tests
pin it (InstructionsToMlirTests.cs:598-884). No GPU needed: below the GPU
threshold the dispatcher launches nothing."""
import pytest

from strict_amd import codegen as cg
from strict_amd import dispatch as d


@pytest.mark.parametrize("iterations,body,target", [
    (8_294_400, 1, d.SH_LOOP_PARALLEL),  # ParallelHintEmitsScfParallel (:598-615)
    (100, 1, d.SH_LOOP_SERIAL),          # small loop stays scf.for (:620-635)
    (10_000, 20, d.SH_LOOP_PARALLEL),    # 200K complexity (:669-672)
    (50_000, 1, d.SH_LOOP_SERIAL),       # 50K complexity (:676-694)
    (921_600, 20, d.SH_LOOP_GPU),        # HighComplexityLoopEmitsGpuLaunch, 18.4M (:710-732)
    (100_000, 2, d.SH_LOOP_PARALLEL),    # MediumComplexityStaysScfParallelNotGpu (:852-873)
])
def test_reference_loop_cases(iterations, body, target):
    assert d.range_loop_target(iterations, body) == target


def test_thresholds_match_the_reference():
    # GpuThresholdConstantIsExposed (:876-884)
    assert d.GPU_COMPLEXITY_THRESHOLD == 10_000_000 > d.PARALLEL_COMPLEXITY_THRESHOLD == 100_000
    # "1280x720 image x 10+ body instructions": 10 stays below, 11 is over
    assert d.range_loop_target(1280 * 720, 10) == d.SH_LOOP_PARALLEL
    assert d.range_loop_target(1280 * 720, 11) == d.SH_LOOP_GPU


def test_strict_comparisons_and_edges():
    assert d.range_loop_target(10_000_000, 1) == d.SH_LOOP_PARALLEL  # > , not >=
    assert d.range_loop_target(10_000_001, 1) == d.SH_LOOP_GPU
    assert d.range_loop_target(100_000, 1) == d.SH_LOOP_SERIAL
    assert d.range_loop_target(100_001, 1) == d.SH_LOOP_PARALLEL
    assert d.range_loop_target(5_000_001, 0) == d.SH_LOOP_PARALLEL  # max(body, 1)
    assert d.range_loop_target(0, 1000) == d.SH_LOOP_SERIAL          # unknown end: 0 iterations
    assert d.range_loop_target(-7, 1000) == d.SH_LOOP_SERIAL
    assert d.range_loop_target(2 ** 62, 1000) == d.SH_LOOP_GPU      # saturating product


def test_dispatcher_leaves_small_loops_to_the_caller():
    # AdjustBrightness.strict's Run: a (1280 / 80) x (720 / 80) image, three
    # channels, body of 4 instructions: 1,728 complexity, a serial loop
    m = cg.Method.parse(["Brighten(current Number) Number", "\tcurrent + 0.25"])
    assert len(m.instructions) == 4
    hook = d.RangeLoopDispatcher(ctx=None)  # never touches a device below the threshold
    assert hook.run(m, 16 * 9 * 3, None, None) == d.SH_LOOP_SERIAL
    assert hook.run(m, 1280 * 720, None, None) == d.SH_LOOP_PARALLEL
