"""GPU parity of the elementwise kernels against the CPU oracle, through the
C ABI (sh_sigmoid_f32, sh_binary_f32, sh_fill_f32, sh_saxpy_f32)."""
import numpy as np
import pytest

import oracle
import strict_amd
from tests.util import seeded_uniform_f32, ulp_distance_f32

pytestmark = pytest.mark.gpu

N_CONFIG = 1 << 24


def _run_sigmoid(ctx, x):
    dx = ctx.upload(x)
    dy = ctx.empty(x.shape, np.float32)
    ctx.sigmoid(dx, dy, x.size)
    ctx.sync()
    y = dy.to_host()
    dx.free()
    dy.free()
    return y


def test_sigmoid_config_2pow24_within_2ulp(ctx):
    # N = 2^24 values uniform[-8, 8] from a seeded generator
    x = seeded_uniform_f32(N_CONFIG, -8.0, 8.0, seed=42)
    y = _run_sigmoid(ctx, x)
    ref = oracle.sigmoid_f32(x, nthreads=oracle.default_threads())
    d = ulp_distance_f32(y, ref)
    print(f"sigmoid 2^24: max ulp {d.max()}, bit-exact {np.mean(d == 0):.4f}", flush=True)
    assert d.max() <= 2  # north_star: sigmoid within 2 ulp fp32


def test_sigmoid_special_values_and_tails(ctx):
    x = np.array([0.0, 0.265, 8.0, -8.0, 20.0, -20.0, -88.0, 88.0, -104.0, 1e-30, -0.0],
                 np.float32)
    y = _run_sigmoid(ctx, x)
    assert y[0] == 0.5 and y[10] == 0.5
    ref = oracle.sigmoid_f32(x)
    assert ulp_distance_f32(y, ref).max() <= 2


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 4097, 262147])
def test_sigmoid_ragged_sizes(ctx, n):
    x = seeded_uniform_f32(n, -8, 8, seed=n)
    assert ulp_distance_f32(_run_sigmoid(ctx, x), oracle.sigmoid_f32(x)).max() <= 2


def test_sigmoid_unaligned_view(ctx):
    x = seeded_uniform_f32(1001, -8, 8, seed=9)
    dx = ctx.upload(x)
    dy = ctx.empty(1001, np.float32)
    # offset by one float: takes the unaligned path
    ctx.sigmoid(dx.view(4, 4000, np.float32), dy.view(4, 4000, np.float32), 1000)
    ctx.sync()
    y = dy.to_host()[1:]
    assert ulp_distance_f32(y, oracle.sigmoid_f32(x[1:])).max() <= 2
    dx.free()
    dy.free()


def test_sigmoid_zero_count_is_noop(ctx):
    ctx.sigmoid(None, None, 0)  # no pointers needed for empty work


def test_sigmoid_out_of_range_pointer_rejected(ctx):
    dx = ctx.empty(16, np.float32)
    dy = ctx.empty(16, np.float32)
    with pytest.raises(strict_amd.StrictHipError) as e:
        ctx.sigmoid(dx, dy, 17)
    assert e.value.status == strict_amd._lib.SH_ERR_INVALID_ARGUMENT
    dx.free()
    dy.free()


@pytest.mark.parametrize("op", [strict_amd.ADD, strict_amd.SUBTRACT, strict_amd.MULTIPLY,
                                strict_amd.DIVIDE])
def test_binary_ops_bit_exact(ctx, op):
    rng = np.random.default_rng(op)
    n = 1_000_003
    a = rng.normal(0, 10, n).astype(np.float32)
    b = rng.normal(0, 10, n).astype(np.float32)
    da, db, do = ctx.upload(a), ctx.upload(b), ctx.empty(n, np.float32)
    ctx.binary(op, da, db, do, n)
    ctx.sync()
    out = do.to_host()
    ref = oracle.binary_f32(op, a, b)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    for v in (da, db, do):
        v.free()


@pytest.mark.parametrize("op,expected", [(strict_amd.ADD, 3.0), (strict_amd.SUBTRACT, -1.0),
                                         (strict_amd.MULTIPLY, 2.0)])
def test_binary_reference_known_answers(ctx, op, expected):
    # CSharpToCudaTranspilerTests.ParseGenerateCudaAndExecute: first={1}, second={2}, count=1
    first, second = ctx.upload(np.array([1.0], np.float32)), ctx.upload(np.array([2.0], np.float32))
    out = ctx.empty(1, np.float32)
    ctx.binary(op, first, second, out, 1)
    ctx.sync()
    assert out.to_host()[0] == expected


def test_fill_initialize_depths(ctx):
    # InitializeDepths: Process(input, width, height, initialDepth = 5) -> 5
    out = ctx.empty(10, np.float32)
    ctx.fill(5.0, out, 10)
    ctx.sync()
    assert np.all(out.to_host() == 5.0)
    big = ctx.empty(1_000_001, np.float32)
    ctx.fill(-2.5, big, 1_000_001)
    ctx.sync()
    assert np.all(big.to_host() == -2.5)


def test_saxpy_bit_exact(ctx):
    rng = np.random.default_rng(11)
    n = 777_777
    x = rng.normal(0, 1, n).astype(np.float32)
    y = rng.normal(0, 1, n).astype(np.float32)
    dx, dy, do = ctx.upload(x), ctx.upload(y), ctx.empty(n, np.float32)
    ctx.saxpy(1.7, dx, dy, do, n)
    ctx.sync()
    ref = oracle.saxpy_f32(1.7, x, y)
    assert np.array_equal(do.to_host().view(np.uint32), ref.view(np.uint32))
