"""Range-loop dispatch hook on the GPU: a loop over the complexity threshold
runs its body as the generated, hipRTC-compiled kernel (strict_amd.dispatch).
Workload: AdjustBrightness.strict's Process at the example's full 1280 x 720
size (RunnerTests.cs:270-289 expects (0.25, 0.25, 0.25) at the centre of a
black image brightened by 0.25), the body `current + 0.25` per channel.
Checker: float32 addition in numpy (x + 0.25 is exact in double, so the
kernel's double add rounded to float equals the float32 sum): bit-exact."""
import numpy as np
import pytest

from strict_amd import codegen as cg
from strict_amd import dispatch as d

pytestmark = pytest.mark.gpu

W, H = 1280, 720
BRIGHTEN = cg.Method.parse(["Brighten(current Number) Number", "\tcurrent + 0.25"])


def test_adjust_brightness_run_on_gpu(ctx):
    hook = d.RangeLoopDispatcher(ctx)
    n = W * H * 3
    src = ctx.upload(np.zeros(n, np.float32))
    dst = ctx.upload(np.full(n, np.nan, np.float32))
    assert hook.run(BRIGHTEN, n, src, dst) == d.SH_LOOP_GPU
    ctx.sync()
    img = dst.to_host().reshape(H, W, 3)
    assert tuple(img[H // 2, W // 2]) == (0.25, 0.25, 0.25)
    assert np.all(img == np.float32(0.25))
    hook.close()


def test_random_image_bit_exact_and_kernel_cached(ctx):
    hook = d.RangeLoopDispatcher(ctx)
    rng = np.random.default_rng(11)
    for n in (W * H * 3, W * H * 3 + 77):  # second run: cached kernel, ragged tail
        x = rng.standard_normal(n).astype(np.float32)
        src = ctx.upload(x)
        dst = ctx.upload(np.full(n + 64, np.nan, np.float32))
        assert hook.run(BRIGHTEN, n, src, dst) == d.SH_LOOP_GPU
        ctx.sync()
        out = dst.to_host()
        assert np.array_equal(out[:n], x + np.float32(0.25))
        assert np.all(np.isnan(out[n:]))
    assert len(hook._kernels) == 1
    hook.close()


def test_below_threshold_launches_nothing(ctx):
    hook = d.RangeLoopDispatcher(ctx)
    n = 16 * 9 * 3
    dst = ctx.upload(np.full(n, np.nan, np.float32))
    assert hook.run(BRIGHTEN, n, ctx.upload(np.zeros(n, np.float32)), dst) == d.SH_LOOP_SERIAL
    ctx.sync()
    assert np.all(np.isnan(dst.to_host()))
    assert not hook._kernels
