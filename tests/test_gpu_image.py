"""GPU parity of the image kernels against the CPU oracle, bit-exact, through
the C ABI (sh_adjust_brightness_u8, sh_box_blur5_u8, sh_brightness_blur5_u8)."""
import numpy as np
import pytest

import oracle
import strict_amd
from tests.util import seeded_bytes

pytestmark = pytest.mark.gpu

W = H = 4096
NT = oracle.default_threads()


def _gpu(ctx, fn, img, *args):
    src = ctx.upload(img)
    dst = ctx.empty(img.shape, np.uint8)
    fn(src, dst, *args)
    ctx.sync()
    out = dst.to_host()
    src.free()
    dst.free()
    return out


@pytest.mark.parametrize("delta", [40, -40])
def test_brightness_config_4096_rgba(ctx, delta):
    img = seeded_bytes(W * H * 4, seed=42)
    out = _gpu(ctx, ctx.adjust_brightness, img, W, H, 4, delta, 0)
    assert np.array_equal(out, oracle.adjust_brightness(img, delta, 4, nthreads=NT))


@pytest.mark.parametrize("w,h,c,delta,flags", [
    (1, 1, 4, 255, 0), (3, 1, 3, 5, 0), (7, 5, 3, -5, 0), (13, 11, 4, 40, 1),
    (33, 17, 1, -40, 0), (99, 7, 2, 100, 0), (1000, 3, 4, -255, 0), (641, 479, 3, 10, 0)])
def test_brightness_shapes(ctx, w, h, c, delta, flags):
    img = seeded_bytes(w * h * c, seed=w + h)
    out = _gpu(ctx, ctx.adjust_brightness, img, w, h, c, delta, flags)
    assert np.array_equal(out, oracle.adjust_brightness(img, delta, c, all_channels=bool(flags)))


def test_brightness_readme_known_answers(ctx):
    # README.md:436-443: Color(0, 1, 2) + 5 -> (5, 6, 7); (0, 0, 0) - 5 -> (0, 0, 0)
    px = np.array([0, 1, 2], np.uint8)
    assert list(_gpu(ctx, ctx.adjust_brightness, px, 1, 1, 3, 5, 0)) == [5, 6, 7]
    assert list(_gpu(ctx, ctx.adjust_brightness, np.zeros(3, np.uint8), 1, 1, 3, -5, 0)) == [0, 0, 0]


def test_brightness_in_place(ctx):
    img = seeded_bytes(640 * 480 * 4, seed=3)
    buf = ctx.upload(img)
    ctx.adjust_brightness(buf, buf, 640, 480, 4, -40, 0)
    ctx.sync()
    assert np.array_equal(buf.to_host(), oracle.adjust_brightness(img, -40, 4))
    buf.free()


def test_brightness_rejects_bad_arguments(ctx):
    buf = ctx.empty(64, np.uint8)
    for args in [(4, 4, 5, 1, 0), (4, 4, 4, 300, 0), (4, 4, 4, 1, 8), (5, 4, 4, 1, 0)]:
        with pytest.raises(strict_amd.StrictHipError):
            ctx.adjust_brightness(buf, buf, *args)
    buf.free()


@pytest.mark.parametrize("mode", [strict_amd.BLUR_CONFIG, strict_amd.BLUR_REFERENCE])
def test_blur_config_4096_rgba(ctx, mode):
    img = seeded_bytes(W * H * 4, seed=42)
    out = _gpu(ctx, ctx.box_blur5, img, W, H, 4, mode)
    ref = (oracle.blur5_config if mode == strict_amd.BLUR_CONFIG else oracle.blur5_reference)(
        img, W, H, 4, nthreads=NT)
    assert np.array_equal(out, ref)


BLUR_SHAPES = [(1, 1, 4), (4, 1, 4), (2, 3, 3), (5, 5, 4), (10, 10, 3), (20, 20, 3),
               (8, 37, 4), (260, 33, 4), (512, 64, 4), (300, 2, 4), (17, 9, 4), (33, 6, 1),
               (1028, 70, 4), (64, 1, 2), (264, 17, 4), (768, 18, 4)]


@pytest.mark.parametrize("w,h,c", BLUR_SHAPES)
@pytest.mark.parametrize("mode", [strict_amd.BLUR_CONFIG, strict_amd.BLUR_REFERENCE])
def test_blur_shapes(ctx, w, h, c, mode):
    img = seeded_bytes(w * h * c, seed=w * 31 + h)
    out = _gpu(ctx, ctx.box_blur5, img, w, h, c, mode)
    ref = (oracle.blur5_config if mode == strict_amd.BLUR_CONFIG else oracle.blur5_reference)(
        img, w, h, c)
    assert np.array_equal(out, ref)


@pytest.mark.parametrize("size", [10, 20])
def test_blur_reference_rgb_known_sizes(ctx, size):
    # BlurProducesCorrectResults sizes (Assembly BlurPerformanceTests.cs:193-206), RGB
    img = seeded_bytes(size * size * 3, seed=42)
    out = _gpu(ctx, ctx.box_blur5, img, size, size, 3, strict_amd.BLUR_REFERENCE)
    assert np.array_equal(out, oracle.blur5_reference(img, size, size, 3))


@pytest.mark.parametrize("delta", [40, -40])
def test_fused_brightness_blur_4096(ctx, delta):
    img = seeded_bytes(W * H * 4, seed=7)
    out = _gpu(ctx, ctx.brightness_blur5, img, W, H, 4, delta, 0, strict_amd.BLUR_CONFIG)
    assert np.array_equal(out, oracle.brightness_blur5_config(img, W, H, delta, 4, nthreads=NT))


@pytest.mark.parametrize("w,h,c,flags", [(13, 11, 4, 0), (260, 40, 4, 1), (9, 9, 3, 0)])
def test_fused_shapes(ctx, w, h, c, flags):
    img = seeded_bytes(w * h * c, seed=w)
    out = _gpu(ctx, ctx.brightness_blur5, img, w, h, c, -40, flags, strict_amd.BLUR_CONFIG)
    ref = oracle.brightness_blur5_config(img, w, h, -40, c, all_channels=bool(flags))
    assert np.array_equal(out, ref)


def test_blur_invariants_on_gpu(ctx):
    const = np.full(512 * 64 * 4, 201, np.uint8)
    for mode in (strict_amd.BLUR_CONFIG, strict_amd.BLUR_REFERENCE):
        assert np.all(_gpu(ctx, ctx.box_blur5, const, 512, 64, 4, mode) == 201)
    # determinism: two runs give identical bytes
    img = seeded_bytes(1024 * 96 * 4, seed=5)
    a = _gpu(ctx, ctx.box_blur5, img, 1024, 96, 4, strict_amd.BLUR_CONFIG)
    b = _gpu(ctx, ctx.box_blur5, img, 1024, 96, 4, strict_amd.BLUR_CONFIG)
    assert np.array_equal(a, b)


def test_blur_rejects_aliasing(ctx):
    buf = ctx.empty(16 * 16 * 4, np.uint8)
    with pytest.raises(strict_amd.StrictHipError):
        ctx.box_blur5(buf, buf, 16, 16, 4)
    buf.free()
