"""GPU parity of the image layout adapters (sh_bgr_to_rgba_u8,
sh_rgb_to_bgr_u8) against the CPU oracle, bit-exact: 24 and 32 bpp, ragged
widths, padded strides, the 4096 x 4096 round trip, argument checks."""
import numpy as np
import pytest

import oracle
import strict_amd
from tests.util import seeded_bytes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("w,h,bpp,pad", [(1, 1, 3, 0), (5, 3, 3, 1), (257, 9, 3, 1),
                                         (300, 17, 4, 0), (1023, 5, 4, 12), (4096, 64, 3, 0)])
def test_bgr_to_rgba_matches_oracle(ctx, w, h, bpp, pad):
    stride = w * bpp + pad
    src = seeded_bytes(stride * h, seed=w + h + bpp)
    d_src = ctx.upload(src)
    d_dst = ctx.upload(np.full(w * h * 4, 0xAB, np.uint8))
    ctx.bgr_to_rgba(d_src, bpp, stride, d_dst, w, h)
    ctx.sync()
    assert np.array_equal(d_dst.to_host(), oracle.bgr_to_rgba(src, w, h, bpp, stride))


@pytest.mark.parametrize("w,h,pad", [(1, 1, 1), (5, 3, 1), (257, 9, 3), (1023, 5, 0)])
def test_rgb_to_bgr_matches_oracle(ctx, w, h, pad):
    stride = 3 * w + pad
    rgb = seeded_bytes(w * h * 3, seed=w * 3 + h)
    canvas = seeded_bytes(stride * h, seed=9)
    d_dst = ctx.upload(canvas)
    ctx.rgb_to_bgr(ctx.upload(rgb), d_dst, w, h, stride)
    ctx.sync()
    assert np.array_equal(d_dst.to_host(), oracle.rgb_to_bgr(rgb, w, h, stride, canvas))


def test_round_trip_4096(ctx):
    w = h = 4096
    rgb = seeded_bytes(w * h * 3, seed=42)
    d_rgb = ctx.upload(rgb)
    d_bmp = ctx.upload(np.zeros(w * h * 3, np.uint8))
    d_rgba = ctx.upload(np.full(w * h * 4, 0xFF, np.uint8))
    ctx.rgb_to_bgr(d_rgb, d_bmp, w, h, 3 * w)
    ctx.bgr_to_rgba(d_bmp, 3, 3 * w, d_rgba, w, h)
    ctx.sync()
    rgba = d_rgba.to_host().reshape(-1, 4)
    assert np.array_equal(rgba[:, :3].reshape(-1), rgb)
    assert not rgba[:, 3].any()


def test_adapters_reject_bad_arguments(ctx):
    buf = ctx.empty(4096, np.uint8)
    other = ctx.empty(4096, np.uint8)
    for args in [(buf, 2, 12, other, 4, 4), (buf, 3, 11, other, 4, 4), (buf, 3, 12, buf, 4, 4)]:
        with pytest.raises(strict_amd.StrictHipError):
            ctx.bgr_to_rgba(*args)
    for args in [(buf, other, 4, 4, 11), (buf, buf, 4, 4, 12)]:
        with pytest.raises(strict_amd.StrictHipError):
            ctx.rgb_to_bgr(*args)
    buf.free()
    other.free()
