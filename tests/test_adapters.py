"""Image layout adapters' oracle (oracle.bgr_to_rgba / rgb_to_bgr), pinned
by known answers, by the reference's pointer walk run literally on tiny
images (a formulation independent of the oracle's strided views), and by
the round trip RGB -> bitmap BGR -> RGBA, which must give back RGB with
alpha 0 and leave the bitmap's row padding alone."""
import numpy as np
import pytest

import oracle
from tests.util import seeded_bytes


def _walk_bgr_to_rgba(src, w, h, bpp):
    # CreateColorImageFromBitmapData's loop (BlurPerformanceTests.cs:89-101):
    # one pointer advanced by bpp per pixel, no row padding skipped
    image = [0] * (w * h * 4)
    p = 0
    for y in range(h):
        for x in range(w):
            image[(x + y * w) * 4] = src[p + 2]
            image[(x + y * w) * 4 + 1] = src[p + 1]
            image[(x + y * w) * 4 + 2] = src[p]
            p += bpp
    return np.array(image, np.uint8)


def test_known_answers():
    assert list(oracle.bgr_to_rgba(np.array([1, 2, 3], np.uint8), 1, 1, 3, 3)) == [3, 2, 1, 0]
    assert list(oracle.bgr_to_rgba(np.array([1, 2, 3, 9], np.uint8), 1, 1, 4, 4)) == [3, 2, 1, 0]
    out = oracle.rgb_to_bgr(np.array([10, 20, 30], np.uint8), 1, 1, 4, np.full(4, 7, np.uint8))
    assert list(out) == [30, 20, 10, 7]


@pytest.mark.parametrize("w,h,bpp", [(1, 1, 3), (3, 2, 3), (5, 3, 4), (7, 4, 3), (2, 5, 4)])
def test_oracle_matches_the_pointer_walk(w, h, bpp):
    src = seeded_bytes(w * h * bpp, seed=w * 10 + h)
    assert np.array_equal(oracle.bgr_to_rgba(src, w, h, bpp, w * bpp),
                          _walk_bgr_to_rgba(list(src), w, h, bpp))


@pytest.mark.parametrize("w,h,pad", [(1, 1, 1), (5, 3, 1), (6, 4, 2), (13, 7, 3)])
def test_round_trip_restores_rgb_and_keeps_padding(w, h, pad):
    rgb = seeded_bytes(w * h * 3, seed=w + 100 * h)
    stride = 3 * w + pad
    canvas = seeded_bytes(stride * h, seed=5)
    bmp = oracle.rgb_to_bgr(rgb, w, h, stride, canvas)
    for y in range(h):  # padding untouched
        assert np.array_equal(bmp[y * stride + 3 * w:(y + 1) * stride],
                              canvas[y * stride + 3 * w:(y + 1) * stride])
    rgba = oracle.bgr_to_rgba(bmp, w, h, 3, stride).reshape(h, w, 4)
    assert np.array_equal(rgba[..., :3].reshape(-1), rgb)
    assert np.all(rgba[..., 3] == 0)
