"""The reference's own known answers (tests/golden/reference_known_answers.json)
through the HIP kernels of the C ABI."""
import json
from pathlib import Path

import numpy as np
import pytest

import strict_amd

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
OPS = {"Add": strict_amd.ADD, "Subtract": strict_amd.SUBTRACT, "Multiply": strict_amd.MULTIPLY,
       "Divide": strict_amd.DIVIDE}


def test_binary_known_answers_on_gpu(ctx):
    for case in GOLDEN["binary_f32"]:
        n = case["count"]
        a = ctx.upload(np.full(n, case["first"], np.float32))
        b = ctx.upload(np.full(n, case["second"], np.float32))
        o = ctx.empty((n,), np.float32)
        ctx.binary(OPS[case["op"]], a, b, o, n)
        ctx.sync()
        assert np.all(o.to_host() == case["expected"]), case
        for v in (a, b, o):
            v.free()


def test_initialize_depths_known_answers_on_gpu(ctx):
    for case in GOLDEN["initialize_depths"]:
        o = ctx.empty((case["count"],), np.float32)
        ctx.fill(case["initial_depth"], o, case["count"])
        ctx.sync()
        assert np.all(o.to_host() == case["expected"])
        o.free()


def test_brightness_known_answers_on_gpu(ctx):
    for case in GOLDEN["brightness_u8"] + GOLDEN["brightness_float_x100"]["cases"]:
        src = ctx.upload(np.array(case["pixel"], np.uint8))
        dst = ctx.empty((3,), np.uint8)
        ctx.adjust_brightness(src, dst, 1, 1, 3, case["delta"], 0)
        ctx.sync()
        assert list(dst.to_host()) == case["expected"], case
        src.free()
        dst.free()
