"""The reference's own known answers (tests/golden/reference_known_answers.json)
against the CPU oracle: pins the oracle's elementwise and brightness
restatements on the values the reference asserts."""
import json
from pathlib import Path

import numpy as np

import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
OPS = {"Add": oracle.ADD, "Subtract": oracle.SUBTRACT, "Multiply": oracle.MULTIPLY,
       "Divide": oracle.DIVIDE}


def test_binary_known_answers():
    for case in GOLDEN["binary_f32"]:
        n = case["count"]
        out = oracle.binary_f32(OPS[case["op"]], np.full(n, case["first"], np.float32),
                                np.full(n, case["second"], np.float32))
        assert np.all(out == case["expected"]), case


def test_initialize_depths_known_answers():
    for case in GOLDEN["initialize_depths"]:
        assert np.all(oracle.fill_f32(case["initial_depth"], case["count"]) == case["expected"])


def test_brightness_known_answers():
    cases = GOLDEN["brightness_u8"] + GOLDEN["brightness_float_x100"]["cases"]
    for case in cases:
        px = np.array(case["pixel"], np.uint8)
        assert list(oracle.adjust_brightness(px, case["delta"], 3)) == case["expected"], case


def test_sigmoid_reference_scalar():
    x = np.float32(GOLDEN["sigmoid_scalar"]["input"])
    y = oracle.sigmoid_f32(np.array([x], np.float32))[0]
    assert y == np.float32(1.0) / (np.float32(1.0) + np.float32(np.exp(-np.float64(x))))
