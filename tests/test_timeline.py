"""The diagnostic timeline reader (strict_amd/timeline.py): its mark
arithmetic and its refusal of a library built without the trace flags.
CPU only; the timelines themselves need a GPU and a diagnostic build."""
import numpy as np
import pytest

from strict_amd import timeline


def test_ns_marks_missing_as_minus_one():
    t = np.array([0, 100, 250], np.int64)
    assert timeline._ns(t, 100).tolist() == [-1, 0, 1500]  # 100 MHz ticks -> ns


def test_median_and_max_skip_missing_marks():
    x = np.array([-1, 30, 10, 20, -1])
    assert timeline._med(x) == 20.0
    assert timeline._max(x) == 30.0
    assert np.isnan(timeline._med(np.array([-1, -1])))


def test_sub_pairs_only_workgroups_with_both_marks():
    a = np.array([0, 10, -1, 40])
    b = np.array([5, 30, 50, -1])
    # pairs (0, 5) and (10, 30): differences 5 and 20
    assert timeline._sub(a, b) == 12.5


def test_product_library_is_refused():
    class NoTrace:  # a library without sh_debug_*_trace
        pass

    with pytest.raises(SystemExit, match="trace flag"):
        timeline._trace(NoTrace(), "sh_debug_decode_trace", (2, 2))
