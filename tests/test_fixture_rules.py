"""Acceptance rules of the reference fixtures (forward_reference.py:212-220,
scripts/validation/README.md:128-142) as dolittle_amd/fixtures.py applies
them: both the maximum absolute error and the relative L2 error must be
within the output's bounds; an all-zero reference has no relative error."""
import math

import numpy as np

from dolittle_amd.fixtures import error, f32_from_bf16, within


def test_error_closed_forms():
    e = error([3.0, 4.0], [3.0, 4.0])
    assert e == {"max_absolute_error": 0.0, "relative_l2": 0.0}
    e = error([3.0, 4.0], [3.0, 5.0])
    assert e["max_absolute_error"] == 1.0 and math.isclose(e["relative_l2"], 1.0 / 5.0)
    assert error([0.0, 0.0], [0.0, 1e-9])["relative_l2"] is None


def test_both_bounds_must_hold():
    bound = {"max_absolute_error": 0.5, "max_relative_l2": 0.1}
    assert within(error([10.0, 0.0], [10.4, 0.0]), bound)
    assert not within(error([10.0, 0.0], [10.6, 0.0]), bound)        # absolute bound
    assert not within(error([1.0, 1.0], [1.4, 1.4]), bound)            # relative bound
    assert within(error([0.0], [0.1]), bound)                          # no relative error at zero


def test_bf16_decoding():
    bits = np.array([0x3F80, 0xC000, 0x0000, 0x8000], np.uint16)
    assert f32_from_bf16(bits).tolist() == [1.0, -2.0, 0.0, -0.0]
