"""Pins the NLA restatement (oracle/nla.c: injection.cu:49-98,
steering.cu:69-159) with closed forms and with inputs whose bits change
under a different reduction: the eight strided lanes (i mod 8, ascending),
the left-to-right lane combination, and the separate multiply/add/divide
rounding points.  Status rules follow the reference kernels."""
import numpy as np
import pytest


def f32(x):
    return np.float32(x)


def test_inject_closed_form(oracle):
    h = np.zeros(8, np.float32)
    h[0], h[1] = 3.0, 4.0
    status, norm, out = oracle.inject(oracle.bf16_from_f32(h), True, True, 150.0)
    assert status == 0 and norm == 5.0
    assert oracle.f32_from_bf16(out)[:2].tolist() == [90.0, 120.0] and not out[2:].any()
    status, norm, out = oracle.inject(h, False, False, 150.0)
    # (3 / 5) and (4 / 5) are rounded before the multiply by 150.
    assert status == 0 and out[0] == f32(f32(3.0) / f32(5.0)) * f32(150.0)
    assert out[1] == f32(f32(4.0) / f32(5.0)) * f32(150.0)


def test_lane_combination_is_left_to_right(oracle):
    # Lane sums 2^24, 1, ..., 1: each +1 is lost to round-to-even when the
    # lanes are added 0..7 in order; any other order keeps some of them.
    h = np.array([4096.0] + [1.0] * 7, np.float32)
    status, norm, _ = oracle.inject(h, False, False, 1.0)
    assert status == 0 and norm == 4096.0


def test_lanes_are_strided(oracle):
    # 4096 then fifteen ones: lanes i mod 8 hold 2^24 + 1 -> 2^24 (lane 0)
    # and 2 (lanes 1..7), so the square sum is 2^24 + 14; an ascending serial
    # sum would lose every one and give 2^24.
    h = np.array([4096.0] + [1.0] * 15, np.float32)
    _, norm, _ = oracle.inject(h, False, False, 1.0)
    assert norm == np.sqrt(f32(16777230.0)) and norm != 4096.0


def test_inject_statuses(oracle):
    zero = np.zeros(16, np.float32)
    status, norm, out = oracle.inject(zero, False, True, 150.0)
    assert status == 1 and norm == 0.0 and not out.any()
    nan = np.ones(16, np.float32)
    nan[5] = np.nan
    assert oracle.inject(nan, False, True, 150.0)[0] == 1
    inf = np.ones(16, np.float32)
    inf[3] = np.inf
    assert oracle.inject(inf, False, False, 1.0)[0] == 1
    # 3.4e38 is finite in FP32 but rounds to +inf in BF16 storage.
    one = np.zeros(16, np.float32)
    one[0] = 1.0
    status, _, out = oracle.inject(one, False, True, 3.4e38)
    assert status == 1 and out[0] == 0x7F80
    assert oracle.inject(one, False, False, 3.4e38)[0] == 0


@pytest.mark.parametrize("width", [1, 7, 1000, 4096])
def test_inject_within_float64_bound(oracle, width):
    rng = np.random.default_rng(width)
    h = oracle.bf16_from_f32(rng.standard_normal(width).astype(np.float32) * 3)
    status, norm, out = oracle.inject(h, True, False, 150.0)
    x = oracle.f32_from_bf16(h).astype(np.float64)
    exact = np.sqrt(np.sum(x * x))
    assert status == 0 and abs(norm - exact) <= 1e-6 * exact
    assert np.allclose(out, x / exact * 150.0, rtol=1e-6, atol=0)


def test_direction(oracle):
    a = np.zeros(8, np.float32)
    b = np.zeros(8, np.float32)
    b[0], b[1] = 3.0, 4.0
    status, u = oracle.direction(a, b, False)
    assert status == 0 and u[0] == f32(3.0) / f32(5.0) and u[1] == f32(4.0) / f32(5.0) and not u[2:].any()
    status, u = oracle.direction(oracle.bf16_from_f32(b), oracle.bf16_from_f32(b), True)
    assert status == 1 and not u.any()
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32)
    y = rng.standard_normal(4096).astype(np.float32)
    status, u = oracle.direction(x, y, False)
    d = y.astype(np.float64) - x.astype(np.float64)
    assert status == 0 and np.allclose(u, d / np.linalg.norm(d), rtol=1e-5, atol=1e-9)


def test_intervene_closed_form_and_count(oracle):
    rows, width = 3, 8
    h = np.zeros((rows, width), np.float32)
    h[1, 0], h[1, 1] = 3.0, 4.0
    hb = oracle.bf16_from_f32(h.ravel())
    u = np.zeros(width, np.float32)
    u[0] = 1.0
    state = np.zeros(2, np.uint32)
    # Chunk positions [10, 13): row 1 is position 11.
    assert oracle.intervene(hb, True, rows, width, u, 10, 11, 1.0, state)
    row = oracle.f32_from_bf16(hb).reshape(rows, width)
    assert state.tolist() == [0, 1] and row[1, 0] == 8.0 and row[1, 1] == 4.0
    assert not row[0].any() and not row[2].any()
    # A second application is invalid and leaves the row unchanged.
    before = hb.copy()
    assert oracle.intervene(hb, True, rows, width, u, 10, 11, 1.0, state)
    assert state.tolist() == [1, 2] and np.array_equal(hb, before)
    # A chunk that does not hold the position changes nothing.
    fresh = np.zeros(2, np.uint32)
    assert not oracle.intervene(hb, True, rows, width, u, 0, 11, 1.0, fresh)
    assert fresh.tolist() == [0, 0]


def test_intervene_separate_rounding(oracle):
    # beta = strength * sqrt(sum) is rounded before it scales u, and
    # beta * u[i] is rounded before the add.
    width = 4
    h = np.array([1.0, 1.0, 1.0, 1.0], np.float32)
    u = np.array([0.1, 0.2, 0.3, 0.4], np.float32)
    state = np.zeros(2, np.uint32)
    assert oracle.intervene(h, False, 1, width, u, 0, 0, 0.7, state)
    beta = f32(0.7) * np.sqrt(f32(4.0))
    expect = np.array([f32(1.0) + f32(beta * u[i]) for i in range(width)], np.float32)
    assert state.tolist() == [0, 1] and np.array_equal(h, expect)


def test_intervene_zero_strength_counts(oracle):
    h = oracle.bf16_from_f32(np.ones(16, np.float32))
    state = np.zeros(2, np.uint32)
    before = h.copy()
    assert oracle.intervene(h, True, 1, 16, np.ones(16, np.float32), 5, 5, 0.0, state)
    assert state.tolist() == [0, 1] and np.array_equal(h, before)
