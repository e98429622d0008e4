"""Pins the contract mirror (oracle/contract.c) operator by operator.

1. Against the independent serial FP32 equations (operator_reference.cpp)
   at the reference's own operator shapes and deterministic operands, with
   the per-operator tolerances of numerical-portability.md:47-52.
2. Against closed forms and hand-derived values chosen so that a wrong
   reduction order, partial count, rounding point or index changes the bits.
"""
import numpy as np
import pytest

BF16_TOL = {"projection": (1e-3, 1.6e-2), "rotary": (1e-3, 1.6e-2), "silu": (1e-3, 1.6e-2),
            "rms_norm": (1e-2, 1e-2), "attention": (3e-2, 2e-2), "add": (0.0, 0.0)}


def close(o, a, b, kind):
    atol, rtol = BF16_TOL[kind]
    fa, fb = o.f32_from_bf16(a), o.f32_from_bf16(b)
    assert np.all(np.isfinite(fa))
    bad = np.abs(fa - fb) > atol + rtol * np.abs(fb)
    assert not bad.any(), (kind, int(bad.sum()), float(np.max(np.abs(fa - fb))))


@pytest.mark.parametrize("width", [128, 4096])
def test_rms_norm_vs_serial(oracle, width):
    x, w = oracle.operand(3 * width, 1), oracle.operand(width, 2)
    close(oracle, oracle.rms_norm(x, w, 3, width, 1e-6), oracle.rms_norm(x, w, 3, width, 1e-6, serial=True),
          "rms_norm")


def test_elementwise_vs_serial(oracle):
    x, up = oracle.operand(3 * 259, 3), oracle.operand(3 * 259, 4)
    x[:3] = oracle.bf16_from_f32(np.array([-80.0, 80.0, 0.0], np.float32))
    close(oracle, oracle.silu_multiply(x, up), oracle.silu_multiply(x, up, serial=True), "silu")
    ref = oracle.bf16_from_f32(oracle.f32_from_bf16(x) + oracle.f32_from_bf16(up))
    assert np.array_equal(oracle.add(x, up), ref)


@pytest.mark.parametrize("rows", [1, 9])
@pytest.mark.parametrize("out_w", [33, 1025])
def test_projection_vs_serial(oracle, rows, out_w):
    x, w = oracle.operand(rows * 128, 5), oracle.operand(out_w * 128, 6)
    close(oracle, oracle.projection(x, w, rows, 128, out_w), oracle.projection(x, w, rows, 128, out_w, serial=True),
          "projection")


def test_rotary_vs_serial(oracle):
    x = oracle.operand(3 * 2 * 128, 7)
    close(oracle, oracle.rotary(x, 3, 2, 128, 4093, 1e6), oracle.rotary(x, 3, 2, 128, 4093, 1e6, serial=True),
          "rotary")


@pytest.mark.parametrize("rows", [1, 37])
def test_attention_vs_serial(oracle, rows):
    q, k, v = oracle.operand(rows * 4 * 128, 8), oracle.operand(rows * 2 * 128, 9), oracle.operand(rows * 2 * 128, 10)
    close(oracle, oracle.attention(q, k, v, rows, 4, 2, 128, 0),
          oracle.attention(q, k, v, rows, 4, 2, 128, 0, serial=True), "attention")


def test_qwen_shapes_vs_serial(oracle):
    """Projection tolerance at the Qwen3-8B P=16 and P=32 shapes."""
    rng = np.random.default_rng(3)
    for in_w, out_w in ((4096, 2048), (4096, 1024), (12288, 64)):
        x = oracle.bf16_from_f32(rng.standard_normal(in_w).astype(np.float32))
        w = oracle.bf16_from_f32((0.02 * rng.standard_normal(in_w * out_w)).astype(np.float32))
        close(oracle, oracle.projection(x, w, 1, in_w, out_w), oracle.projection(x, w, 1, in_w, out_w, serial=True),
              "projection")


# ---------------------------------------------------------------- structure
def bf(values):
    import oracle as o
    return o.bf16_from_f32(np.asarray(values, np.float32))


def test_projection_partial_count_and_order(oracle):
    """Hand-derived values that only the reference tree produces.

    I = 64, x = 1, weights f0 = 1, f16 = 2^24, f32 = -2^24 (others 0):
      P = 16 (O > 1024): partial 0 is the chain 1, +2^24 (-> 2^24, the +1 is
        lost to round-to-even), -2^24 -> 0; result 0.
      P = 32 (O = 1024): partial 0 = 1 - 2^24 = -16777215 (exact), partial
        16 = 2^24; the offset-16 merge gives 1.
      A serial sum gives 0; a P mix-up flips the result."""
    x = bf(np.ones(64))
    for out_w, expected in ((1040, 0.0), (1024, 1.0)):
        w = np.zeros((out_w, 64), np.float32)
        w[0, 0], w[0, 16], w[0, 32] = 1.0, 2.0**24, -(2.0**24)
        y = oracle.f32_from_bf16(oracle.projection(x, bf(w), 1, 64, out_w))
        assert y[0] == expected, out_w


def test_projection_merge_offsets(oracle):
    """Merge upper into lower at offsets 8,4,2,1 (P = 16): partials
    p0 = 2^24, p1 = 1, p8 = -2^24 give (p0+p8) + ... + (p1+p9) = 1, while an
    adjacent-first tree gives (2^24+1 -> 2^24) - 2^24 = 0."""
    x = bf(np.ones(16))
    w = np.zeros((1040, 16), np.float32)
    w[0, 0], w[0, 1], w[0, 8] = 2.0**24, 1.0, -(2.0**24)
    assert oracle.f32_from_bf16(oracle.projection(x, bf(w), 1, 16, 1040))[0] == 1.0
    assert oracle.f32_from_bf16(oracle.projection(x, bf(w), 1, 16, 1040, serial=True))[0] == 0.0


def test_projection_ragged_tail_padding(oracle):
    """A width that is not a multiple of 16 adds the tiled kernel's padding
    FMA fma(0, 0, acc) to the tail partials; it turns a -0 partial into +0."""
    in_w, out_w = 20, 1025  # P = 16
    x = bf(np.ones(in_w))
    w = np.zeros((out_w, in_w), np.float32)
    w[0, :] = -0.0
    y = oracle.projection(x, bf(w), 1, in_w, out_w)
    assert y[0] == 0x0000  # +0, not -0x8000
    assert np.all(y == 0)


def test_rms_norm_closed_forms(oracle):
    # constant row c: inverse = 1/sqrt(c^2 + eps); gains 1 -> round(c * inverse)
    for c in (1.0, 0.5, 3.0):
        x = bf(np.full(4096, c))
        y = oracle.f32_from_bf16(oracle.rms_norm(x, bf(np.ones(4096)), 1, 4096, 1e-6))
        inv = np.float32(1.0) / np.sqrt(np.float32(np.float32(c * c) + np.float32(1e-6)))
        assert np.all(y == oracle.f32_from_bf16(bf([np.float32(c) * inv]))[0])
    # gain rounding point: round(round(x * inv) * w), not round(x * inv * w)
    x = bf(np.full(128, 1.0))
    w = bf(np.full(128, 1.0078125))  # 1 + 2^-7
    y = oracle.f32_from_bf16(oracle.rms_norm(x, w, 1, 128, 1e-6))
    inv = np.float32(1.0) / np.sqrt(np.float32(np.float32(1.0) + np.float32(1e-6)))
    n = oracle.f32_from_bf16(bf([inv]))[0]
    assert np.all(y == oracle.f32_from_bf16(bf([n * np.float32(1.0078125)]))[0])


def test_rms_norm_lane_tree(oracle):
    """Component sums and the 32-lane tree, checked on the inverse RMS.

    Lane t owns features 4t + c (width > 128).  Squares 1, 2^-24, 2^-24 in
    lanes 0, 2, 3 (features 0, 8, 12): the adjacent-first tree (shuffle
    offsets 1,2,4,8,16) adds 2^-24 + 2^-24 first and keeps it,
    total = 1 + 2^-23; a halving tree (offsets 16..1) would lose both halves
    to round-to-even, total = 1.  For width <= 128 lane t owns features
    t + 32c, so the same squares at features 0, 2, 3 land in lanes 0, 2, 3."""
    f = np.float32
    eps = f(1e-6)
    for D, idx in ((256, (0, 8, 12)), (128, (0, 2, 3))):
        xv = np.zeros(D, np.float32)
        xv[idx[0]], xv[idx[1]], xv[idx[2]] = 1.0, 2.0**-12, 2.0**-12
        inv = oracle.lib().orc_rms_inverse(bf(xv), D, 1e-6)
        right = f(1.0) / np.sqrt(f(f(f(1.0 + 2.0**-23) * f(1.0 / D)) + eps))
        wrong = f(1.0) / np.sqrt(f(f(f(1.0) * f(1.0 / D)) + eps))
        assert f(inv) == right
        if D == 256:
            assert right != wrong
    # components combine left to right within a lane: c0 + c1 + c2 + c3
    xv = np.zeros(256, np.float32)
    xv[0], xv[1], xv[2] = 1.0, 2.0**-12, 2.0**-12  # lane 0 components 0, 1, 2
    inv = oracle.lib().orc_rms_inverse(bf(xv), 256, 1e-6)
    left_to_right = f(f(f(1.0) + f(2.0**-24)) + f(2.0**-24))  # = 1 (both lost)
    assert f(inv) == f(1.0) / np.sqrt(f(f(left_to_right * f(1.0 / 256)) + eps))


def test_rotary_closed_forms(oracle):
    x = oracle.operand(2 * 3 * 128, 7)
    # position 0: cos = 1, sin = 0 -> identity
    assert np.array_equal(oracle.rotary(x[:3 * 128], 1, 3, 128, 0, 1e6), x[:3 * 128])
    # pair i = 0 has frequency 1: angle = position
    y = oracle.f32_from_bf16(oracle.rotary(x[:128], 1, 1, 128, 1, 1e6))
    a, b = oracle.f32_from_bf16(x[0:1])[0], oracle.f32_from_bf16(x[64:65])[0]
    c, s = [oracle.f32_from_bf16(bf([v]))[0] for v in (np.cos(1.0), np.sin(1.0))]
    r = lambda v: oracle.f32_from_bf16(bf([v]))[0]  # noqa: E731
    assert y[0] == r(r(a * c) - r(b * s))
    assert y[64] == r(r(b * c) + r(a * s))


def test_attention_closed_forms(oracle):
    # a single visible key: p = 1 exactly and the output is the V row
    q = oracle.operand(4 * 128, 8)
    k = oracle.operand(2 * 128, 9)
    v = oracle.operand(2 * 128, 10)
    y = oracle.attention(q, k, v, 1, 4, 2, 128, 0)
    assert np.array_equal(y.reshape(4, 128)[0], v.reshape(2, 128)[0])
    assert np.array_equal(y.reshape(4, 128)[3], v.reshape(2, 128)[1])
    # identical keys and values: uniform p = 1/n and the output is V
    n = 5
    k3 = np.tile(oracle.operand(2 * 128, 9), n)
    v3 = np.tile(bf(np.full(2 * 128, 3.0)), n)
    q3 = np.concatenate([oracle.operand(4 * 128, 8)] * n)
    y3 = oracle.f32_from_bf16(oracle.attention(q3, k3, v3, n, 4, 2, 128, 0))
    assert np.all(y3 == 3.0)


def test_attention_probability_rounding_point(oracle):
    """p is rounded to FP32 before weighting V (attention.cu:331-375): with
    two keys whose scores differ, out = round(fma(p0, v0, 0) + fma(p1, v1, 0))
    where p_j = FP32(e_j / l); the second key falls in the second range."""
    q = np.zeros((2, 4, 128), np.float32)
    q[:, :, 0] = 1.0
    k = np.zeros((2, 2, 128), np.float32)
    k[0, :, 0] = 8.0
    v = np.zeros((2, 2, 128), np.float32)
    v[0, :, :] = 1.0
    v[1, :, :] = 2.0
    y = oracle.f32_from_bf16(oracle.attention(bf(q.ravel()), bf(k.ravel()), bf(v.ravel()), 2, 4, 2, 128, 0))
    f = np.float32
    scale = f(1.0 / np.sqrt(128.0))
    s0, s1 = f(f(8.0) * scale), f(0.0)
    m = max(s0, s1)
    e0, e1 = f(np.exp(np.float64(f(s0 - m)))), f(np.exp(np.float64(f(s1 - m))))
    l = f(e0 + e1)
    p0, p1 = f(e0 / l), f(e1 / l)
    expected = oracle.f32_from_bf16(bf([f(f(p0 * f(1.0)) + f(p1 * f(2.0)))]))[0]
    assert np.all(y.reshape(2, 4, 128)[1, :, :] == expected)


def test_attention_scale(oracle):
    assert oracle.lib().orc_attention_scale(128) == np.float32(1.0 / np.sqrt(128.0))




def test_steer_closed_forms(oracle):
    """h <- BF16(FP32(h) + v): zero vector is the identity, exact sums stay
    exact, and ties round to even once (1 + 2^-8 -> 1, 1 + 3*2^-8 -> 1 + 2^-6)."""
    h0 = oracle.normal_bf16(4096, 3, 5, 1.0)
    h = h0.copy()
    oracle.steer(h, np.zeros(4096, np.float32))
    assert np.array_equal(h, h0)
    h = oracle.bf16_from_f32(np.array([1.0, 1.0, 1.0, -2.0], np.float32))
    oracle.steer(h, np.array([2.0**-8, 3 * 2.0**-8, 0.5, 0.25], np.float32))
    assert oracle.f32_from_bf16(h).tolist() == [1.0, 1.0 + 2.0**-6, 1.5, -1.75]
