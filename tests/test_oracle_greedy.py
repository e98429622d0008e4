"""Pins the oracle's greedy selection (orc_greedy_bf16, the greedy oracle of
every token-stream test) against the reference's own categorical.cpp
(src/inference/sampling/categorical.cpp:146-201, compiled into oracle/_ref)
and against closed forms.

The reference's greedy is min_element over the finite candidates under
(value descending, id ascending); NaN or +inf anywhere throws
invalid_argument, and so does a row with no finite value.  The oracle
returns status 1 for the first case and 2 for the second; both correspond to
the reference's throw (status 1 of the _ref harness).
"""
import numpy as np
import pytest

from test_oracle_kat import _device_kat_logits, _ref_select

NEG_ZERO, POS_ZERO, NEG_INF, POS_INF, NAN = 0x8000, 0x0000, 0xFF80, 0x7F80, 0x7FC0


def bf16_row(oracle, values):
    return oracle.bf16_from_f32(np.asarray(values, np.float32))


def check_against_reference(oracle, bits):
    """Oracle and reference agree on the selection or on the rejection."""
    status, got = oracle.greedy(bits)
    values = oracle.f32_from_bf16(bits).astype(np.float32)
    if oracle.ref() is not None:
        ref_status, ref_ids = _ref_select(oracle, values, 0, 1.0, 0, 1.0, 0)
        assert (status != 0) == (ref_status != 0), (status, ref_status)
        if status == 0:
            assert got == int(ref_ids[0]), (got, int(ref_ids[0]))
    return status, got


def closed_form(oracle, bits):
    """argmax over the finite values, lowest id on ties (-0 == +0)."""
    v = oracle.f32_from_bf16(bits).astype(np.float64)
    if np.any(np.isnan(v)) or np.any(v == np.inf):
        return 1, None
    finite = np.isfinite(v)
    if not finite.any():
        return 2, None
    best = v[finite].max()
    return 0, int(np.nonzero(finite & (v == best))[0][0])


@pytest.mark.parametrize("n", [1, 513, 151936])
def test_greedy_on_the_reference_device_grid(oracle, n):
    # tests/gpu/test_device.cpp:285-320: (i mod 97 - 48) / 8, -0 and +0 at
    # ids 0 and 1, -inf last; as BF16 (every grid value is exact in BF16).
    values = _device_kat_logits(n)
    bits = bf16_row(oracle, values)
    assert np.array_equal(oracle.f32_from_bf16(bits), values.astype(np.float32))
    status, got = check_against_reference(oracle, bits)
    want = closed_form(oracle, bits)
    assert (status, got if status == 0 else None) == want


def test_greedy_edges(oracle):
    cases = {
        # +0 and -0 tie: the lowest id wins whichever sign it carries.
        "zeros -0 first": ([NEG_ZERO, POS_ZERO] + [0xBF80] * 6, (0, 0)),
        "zeros +0 first": ([POS_ZERO, NEG_ZERO] + [0xBF80] * 6, (0, 0)),
        "zero after negatives": ([0xBF80, 0xC000, NEG_ZERO, POS_ZERO], (0, 2)),
        "three-way tie": ([0x3F80, 0x4000, 0x3F80, 0x4000, 0x4000], (0, 1)),
        "-inf skipped": ([NEG_INF, 0xC040, NEG_INF, 0xC000], (0, 3)),
        "only one finite": ([NEG_INF] * 5 + [0xC2C8] + [NEG_INF] * 2, (0, 5)),
        "all -inf": ([NEG_INF] * 8, (2, None)),
        "NaN": ([0x3F80, NAN, 0x4000], (1, None)),
        "negative NaN": ([0x3F80, 0xFFC1, 0x4000], (1, None)),
        "+inf": ([0x3F80, 0x4000, POS_INF], (1, None)),
        "+inf among -inf": ([NEG_INF, POS_INF], (1, None)),
        "largest finite": ([0x7F7F, 0x7F7E, 0xFF7F], (0, 0)),
        "subnormals": ([0x0001, 0x0002, 0x8003], (0, 1)),
    }
    for name, (row, want) in cases.items():
        bits = np.array(row, np.uint16)
        status, got = check_against_reference(oracle, bits)
        assert (status, got if status == 0 else None) == want, name
        assert closed_form(oracle, bits) == want, name


def test_greedy_random_rows_with_ties(oracle):
    """Rows drawn from a few values (many ties), with -0, -inf and a rare
    NaN or +inf, against the reference and the closed form."""
    rng = np.random.default_rng(11)
    pool = np.array([0x3F80, 0x4000, 0x4040, 0xBF80, POS_ZERO, NEG_ZERO, NEG_INF, 0x3F81, 0x4001], np.uint16)
    for trial in range(300):
        n = int(rng.integers(1, 600))
        bits = pool[rng.integers(0, pool.size, n)]
        if trial % 10 == 3:
            bits[rng.integers(0, n)] = NAN
        if trial % 10 == 7:
            bits[rng.integers(0, n)] = POS_INF
        if trial % 17 == 0:
            bits[:] = NEG_INF
        status, got = check_against_reference(oracle, bits)
        assert (status, got if status == 0 else None) == closed_form(oracle, bits), trial


def test_greedy_full_vocabulary_random_bf16(oracle):
    """151,936 random finite BF16 logits with the maximum planted twice."""
    rng = np.random.default_rng(5)
    values = rng.standard_normal(151936).astype(np.float32) * 3
    bits = bf16_row(oracle, values)
    bits[[90000, 1234]] = 0x41A0  # 20.0, above every N(0, 9) draw here (max 13.1)
    status, got = check_against_reference(oracle, bits)
    assert (status, got) == (0, 1234)
