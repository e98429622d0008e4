"""Pins the CPU oracle's integer/bit/sampling parts against known answers:
the reference's own test vectors, the reference's own host sources compiled
into oracle/_ref (when available), and standard-fixed values."""
import math
import struct

import numpy as np
import pytest


def f32(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", bits))[0]


# tests/core/test_bf16.cpp:54-66 (rounding KAT table)
BF16_CASES = [
    (0x00000000, 0x0000), (0x80000000, 0x8000), (0x00008000, 0x0000), (0x80008000, 0x8000),
    (0x00008001, 0x0001), (0x80008001, 0x8001), (0x00018000, 0x0002), (0x80018000, 0x8002),
    (0x007f8000, 0x0080), (0x807f8000, 0x8080), (0x3f807fff, 0x3f80), (0x3f808000, 0x3f80),
    (0x3f808001, 0x3f81), (0x3f818000, 0x3f82), (0xbf808000, 0xbf80), (0xbf818000, 0xbf82),
    (0x7f7f7fff, 0x7f7f), (0x7f7f8000, 0x7f80), (0xff7f8000, 0xff80), (0x7f800000, 0x7f80),
    (0xff800000, 0xff80), (0x7f800001, 0x7fc0), (0xff800001, 0x7fc0), (0x7fffffff, 0x7fc0),
    (0xffffffff, 0x7fc0),
]


def test_bf16_rounding_kat(oracle):
    lib = oracle.lib()
    for inp, expected in BF16_CASES:
        assert lib.or_bf16_from_f32(f32(inp)) == expected, hex(inp)
    bits = np.array([i for i, _ in BF16_CASES], dtype=np.uint32)
    vec = oracle.bf16_from_f32(bits.view(np.float32))
    assert list(vec) == [e for _, e in BF16_CASES]


def test_bf16_exhaustive_round_trip(oracle):
    # tests/core/test_bf16.cpp:33-52: every encoding widens exactly; exact
    # values survive narrowing; NaNs canonicalise to 0x7fc0.
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    widened = oracle.f32_from_bf16(allbits)
    assert np.array_equal(widened.view(np.uint32), allbits.astype(np.uint32) << 16)
    nan = (allbits & 0x7FFF) > 0x7F80
    back = oracle.bf16_from_f32(widened)
    assert np.array_equal(back[~nan], allbits[~nan])
    assert np.all(back[nan] == 0x7FC0)


def test_bf16_matches_reference_sources(oracle):
    ref = oracle.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    lib = oracle.lib()
    rng = np.random.default_rng(5)
    for bits in list(rng.integers(0, 2**32, 20000, dtype=np.uint64)) + [i for i, _ in BF16_CASES]:
        v = f32(int(bits))
        assert lib.or_bf16_from_f32(v) == ref.dlref_bf16_from_f32(v)


def test_mt19937_64_standard_value(oracle):
    # The C++ standard fixes the 10000th output of a default-seeded
    # std::mt19937_64 ([rand.predef]): 9981545732273789042.
    rng = oracle.MT19937_64(5489)
    for _ in range(9999):
        rng()
    assert rng() == 9981545732273789042


def test_mt19937_64_matches_std(oracle):
    ref = oracle.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    for seed in (0, 1, 42, 2**63 + 7):
        rng = oracle.MT19937_64(seed)
        values = [rng() for _ in range(700)]
        for skip in (0, 1, 311, 312, 313, 699):
            assert values[skip] == ref.dlref_mt64(seed, skip)


def _device_kat_logits(n):
    # tests/gpu/test_device.cpp:268-283
    logits = np.array([((i % 97) - 48) / 8.0 for i in range(n)], dtype=np.float32)
    logits[0] = -0.0
    if n > 1:
        logits[1] = 0.0
        logits[-1] = -np.inf
    return logits


def _ref_select(oracle, logits, mode, t, k, p, seed, draws=1):
    ref = oracle.ref()
    out = np.zeros(draws, dtype=np.uint32)
    status = ref.dlref_categorical_select(np.ascontiguousarray(logits, np.float32), len(logits), mode, t, k, p,
                                          seed, draws, out)
    return status, out


@pytest.mark.parametrize("n", [1, 513, 151936])
def test_sampler_law_matches_reference_device_kat(oracle, n):
    """The device-KAT grid of tests/gpu/test_device.cpp:285-320 run through
    the oracle's law and through the reference's own categorical.cpp."""
    if oracle.ref() is None:
        pytest.skip("oracle/_ref not built")
    logits = _device_kat_logits(n)
    for mode in (0, 1):
        for k in (0, min(n, 20)):
            for p in (0.01, 0.5, 0.95, 1.0):
                for seed in range(8):
                    t, kk, pp = (1.0, 0, 1.0) if mode == 0 else (0.6, k, p)
                    status, expected = _ref_select(oracle, logits, mode, t, kk, pp, seed)
                    assert status == 0
                    bits = oracle.MT19937_64(seed)() if mode == 1 else 0
                    st, got = oracle.categorical_bits(logits, mode, t, kk, pp, bits)
                    assert st == 0 and got == expected[0], (mode, k, p, seed)
                    if mode == 0:
                        break
                if mode == 0:
                    break
            if mode == 0:
                break


def test_sampler_law_700_draw_sequence(oracle):
    # tests/gpu/test_device.cpp:321-345: 700 draws at n=513, seed 42, T 0.6, p 0.95
    if oracle.ref() is None:
        pytest.skip("oracle/_ref not built")
    logits = _device_kat_logits(513)
    status, expected = _ref_select(oracle, logits, 1, 0.6, 0, 0.95, 42, draws=700)
    assert status == 0
    rng = oracle.MT19937_64(42)
    import ctypes as C
    for i in range(700):
        out = C.c_uint32()
        st = oracle.lib().ors_categorical_select(logits, len(logits), 1, 0.6, 0, 0.95, C.byref(rng.state),
                                                 C.byref(out))
        assert st == 0 and out.value == expected[i], i


def test_sampler_contract_cases(oracle):
    # tests/core/test_sampling.cpp:128-160 known answers
    masked = -np.inf
    logits = np.array([masked, 3.0, 3.0, 1.0], dtype=np.float32)
    assert oracle.categorical_bits(logits, 0, 1.0, 0, 1.0, 0) == (0, 1)  # greedy tie -> lowest id
    assert oracle.categorical_bits(logits, 1, 1.0, 1, 1.0, 12345)[1] == 1  # top-k keeps lowest tied id
    assert oracle.categorical_bits(logits, 1, 1.0, 0, 0.25, 2**63)[1] == 1  # nucleus keeps one
    uniform = np.zeros(4, dtype=np.float32)
    rng = oracle.MT19937_64(51)
    bits = rng()
    u = (bits >> 11) * 2.0**-53
    assert oracle.categorical_bits(uniform, 1, 1.0, 0, 0.5, bits)[1] == (0 if u < 0.5 else 1)
    bad = logits.copy()
    bad[2] = np.nan
    assert oracle.categorical_bits(bad, 0, 1.0, 0, 1.0, 0)[0] == 1
    assert oracle.categorical_bits(np.full(4, masked, np.float32), 0, 1.0, 0, 1.0, 0)[0] == 2
    for t, k, p, mode in ((0.0, 0, 1.0, 1), (1.0, 5, 1.0, 1), (1.0, 0, 0.0, 1), (0.5, 0, 1.0, 0)):
        assert oracle.categorical_bits(logits, mode, t, k, p, 0)[0] == 3


def test_sampler_distribution_contract_against_reference(oracle):
    # tests/core/test_sampling.cpp:66-108: ties, signed zeros, subnormals, masks
    if oracle.ref() is None:
        pytest.skip("oracle/_ref not built")
    gen = oracle.MT19937_64(7391)
    for size in (17, 1023, 4096):
        values = np.array([((gen() % 4001) - 2000) / 127.0 for _ in range(size)], dtype=np.float32)
        edges = [0.0, -0.0, np.float32(1e-45), -np.float32(1e-45), -np.inf, 1.0, 1.0]
        values[:7] = np.array(edges, dtype=np.float32)
        for t, k, p in ((1, 0, 1), (0.6, 0, 0.95), (2, 11, 0.7)):
            seed = gen()
            status, expected = _ref_select(oracle, values, 1, t, k, p, seed, draws=64)
            assert status == 0
            rng = oracle.MT19937_64(seed)
            for i in range(64):
                st, got = oracle.categorical_bits(values, 1, t, k, p, rng())
                assert st == 0 and got == expected[i]


def test_sampler_trace_restates_the_law(oracle):
    """The serial trace used to place boundary draws: F_n is the serial fold
    (checked against a Python left fold), G at the cutoff is within a few
    ulps of 1, a draw at G_i picks candidate i + 1 and one below picks i, and
    the glibc-exp law equals the default law."""
    gen = oracle.MT19937_64(11)
    logits = oracle.f32_from_bf16(oracle.normal_bf16(3000, 5, 77, 1.28))
    ids, fold, cumulative = oracle.categorical_trace(logits, 1.0, 0, 0.9)
    order = sorted(range(len(logits)), key=lambda i: (-float(logits[i]), i))
    assert ids.tolist() == order
    z0 = float(logits[order[0]])
    total = 0.0
    for i in order:
        total += math.exp(float(logits[i]) - z0)
    assert fold[-1] == total
    assert abs(cumulative[-1] - 1.0) < 1e-12
    c = len(cumulative)
    assert fold[c - 1] / fold[-1] >= 0.9 and fold[c - 2] / fold[-1] < 0.9
    for i in (0, c // 2, c - 2):
        u = cumulative[i]
        m = int(u * 2.0**53)
        if m * 2.0**-53 != u:
            continue
        assert oracle.categorical_bits(logits, 1, 1.0, 0, 0.9, m << 11)[1] == ids[i + 1]
        assert oracle.categorical_bits(logits, 1, 1.0, 0, 0.9, (m - 1) << 11)[1] == ids[i]
    for _ in range(20):
        bits = gen()
        assert oracle.categorical_bits_exp(logits, 1, 1.0, 0, 0.9, bits, False) == \
            oracle.categorical_bits(logits, 1, 1.0, 0, 0.9, bits)


def test_sampler_build_exp_law_agrees_off_boundary(oracle):
    """With the build's exp the law picks the same ids as with glibc exp for
    ordinary draws (they differ only on draws within ~1e-12 of a boundary)."""
    gen = oracle.MT19937_64(12)
    logits = oracle.f32_from_bf16(oracle.normal_bf16(151936, 6, 77, 1.28))
    for _ in range(16):
        bits = gen()
        assert oracle.categorical_bits_exp(logits, 1, 1.0, 0, 0.95, bits, True) == \
            oracle.categorical_bits_exp(logits, 1, 1.0, 0, 0.95, bits, False)


def _ulp64(a, b):
    ia = a.view(np.int64).copy()
    ib = b.view(np.int64).copy()
    ia[ia < 0] = np.iinfo(np.int64).min - ia[ia < 0]
    ib[ib < 0] = np.iinfo(np.int64).min - ib[ib < 0]
    return np.abs(ia - ib)


def _ulp32(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia[ia < 0] = np.iinfo(np.int32).min - ia[ia < 0]
    ib[ib < 0] = np.iinfo(np.int32).min - ib[ib < 0]
    return np.abs(ia - ib)


def test_shared_math_against_libm(oracle):
    """dl_math.h (shared by the device kernels and the contract mirror) is
    faithful against an independent libm: exp/expf/pow within 1-2 ulp, log
    and sin/cos within 2 ulp on the ranges the kernels use."""
    lib = oracle.lib()
    rng = np.random.default_rng(11)
    x = np.concatenate([-rng.random(200000) * 745.0, rng.random(50000) * 709.0, [0.0, -0.0, -745.0, 709.7]])
    y = np.empty_like(x)
    lib.or_math_exp(x, y, x.size)
    assert _ulp64(y, np.exp(x)).max() <= 1
    xf = (-rng.random(200000) * 104.0).astype(np.float32)
    yf = np.empty_like(xf)
    lib.or_math_expf(xf, yf, xf.size)
    assert _ulp32(yf, np.exp(xf.astype(np.float64)).astype(np.float32)).max() <= 1
    u = np.concatenate([rng.random(200000), [1.0, 2.0**-1074, 0.5, 2.0**-53]])
    lg = np.empty_like(u)
    lib.or_math_log(u, lg, u.size)
    assert _ulp64(lg[u != 1.0], np.log(u[u != 1.0])).max() <= 2
    assert lg[u == 1.0][0] == 0.0
    a = (rng.random(200000) - 0.5) * 20000.0
    s = np.empty_like(a)
    c = np.empty_like(a)
    lib.or_math_sincos(a, s, c, a.size)
    ok = np.abs(np.sin(a)) > 1e-3
    assert _ulp64(s[ok], np.sin(a[ok])).max() <= 2
    ok = np.abs(np.cos(a)) > 1e-3
    assert _ulp64(c[ok], np.cos(a[ok])).max() <= 2
    e = np.arange(64, dtype=np.float64) / 64.0
    b = np.full_like(e, 1e6)
    pw = np.empty_like(e)
    lib.or_math_pow(b, e, pw, e.size)
    assert np.max(np.abs(pw / np.power(1e6, e) - 1.0)) < 1e-14
    assert pw[0] == 1.0


def test_rope_angles_closed_forms(oracle):
    lib = oracle.lib()
    cosv = np.empty(64, np.float32)
    sinv = np.empty(64, np.float32)
    lib.orc_rope_angles(0, 128, 1e6, cosv, sinv)  # position 0 is the identity rotation
    assert np.all(cosv == 1.0) and np.all(sinv == 0.0)
    for pos in (1, 511, 4093, 8191):
        lib.orc_rope_angles(pos, 128, 1e6, cosv, sinv)
        exponent = ((np.arange(64) * 2).astype(np.float32) / np.float32(128)).astype(np.float64)
        f = (1.0 / np.power(np.float64(1e6), exponent)).astype(np.float32)
        ang = (np.float32(pos) * f).astype(np.float32).astype(np.float64)
        # BF16-rounded cos/sin: within half a BF16 ulp (plus tiny slack) of the true value
        for got, want in ((cosv, np.cos(ang)), (sinv, np.sin(ang))):
            tol = np.maximum(np.abs(want), 2.0**-126) * 2.0**-8 * 1.01
            assert np.all(np.abs(got - want) <= tol)
