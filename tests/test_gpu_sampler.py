"""GPU parity of the device sampler (DeviceCategorical) with the host law.

- the reference's device selection grid (tests/gpu/test_device.cpp:268-345):
  n in {1, 513, 151936}, logits (i mod 97 - 48) / 8 with -0, +0 and -inf,
  greedy and categorical (T 0.6, k in {0, 20}, p in {0.01, 0.5, 0.95, 1}),
  draws from MT19937-64 seeds 0..7, and the 700-draw live stream;
- random-model logits (N(0, 1.28) in BF16, 151,936 values, T 1, top-p 0.95,
  the interpretation-sampling workload): ids bit-exact with the host law;
- draws and top-p values placed exactly on the law's boundaries, where the
  device must fall back to its serial replay, and the forced replay;
- rejection (NaN/+inf, all -inf), ties and signed zeros, the terminal latch.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V = 151936


def kat_logits(n):
    x = np.array([(i % 97 - 48) / 8.0 for i in range(n)], np.float32)
    x[0] = -0.0
    if n > 1:
        x[1] = 0.0
        x[-1] = -np.inf
    return x


def bf16_bits(oracle, x):
    return oracle.bf16_from_f32(np.ascontiguousarray(x, np.float32))


@pytest.fixture(scope="module")
def rows(device):
    return device.allocate(V * 2 * 4)


def sampler(device, queue, n):
    from dolittle_amd.sampling import DeviceCategorical
    return DeviceCategorical(device, queue, n)


def select(s, queue, buf, bits16, settings, draw):
    queue.write(buf, np.ascontiguousarray(bits16, np.uint16))
    s.submit(buf, settings, draw)
    return s.result()


@pytest.mark.parametrize("n", [1, 513, V])
def test_reference_device_grid(device, queue, oracle, rows, n):
    from dolittle_amd.sampling import Settings
    logits = kat_logits(n)
    bits16 = bf16_bits(oracle, logits)
    assert np.array_equal(oracle.f32_from_bf16(bits16), logits)
    s = sampler(device, queue, n)
    queue.write(rows, bits16)
    checked = 0
    for mode in ("greedy", "categorical"):
        for k in (0, min(n, 20)):
            for p in (0.01, 0.5, 0.95, 1.0):
                for seed in range(8):
                    if mode == "greedy":
                        settings = Settings("greedy", 1.0, 0, 1.0)
                    else:
                        settings = Settings("categorical", 0.6, k, p)
                    draw = oracle.MT19937_64(seed)() if mode == "categorical" else 0
                    status, want = oracle.categorical_bits(logits, 0 if mode == "greedy" else 1,
                                                           settings.temperature, settings.top_k,
                                                           settings.top_p, draw)
                    assert status == 0
                    s.submit(rows, settings, draw)
                    assert s.result() == (want, 0), (mode, k, p, seed)
                    checked += 1
    assert checked == 128


def test_live_stream_700_draws(device, queue, oracle, rows):
    """start + submit_next crosses two MT19937-64 twists (312 words each)."""
    from dolittle_amd.sampling import Settings
    n = 513
    logits = kat_logits(n)
    s = sampler(device, queue, n)
    queue.write(rows, bf16_bits(oracle, logits))
    settings = Settings("categorical", 0.6, 0, 0.95)
    s.start(settings, 42)
    rng = oracle.MT19937_64(42)
    for i in range(700):
        status, want = oracle.categorical_bits(logits, 1, 0.6, 0, 0.95, rng())
        s.submit_next(rows)
        assert s.result() == (want, 0), i


def model_logits(oracle, seed, n=V, scale=1.28):
    bits16 = oracle.normal_bf16(n, seed, 77, scale)
    return bits16, oracle.f32_from_bf16(bits16)


@pytest.mark.parametrize("temperature,top_k,top_p", [(1.0, 0, 0.95), (0.7, 0, 0.9), (1.0, 50, 1.0),
                                                     (1.3, 0, 1.0)])
def test_random_model_rows(device, queue, oracle, rows, temperature, top_k, top_p):
    from dolittle_amd.sampling import Settings
    s = sampler(device, queue, V)
    settings = Settings("categorical", temperature, top_k, top_p)
    for r in range(4):
        bits16, logits = model_logits(oracle, 1000 + r)
        queue.write(rows, bits16)
        rng = oracle.MT19937_64(r)
        for _ in range(24):
            draw = rng()
            status, want = oracle.categorical_bits(logits, 1, temperature, top_k, top_p, draw)
            assert status == 0
            s.submit(rows, settings, draw)
            assert s.result() == (want, 0)
    assert s.exact_replays() <= 2


def bits_for(u):
    """Draw bits whose unit value (x >> 11) * 2^-53 is the largest <= u."""
    m = int(np.floor(np.float64(u) * 2.0 ** 53))
    m = min(max(m, 0), 2 ** 53 - 1)
    return m << 11


@pytest.mark.parametrize("n,temperature,top_p", [(513, 0.6, 0.95), (V, 1.0, 0.95), (4096, 1.0, 1.0)])
def test_boundary_draws_take_the_serial_replay(device, queue, oracle, rows, n, temperature, top_p):
    """u placed on G_i (and one unit below) lies inside every error band: the
    device decides by its serial replay and matches the law bit for bit."""
    from dolittle_amd.sampling import Settings
    if n == 513:
        logits = kat_logits(n)
        bits16 = bf16_bits(oracle, logits)
    else:
        bits16, logits = model_logits(oracle, 2024 + n, n)
    s = sampler(device, queue, n)
    queue.write(rows, bits16)
    ids, fold, cumulative = oracle.categorical_trace(logits, temperature, 0, top_p, build_exp=True)
    settings = Settings("categorical", temperature, 0, top_p)
    picks = sorted({1, 2, len(cumulative) // 3, len(cumulative) // 2, len(cumulative) - 2})
    before = s.exact_replays()
    cases = 0
    for i in picks:
        if i < 0 or i >= len(cumulative) or cumulative[i] >= 1.0:
            continue
        base = bits_for(cumulative[i])
        for draw in (base, max(base - (1 << 11), 0), base + (1 << 11)):
            status, want = oracle.categorical_bits_exp(logits, 1, temperature, 0, top_p, draw, True)
            assert status == 0
            s.submit(rows, settings, draw)
            assert s.result() == (want, 0), (i, draw)
            cases += 1
    assert cases >= 6
    assert s.exact_replays() - before >= cases // 3


def test_boundary_top_p_takes_the_serial_replay(device, queue, oracle, rows):
    """top_p = F_k / F_n exactly puts the cutoff on the band."""
    from dolittle_amd.sampling import Settings
    n = 4096
    bits16, logits = model_logits(oracle, 99, n)
    s = sampler(device, queue, n)
    queue.write(rows, bits16)
    ids, fold, _ = oracle.categorical_trace(logits, 1.0, 0, 1.0, build_exp=True)
    before = s.exact_replays()
    for k in (5, n // 2, n - 10):
        p = float(np.float64(fold[k - 1]) / np.float64(fold[-1]))
        settings = Settings("categorical", 1.0, 0, p)
        _, _, cumulative = oracle.categorical_trace(logits, 1.0, 0, p, build_exp=True)
        draw = bits_for(0.999999) if len(cumulative) else 0
        status, want = oracle.categorical_bits_exp(logits, 1, 1.0, 0, p, draw, True)
        s.submit(rows, settings, draw)
        assert s.result() == (want, 0), k
    assert s.exact_replays() > before


def test_forced_replay_equals_law(device, queue, oracle, rows):
    from dolittle_amd.sampling import Settings
    s = sampler(device, queue, V)
    s.set_exact(True)
    bits16, logits = model_logits(oracle, 5)
    queue.write(rows, bits16)
    rng = oracle.MT19937_64(3)
    for top_k, top_p in ((0, 0.95), (20, 0.5), (0, 1.0)):
        settings = Settings("categorical", 1.0, top_k, top_p)
        for _ in range(3):
            draw = rng()
            status, want = oracle.categorical_bits_exp(logits, 1, 1.0, top_k, top_p, draw, True)
            s.submit(rows, settings, draw)
            assert s.result() == (want, 0)
    assert s.exact_replays() == 9


def test_rejection_ties_and_signed_zeros(device, queue, oracle, rows):
    from dolittle_amd.sampling import Settings
    n = 1000
    s = sampler(device, queue, n)
    greedy = Settings("greedy", 1.0, 0, 1.0)
    cat = Settings("categorical", 1.0, 0, 1.0)
    x = np.full(n, -np.inf, np.float32)
    for settings in (greedy, cat):
        assert select(s, queue, rows, bf16_bits(oracle, x), settings, 0)[1] == 2
    for bad in (np.nan, np.inf):
        y = np.zeros(n, np.float32)
        y[n // 2] = bad
        for settings in (greedy, cat):
            assert select(s, queue, rows, bf16_bits(oracle, y), settings, 0) == (0, 1)
    z = np.full(n, -1.0, np.float32)
    z[700], z[300] = 0.0, -0.0
    assert select(s, queue, rows, bf16_bits(oracle, z), greedy, 0) == (300, 0)
    # Equal weights: the draw walks ids in ascending order within a value.
    t = np.zeros(n, np.float32)
    for draw in (0, bits_for(0.5), bits_for(0.999)):
        status, want = oracle.categorical_bits(t, 1, 1.0, 0, 1.0, draw)
        assert select(s, queue, rows, bf16_bits(oracle, t), cat, draw) == (want, 0)


def test_settings_and_shape_validation(device, queue, oracle, rows):
    from dolittle_amd import InvalidArgument, LengthError
    from dolittle_amd.sampling import DeviceCategorical, Settings
    s = sampler(device, queue, 100)
    with pytest.raises(InvalidArgument):
        s.submit(rows, Settings("categorical", 0.0, 0, 0.9), 0)
    with pytest.raises(InvalidArgument):
        s.submit(rows, Settings("categorical", 1.0, 101, 0.9), 0)
    with pytest.raises(InvalidArgument):
        s.submit(rows, Settings("greedy", 0.5, 0, 1.0), 0)
    with pytest.raises(InvalidArgument):
        s.current_token_address()
    with pytest.raises(InvalidArgument):
        s.submit_next(rows)
    with pytest.raises(LengthError):
        DeviceCategorical(device, queue, 100, budget=1000)
    with pytest.raises(InvalidArgument):
        DeviceCategorical(device, queue, 100, dtype="f32")
    with pytest.raises(InvalidArgument):
        DeviceCategorical(device, queue, 0)


def test_terminal_latch_freezes_result(device, queue, oracle, rows):
    """A stop id latches the stream: later selections repeat the stopped
    result and draw nothing (sampling.cu commit_selection)."""
    from dolittle_amd.sampling import Settings
    n = 513
    logits = kat_logits(n)
    s = sampler(device, queue, n)
    queue.write(rows, bf16_bits(oracle, logits))
    settings = Settings("categorical", 0.6, 0, 0.95)
    rng = oracle.MT19937_64(7)
    stream = [oracle.categorical_bits(logits, 1, 0.6, 0, 0.95, rng())[1] for _ in range(6)]
    stop = stream[3]
    s.start(settings, 7, [stop])
    first = stream.index(stop)
    got = []
    for _ in range(6):
        s.submit_next(rows)
        got.append(s.result()[0])
    assert got[: first + 1] == stream[: first + 1]
    assert all(t == stop for t in got[first:])
    assert s.current_token_address() == s.result_address()
    assert s.terminal_address() != 0
    with pytest.raises(Exception):
        s.start(settings, 7, [])
