"""GPU parity of the NLA device objects (dl_injection_*, dl_direction_*,
dl_intervention_*; injection.cu:49-98, steering.cu:69-159) with the oracle
restatement (oracle/nla.c), bit for bit, through the C ABI and the Python
mirror (dolittle_amd/interventions.py): FP32 and BF16 storage, the
reference's status rules, the chunk selection by device position and the
exactly-once count."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def up(device, queue, array):
    return device.upload_array(queue, np.ascontiguousarray(array))


def region(buf, nbytes, offset=0):
    from dolittle_amd.interventions import Region
    return Region(buf, offset, nbytes)


def source(oracle, width, seed, bf16, scale=3.0):
    x = (np.random.default_rng(seed).standard_normal(width) * scale).astype(np.float32)
    return oracle.bf16_from_f32(x) if bf16 else x


@pytest.mark.parametrize("width", [1, 7, 1000, 4096])
@pytest.mark.parametrize("src_bf16,out_bf16", [(True, True), (True, False), (False, True), (False, False)])
def test_injection_matches_oracle(device, queue, oracle, width, src_bf16, out_bf16):
    from dolittle_amd.interventions import DeviceInjection
    x = source(oracle, width, width * 3 + src_bf16, src_bf16)
    buf = up(device, queue, x)
    inj = DeviceInjection(device, queue, region(buf, x.nbytes), "bfloat16" if src_bf16 else "float32",
                          "bfloat16" if out_bf16 else "float32", width, 150.0)
    inj.submit()
    queue.drain()
    status, norm, out = oracle.inject(x, src_bf16, out_bf16, 150.0)
    raw = queue.read(inj.storage, np.uint8, inj.storage.nbytes)
    assert raw[4:8].view(np.uint32)[0] == status == 0
    assert raw[0:4].view(np.float32)[0] == norm
    got = raw[8:].view(np.uint16 if out_bf16 else np.float32)
    assert np.array_equal(got, out)
    assert np.array_equal(queue.read(buf, x.dtype, width), x)  # source unchanged


def test_injection_statuses(device, queue, oracle):
    from dolittle_amd import _lib
    import ctypes as C
    cases = []
    zero = np.zeros(64, np.float32)
    nan = np.ones(64, np.float32)
    nan[9] = np.nan
    one = np.zeros(64, np.float32)
    one[0] = 1.0
    cases = [(zero, 150.0, True), (nan, 150.0, True), (one, 3.4e38, True), (one, 3.4e38, False)]
    for x, scale, out_bf16 in cases:
        bx = up(device, queue, x)
        nbytes = C.c_uint64()
        _lib.call("dl_injection_bytes", 64, 1 if out_bf16 else 2, C.byref(nbytes))
        st = device.allocate(nbytes.value, 4)
        queue.write(st, np.zeros(nbytes.value, np.uint8))
        _lib.call("dl_injection_submit", queue.handle, bx.ptr(), 2, 1 if out_bf16 else 2, 64, C.c_float(scale),
                  st.ptr())
        queue.drain()
        status, norm, out = oracle.inject(x, False, out_bf16, scale)
        raw = queue.read(st, np.uint8, nbytes.value)
        assert raw[4:8].view(np.uint32)[0] == status, (scale, out_bf16)
        if not np.isnan(norm):
            assert raw[0:4].view(np.float32)[0] == norm
        assert np.array_equal(raw[8:].view(np.uint16 if out_bf16 else np.float32), out)
    with pytest.raises(Exception):
        _lib.call("dl_injection_submit", queue.handle, bx.ptr(), 2, 1, 64, C.c_float(0.0), st.ptr())


@pytest.mark.parametrize("width,bf16", [(4096, True), (4096, False), (33, True)])
def test_direction_matches_oracle(device, queue, oracle, width, bf16):
    from dolittle_amd.interventions import DeviceDirection
    a, b = source(oracle, width, 1, bf16), source(oracle, width, 2, bf16)
    ba, bb = up(device, queue, a), up(device, queue, b)
    d = DeviceDirection(device, queue, region(ba, a.nbytes), region(bb, b.nbytes),
                        "bfloat16" if bf16 else "float32", width)
    d.submit()
    u = d.finish()
    status, expect = oracle.direction(a, b, bf16)
    assert status == 0
    assert np.array_equal(queue.read(u.owner, np.float32, width, u.offset), expect)
    same = DeviceDirection(device, queue, region(ba, a.nbytes), region(ba, a.nbytes),
                           "bfloat16" if bf16 else "float32", width)
    same.submit()
    with pytest.raises(ValueError):
        same.finish()


@pytest.mark.parametrize("bf16", [True, False])
def test_intervention_matches_oracle(device, queue, oracle, bf16):
    from dolittle_amd.interventions import DeviceIntervention
    rows, width = 8, 4096
    h = source(oracle, rows * width, 11, bf16)
    _, u = oracle.direction(source(oracle, width, 12, bf16), source(oracle, width, 13, bf16), bf16)
    bh, bu = up(device, queue, h), up(device, queue, u)
    pos = up(device, queue, np.array([40], np.uint64))
    iv = DeviceIntervention(device, queue, region(bu, u.nbytes), width, 43, 0.37, "bfloat16" if bf16 else "float32")
    iv.initialize()
    iv.submit(region(bh, h.nbytes), region(pos, 8), rows)
    queue.drain()
    state = np.zeros(2, np.uint32)
    expect = h.copy()
    assert oracle.intervene(expect, bf16, rows, width, u, 40, 43, 0.37, state)
    assert np.array_equal(queue.read(bh, h.dtype, h.size), expect)
    assert np.array_equal(queue.read(iv.state, np.uint32, 2), state) and state.tolist() == [0, 1]
    # The same chunk again: a second application is invalid, the row stays.
    iv.submit(region(bh, h.nbytes), region(pos, 8), rows)
    queue.drain()
    assert oracle.intervene(expect, bf16, rows, width, u, 40, 43, 0.37, state)
    assert np.array_equal(queue.read(bh, h.dtype, h.size), expect)
    assert queue.read(iv.state, np.uint32, 2).tolist() == state.tolist() == [1, 2]
    # A chunk that does not hold position 43 changes nothing.
    iv.initialize()
    queue.write(pos, np.array([44], np.uint64))
    iv.submit(region(bh, h.nbytes), region(pos, 8), rows)
    queue.drain()
    assert np.array_equal(queue.read(bh, h.dtype, h.size), expect)
    assert queue.read(iv.state, np.uint32, 2).tolist() == [0, 0]


def test_intervention_overflow_latches(device, queue, oracle):
    from dolittle_amd.interventions import DeviceIntervention
    width = 256
    h = oracle.bf16_from_f32(np.full(width, 1e37, np.float32))
    u = np.full(width, 1.0 / 16.0, np.float32)
    bh, bu = up(device, queue, h), up(device, queue, u)
    pos = up(device, queue, np.array([0], np.uint64))
    iv = DeviceIntervention(device, queue, region(bu, u.nbytes), width, 0, 100.0, "bfloat16")
    iv.initialize()
    iv.submit(region(bh, h.nbytes), region(pos, 8), 1)
    queue.drain()
    state = np.zeros(2, np.uint32)
    expect = h.copy()
    oracle.intervene(expect, True, 1, width, u, 0, 0, 100.0, state)
    assert state[0] == 1
    assert queue.read(iv.state, np.uint32, 2).tolist() == state.tolist()
    assert np.array_equal(queue.read(bh, np.uint16, width), expect)
