"""dl_sample_noalloc (the allocation-free selection) against
dl_sampler_submit (the selection over an allocated sampler workspace), both
called through the C ABI: two calls in a row, the second over a smaller
vocabulary, for greedy and top-p categorical settings; the results must be
identical ({token, status}, bit for bit, as the sampler tests hold
dl_sampler_submit to the host law).  The second call also checks that the
shared static scratch keeps no state from the first (its histogram is
cleared on every call)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def logits_row(oracle, n, seed):
    """Random-model logits N(0, 1.28) in BF16 with ties (the interpretation
    sampling workload's shape), plus repeated values to exercise equal-key
    ordering."""
    x = np.random.default_rng(seed).standard_normal(n).astype(np.float32) * np.float32(1.28)
    x[::7] = x[0]
    return oracle.bf16_from_f32(x)


def run_pair(lib, device, queue, rows, result, n, bits16, settings, draw):
    from dolittle_amd import _lib
    from dolittle_amd.sampling import DeviceCategorical
    queue.write(rows, np.ascontiguousarray(bits16, np.uint16))
    s = DeviceCategorical(device, queue, n)
    s.submit(rows, settings, draw)
    want = s.result()
    s.close()
    sc = settings.ctype()
    _lib.call("dl_sample_noalloc", queue.handle, rows.ptr(), n * 2, n, C.byref(sc), draw,
              C.cast(result.ptr(), _lib.u32p))
    got = queue.read(result, np.uint32, 2)
    return want, (int(got[0]), int(got[1]))


@pytest.mark.parametrize("mode", ["greedy", "top_p"])
def test_noalloc_selection_equals_sampler_submit(device, queue, oracle, mode):
    from dolittle_amd import _lib
    from dolittle_amd.sampling import Settings
    lib = _lib.load()
    settings = Settings() if mode == "greedy" else Settings("categorical", 1.0, 0, 0.95)
    rows = device.allocate(151936 * 2)
    result = device.allocate(8)
    draws = [0x9E3779B97F4A7C15, 0x0123456789ABCDEF]
    for call, (n, seed) in enumerate(((151936, 1), (513, 2))):
        bits16 = logits_row(oracle, n, seed + (10 if mode == "top_p" else 0))
        want, got = run_pair(lib, device, queue, rows, result, n, bits16, settings, draws[call])
        print(f"{mode} call {call} n={n}: sampler {want}, no-alloc {got}")
        assert got == want, (call, n)
        assert got[1] == 0
