"""GPU checks of the exact chunked prompt pass (dl_plan_prefill).

The pass runs the prompt positions in chunks of up to 512 positions: the
projections of a chunk of 16 positions or more as many-row exact GEMMs,
fewer through the batched decode GEMVs; from 1536 keys the attention of a
chunk of 8 rows or more shares key tiles and V rows across rows.  Parity is
bit-exact: for every case the caches, the
token streams and the last logits equal those of a plan that consumes the
same prompt one position per step through the token loop (itself bit-exact
with the CPU contract mirror, tests/test_gpu_model.py).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 9151


def qwen_config(layers, vocab=151936):
    from dolittle_amd.qwen3 import Qwen3Config
    return Qwen3Config(layers=layers, vocab=vocab)


@pytest.fixture(scope="module")
def model2(device, queue):
    from dolittle_amd.qwen3 import Qwen3Model
    model = Qwen3Model(device, queue, qwen_config(layers=2))
    model.fill_synthetic(SEED, 0.02)
    return model


@pytest.fixture(scope="module")
def model1(device, queue):
    from dolittle_amd.qwen3 import Qwen3Model
    model = Qwen3Model(device, queue, qwen_config(layers=1, vocab=2048))
    model.fill_synthetic(SEED + 1, 0.02)
    return model


def run_pair(model, prompt, max_new, batch=1, capacity=64, setup=None, sampling=None, seeds=None):
    """(exact prefill + generate, generate only): tokens, results, plans."""
    from dolittle_amd.qwen3 import Plan
    out = []
    for exact in (True, False):
        plan = Plan(model, batch=batch, capacity=capacity)
        if setup:
            setup(plan)
        if exact:
            plan.prefill(prompt)
        plan.generate(prompt, max_new, sampling, seeds)
        tokens, results = plan.collect()
        out.append((tokens, results, plan))
    return out


def assert_same(model, a, b, prompt_len, batch=1):
    (ta, ra, pa), (tb, rb, pb) = a, b
    assert ta.tolist() == tb.tolist()
    for x, y in zip(ra, rb):
        assert x["generated"] == y["generated"] and x["position"] == y["position"]
    for s in range(batch):
        assert np.array_equal(pa.logits(s), pb.logits(s)), s
        for layer in range(model.config.layers):
            ka, va = pa.read_cache(layer, 0, prompt_len, s)
            kb, vb = pb.read_cache(layer, 0, prompt_len, s)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), (s, layer)


@pytest.mark.parametrize("length", [1, 2, 9, 12, 17, 30])
def test_exact_prefill_equals_token_loop(model2, length):
    """Chunks of 8 with every remainder (1, 8 + 3, 8 + 8, ...), and prompts
    too short to need a pass."""
    prompt = [int(t) for t in np.random.default_rng(length).integers(0, 151936, length)]
    a, b = run_pair(model2, prompt, 6, capacity=48)
    assert_same(model2, a, b, length + 6)


def test_exact_prefill_across_the_fused_attention_limit(model1):
    """A 1600-id prompt: chunks below 1536 keys use the one-kernel attention,
    the later ones the split long-context kernels."""
    prompt = [int(t) for t in np.random.default_rng(77).integers(0, 2048, 1600)]
    a, b = run_pair(model1, prompt, 4, capacity=1664)
    assert_same(model1, a, b, 1604)


@pytest.mark.parametrize("length", [1545, 1551, 1561, 1541])
def test_exact_prefill_chunk_remainders_past_the_fused_limit(model1, length):
    """Prompts whose last chunk lies past 1536 keys with 8, 14, 24 and 4
    rows: the row-block attention with whole and partial last blocks (8, 14
    and 24 rows), the batched GEMVs (8 and 14 rows), the many-row GEMM (24
    rows) and the one-row-per-workgroup kernels (4 rows), each row at its
    own split point."""
    prompt = [int(t) for t in np.random.default_rng(length).integers(0, 2048, length)]
    a, b = run_pair(model1, prompt, 3, capacity=1728)
    assert_same(model1, a, b, length + 3)


def test_exact_prefill_batch_with_capture_and_steering(model2, device, queue):
    """Batch 2 with block-1 capture and steering of sequence 1 (each sequence
    gets its own pass) and batch 3 without hooks (one pass, copied)."""
    from dolittle_amd.qwen3 import SamplingSettings
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, 151936, 19)]
    vec = (np.random.default_rng(6).standard_normal(4096) * 0.5).astype(np.float32)

    def hooks(plan):
        plan.set_capture(1)
        plan.set_steering(1, 1, vec)

    a, b = run_pair(model2, prompt, 5, batch=2, capacity=40, setup=hooks)
    assert_same(model2, a, b, 24, batch=2)
    assert np.array_equal(a[2].read_capture(0, 0, 23), b[2].read_capture(0, 0, 23))
    assert np.array_equal(a[2].read_capture(1, 0, 23), b[2].read_capture(1, 0, 23))
    settings = SamplingSettings("categorical", 1.0, 0, 0.95)
    a, b = run_pair(model2, prompt, 5, batch=3, capacity=40, sampling=settings, seeds=[1, 2, 3])
    assert_same(model2, a, b, 24, batch=3)


def test_exact_prefill_with_embedding_override(model2):
    """A replaced embedding row inside the prompt (BASELINE config 5's
    injection slot) is applied by the pass exactly as by the loop."""
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, 151936, 14)]
    row = (np.random.default_rng(9).standard_normal(4096) * 40.0).astype(np.float32)
    bits = ((row.view(np.uint32).astype(np.uint64) + 0x7FFF + ((row.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    a, b = run_pair(model2, prompt, 4, batch=2, capacity=32,
                    setup=lambda plan: plan.set_embedding_override(6, bits, 0b10))
    assert_same(model2, a, b, 18, batch=2)


@pytest.mark.parametrize("change", ["steering", "capture", "override"])
def test_hooks_set_after_a_prefill_are_not_skipped(model2, change):
    """A prefill followed by a hook change (steering of sequence 1, a capture
    layer, an embedding override) and then generate() with the same prompt
    must not resume over caches built without the hook: the result equals a
    plan that never prefilled, captures included."""
    from dolittle_amd.qwen3 import Plan
    p = [int(t) for t in np.random.default_rng(61).integers(0, 151936, 20)]
    new, layer = 4, 1
    v = np.random.default_rng(62).standard_normal(4096).astype(np.float32)
    row = np.random.default_rng(63).integers(0, 1 << 14, 4096).astype(np.uint16)

    def hook(plan):
        if change == "steering":
            plan.set_steering(1, layer, v)
        elif change == "capture":
            plan.set_capture(layer)
        else:
            plan.set_embedding_override(7, row, 0b10)

    out = []
    for prefill in (True, False):
        plan = Plan(model2, batch=2, capacity=32)
        if prefill:
            plan.prefill(p)
        hook(plan)
        plan.generate(p, new)
        tokens, results = plan.collect()
        out.append((tokens, results, plan))
    (ta, ra, pa), (tb, rb, pb) = out
    assert ta.tolist() == tb.tolist()
    for s in range(2):
        assert np.array_equal(pa.logits(s), pb.logits(s)), s
        assert ra[s]["position"] == rb[s]["position"] == len(p) + new
    if change == "capture":
        for s in range(2):
            assert np.array_equal(pa.read_capture(s, 0, len(p) + new), pb.read_capture(s, 0, len(p) + new))
    else:
        # The hook reached sequence 1 only.
        assert ta[0].tolist() != ta[1].tolist() or not np.array_equal(pa.logits(0), pa.logits(1))


def test_wrapped_ranges_are_length_errors(model2):
    """A first position near 2^64 with a small count wraps first + count
    around; the range checks reject it before any copy or launch."""
    from dolittle_amd import _lib
    from dolittle_amd.qwen3 import Plan
    plan = Plan(model2, batch=1, capacity=32)
    plan.set_capture(0)
    huge = (1 << 64) - 2
    buf = np.zeros(4 * 1024 * 4, np.uint16)
    ptr = buf.ctypes.data_as(_lib.u16p)
    with pytest.raises(_lib.LengthError):
        _lib.call("dl_plan_read_cache", plan.handle, 0, 0, huge, 4, ptr, ptr)
    with pytest.raises(_lib.LengthError):
        _lib.call("dl_plan_write_cache", plan.handle, 0, 0, huge, 4, ptr, ptr)
    with pytest.raises(_lib.LengthError):
        _lib.call("dl_plan_read_capture", plan.handle, 0, huge, 4, ptr)
    plan.prefill([1, 2, 3, 4, 5])
    with pytest.raises(_lib.LengthError):
        _lib.call("dl_plan_read_prefill_hidden", plan.handle, huge, 4, ptr)


def test_scratch_follows_the_longest_chunk_and_is_counted(model1):
    """The pass's row buffers and score/probability rows are sized to the
    longest chunk a pass has needed (at most 512 rows), not to 512 rows up
    front, and dl_plan_device_bytes counts them; a shorter pass after a
    longer one reuses the larger buffers and stays bit-exact."""
    from dolittle_amd.qwen3 import Plan
    cfg = model1.config
    cap = 640
    plan = Plan(model1, batch=1, capacity=cap)
    base = plan.device_bytes()
    rng = np.random.default_rng(77)
    short = [int(t) for t in rng.integers(0, cfg.vocab, 10)]
    long = [int(t) for t in rng.integers(0, cfg.vocab, 600)]
    qw, kw = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim

    def scratch(rows):
        per_row = 2 * (3 * cfg.hidden + 2 * qw + kw + cfg.ffn) + 2 * 4 * cfg.q_heads * cap
        return rows * per_row

    plan.prefill(short)
    grown = plan.device_bytes() - base
    assert scratch(9) <= grown <= scratch(9) + 4096, (grown, scratch(9))
    plan.prefill(long)
    grown = plan.device_bytes() - base
    assert scratch(512) <= grown <= scratch(512) + 4096, (grown, scratch(512))
    plan.prefill(short)
    assert plan.device_bytes() - base == grown
    plan.generate(short, 4)
    tokens, _ = plan.collect()
    loop = Plan(model1, batch=1, capacity=cap)
    loop.generate(short, 4)
    want, _ = loop.collect()
    assert tokens.tolist() == want.tolist()
    assert np.array_equal(plan.logits(0), loop.logits(0))
