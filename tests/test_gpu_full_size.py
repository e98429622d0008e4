"""Size-independent properties at the BASELINE sizes: the full 36-block
Qwen3-8B architecture (tied 151,936-row LM head, seeded synthetic weights),
where the CPU mirror is too slow to run the whole model.  The smaller tests
pin every kernel to the mirror bit for bit; these check that the composed
loop keeps the properties the reference's loop has at full size:
- a sequence's greedy tokens and logits do not depend on its batch (configs
  2, 4, 5 shapes), also with block-24 capture and steering of one sequence;
- the exact chunked prompt pass leaves the loop exactly where consuming the
  prompt one position per step does (config 3's path, at a 600-id prompt
  that crosses the 512-key prefetch and the 64-key cache tiles);
- each sequence of a batch-8 top-p run draws the same ids as that sequence
  run alone with its seed (config 5)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full_model(device, queue):
    from dolittle_amd.qwen3 import Qwen3Config, Qwen3Model
    model = Qwen3Model(device, queue, Qwen3Config())
    model.fill_synthetic(20261201, 0.02)
    return model


def prompt(seed, n):
    return [int(t) for t in np.random.default_rng(seed).integers(0, 151936, n)]


def test_batch_invariance_full_size(full_model):
    from dolittle_amd.qwen3 import Plan
    p, new = prompt(1, 40), 12
    one = Plan(full_model, batch=1, capacity=64)
    one.generate(p, new)
    want, _ = one.collect()
    logits = one.logits(0)
    for batch in (2, 8):
        plan = Plan(full_model, batch=batch, capacity=64)
        plan.generate(p, new)
        got, results = plan.collect()
        for seq in range(batch):
            assert results[seq]["generated"] == new and results[seq]["status"] == 0
            assert got[seq].tolist() == want[0].tolist(), (batch, seq)
            assert np.array_equal(plan.logits(seq), logits), (batch, seq)


def test_capture_and_steering_full_size(full_model):
    """Config 4 semantics: batch 2, block-24 capture, sequence 1 steered at
    block 24.  Sequence 0 equals an unhooked batch-1 run; sequence 1 equals
    a batch-1 run steered the same way, captures included."""
    from dolittle_amd.qwen3 import Plan
    p, new, layer = prompt(2, 32), 8, 24
    rng = np.random.default_rng(3)
    v = rng.standard_normal(4096).astype(np.float32)
    v = (v / np.float32(np.linalg.norm(v.astype(np.float64)))).astype(np.float32) * np.float32(8.0)
    consumed = len(p) + new
    plain = Plan(full_model, batch=1, capacity=64)
    plain.set_capture(layer)
    plain.generate(p, new)
    plain_tokens, _ = plain.collect()
    plain_capture = plain.read_capture(0, 0, consumed)
    steered = Plan(full_model, batch=1, capacity=64)
    steered.set_capture(layer)
    steered.set_steering(0, layer, v)
    steered.generate(p, new)
    steered_tokens, _ = steered.collect()
    steered_capture = steered.read_capture(0, 0, consumed)
    both = Plan(full_model, batch=2, capacity=64)
    both.set_capture(layer)
    both.set_steering(1, layer, v)
    both.generate(p, new)
    tokens, results = both.collect()
    assert tokens[0].tolist() == plain_tokens[0].tolist()
    assert tokens[1].tolist() == steered_tokens[0].tolist()
    assert np.array_equal(both.read_capture(0, 0, consumed), plain_capture)
    assert np.array_equal(both.read_capture(1, 0, consumed), steered_capture)
    assert not np.array_equal(plain_capture, steered_capture)


def test_capture_and_steering_two_rows_past_1k_keys(full_model):
    """The same semantics at 1100-1106 keys, where a step of one or two rows
    runs QKV, attention and O as one launch (below 1536 keys) and each
    attention workgroup reads its own row's cache over several 64-key
    blocks: batch 2 with sequence 1 steered at block 24 equals the two
    batch-1 runs (tokens, last logits, every captured block-24 row)."""
    from dolittle_amd.qwen3 import Plan
    p, new, layer = prompt(11, 1100), 6, 24
    rng = np.random.default_rng(12)
    v = rng.standard_normal(4096).astype(np.float32)
    v = (v / np.float32(np.linalg.norm(v.astype(np.float64)))).astype(np.float32) * np.float32(8.0)
    consumed, cap = len(p) + new, len(p) + new + 1

    def run(batch, steer_seq):
        plan = Plan(full_model, batch=batch, capacity=cap)
        plan.set_capture(layer)
        if steer_seq is not None:
            plan.set_steering(steer_seq, layer, v)
        plan.prefill(p)
        plan.generate(p, new)
        tokens, results = plan.collect()
        assert all(r["generated"] == new and r["status"] == 0 for r in results)
        return plan, tokens

    plain, plain_tokens = run(1, None)
    plain_capture, plain_logits = plain.read_capture(0, 0, consumed), plain.logits(0)
    del plain
    steered, steered_tokens = run(1, 0)
    steered_capture, steered_logits = steered.read_capture(0, 0, consumed), steered.logits(0)
    del steered
    both, tokens = run(2, 1)
    assert tokens[0].tolist() == plain_tokens[0].tolist()
    assert tokens[1].tolist() == steered_tokens[0].tolist()
    assert np.array_equal(both.logits(0), plain_logits)
    assert np.array_equal(both.logits(1), steered_logits)
    assert np.array_equal(both.read_capture(0, 0, consumed), plain_capture)
    assert np.array_equal(both.read_capture(1, 0, consumed), steered_capture)
    assert not np.array_equal(plain_capture, steered_capture)


def test_exact_prefill_equals_token_loop_full_size(full_model):
    from dolittle_amd.qwen3 import Plan
    p, new = prompt(4, 600), 6
    loop = Plan(full_model, batch=1, capacity=640)
    loop.generate(p, new)
    want, _ = loop.collect()
    pre = Plan(full_model, batch=1, capacity=640)
    pre.prefill(p)
    pre.generate(p, new)
    got, results = pre.collect()
    assert results[0]["status"] == 0 and got[0].tolist() == want[0].tolist()
    assert np.array_equal(pre.logits(0), loop.logits(0))
    for layer in (0, 24, 35):
        k0, v0 = loop.read_cache(layer, 0, len(p) + new - 1)
        k1, v1 = pre.read_cache(layer, 0, len(p) + new - 1)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1), layer


def test_topp_batch_invariance_full_size(full_model):
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    p, new = prompt(5, 48), 10
    settings = SamplingSettings("categorical", 1.0, 0, 0.95)
    seeds = [7000 + 13 * b for b in range(8)]
    batch = Plan(full_model, batch=8, capacity=64)
    batch.generate(p, new, settings, seeds=seeds)
    tokens, results = batch.collect()
    assert all(r["generated"] == new and r["status"] == 0 for r in results)
    assert len({tuple(t) for t in tokens.tolist()}) > 1
    for b in (0, 3, 7):
        alone = Plan(full_model, batch=1, capacity=64)
        alone.generate(p, new, settings, seeds=[seeds[b]])
        got, _ = alone.collect()
        assert got[0].tolist() == tokens[b].tolist(), b


def test_nla_steps_full_size(full_model, device, queue):
    """The NLA steps around the block-24 capture at full size: a captured
    row normalized by DeviceInjection (scale 150) replaces a prompt
    embedding, and a one-row intervention at block 24 hits sequence 1 of a
    batch of two.  Sequence 0 equals the plain batch-1 run, sequence 1 its
    own batch-1 run with the same injection and intervention; the count is
    one and no status is latched."""
    from dolittle_amd.interventions import DeviceInjection, Region
    from dolittle_amd.qwen3 import Plan
    p, new, layer = prompt(6, 24), 6, 24
    source = Plan(full_model, batch=1, capacity=64)
    source.set_capture(layer)
    source.generate(p, new)
    source.collect()
    row = source.read_capture(0, 10, 1).reshape(-1)
    buf = device.upload_array(queue, row)
    inj = DeviceInjection(device, queue, Region(buf, 0, row.nbytes), "bfloat16", "bfloat16", 4096, 150.0)
    inj.submit()
    u = np.random.default_rng(8).standard_normal(4096).astype(np.float32)
    u = (u / np.float32(np.linalg.norm(u.astype(np.float64)))).astype(np.float32)

    def run(batch, seq_mask, seq):
        plan = Plan(full_model, batch=batch, capacity=64)
        plan.set_injection(inj, 5, seq_mask)
        plan.set_intervention(seq, layer, 12, u, 0.5)
        plan.generate(p, new)
        tokens, results = plan.collect()
        assert all(r["status"] == 0 for r in results), results
        assert plan.read_intervention() == (0, 1)
        return tokens, plan

    plain = Plan(full_model, batch=1, capacity=64)
    plain.generate(p, new)
    plain_tokens, _ = plain.collect()
    alone, alone_plan = run(1, 1, 0)
    both, both_plan = run(2, 0b10, 1)
    assert both[0].tolist() == plain_tokens[0].tolist()
    assert both[1].tolist() == alone[0].tolist()
    assert np.array_equal(both_plan.logits(1), alone_plan.logits(0))
