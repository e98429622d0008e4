"""GPU parity of the plan's live injection and residual intervention
(dl_plan_set_injection / dl_plan_set_intervention; executor.cpp:1583-1643,
executor.cpp:1717-1748, decode.cu:104-190) with the CPU contract mirror:
the oracle's block composition with oracle/nla.c's injection normalization
and one-row intervention at the same points, bit for bit on the exact
paths (decode steps, the exact prompt pass) and through a with/without
comparison on the MFMA prefill.  Status rules: an invalid injection ends
the loop before it consumes anything (status 8), a failed intervention ends
it after the failing position (status 16), and the count is exactly one."""
import numpy as np
import pytest

from test_gpu_model import oracle_weights, small_model  # noqa: F401  (module fixture)

pytestmark = pytest.mark.gpu


def oracle_stream(o, w, prompt, max_new, capture_layer=None, inject=None, intervene=None):
    """Greedy stream of one sequence.  inject: (position, BF16 row);
    intervene: (layer, position, FP32 direction, strength)."""
    d = w.dims
    kw = d.kv_heads * d.head_dim
    k = [np.zeros(64 * kw, np.uint16) for _ in w.blocks]
    v = [np.zeros(64 * kw, np.uint16) for _ in w.blocks]
    stream, captures, logits = list(prompt), [], None
    state = np.zeros(2, np.uint32)
    consumed = len(prompt) + max_new
    for pos in range(consumed):
        if inject is not None and pos == inject[0]:
            h = inject[1].copy()
        else:
            h = w.embedding.reshape(d.vocab, d.hidden)[stream[pos]].copy()
        for layer in range(len(w.blocks)):
            o.block_forward(w, layer, h, 1, pos, k[layer], v[layer])
            if intervene is not None and layer == intervene[0]:
                o.intervene(h, True, 1, d.hidden, intervene[2], pos, intervene[1], intervene[3], state)
            if layer == capture_layer:
                captures.append(h.copy())
        if pos >= len(prompt) - 1 and len(stream) < consumed:
            logits = o.logits(w, h)
            status, nxt = o.greedy(logits)
            assert status == 0
            stream.append(nxt)
    return stream[len(prompt):], captures, logits, state


def unit_direction(o, d, seed):
    rng = np.random.default_rng(seed)
    a = o.bf16_from_f32(rng.standard_normal(d.hidden).astype(np.float32))
    b = o.bf16_from_f32(rng.standard_normal(d.hidden).astype(np.float32))
    status, u = o.direction(a, b, True)
    assert status == 0
    return u


@pytest.mark.parametrize("exact_prefill", [False, True])
def test_intervention_matches_oracle(small_model, oracle, exact_prefill):
    """Batch two, sequence 1 intervened at block 1 of position 4 (a prompt
    row: a decode step, or the exact prompt pass when prefilled), the
    capture of that block sees the intervened row; sequence 0 is
    untouched.  Tokens, captures and final logits equal the oracle."""
    from dolittle_amd.qwen3 import Plan
    w = oracle_weights(oracle, small_model)
    d = w.dims
    layer, position, strength = 1, 4, 0.75
    u = unit_direction(oracle, d, 7)
    rng = np.random.default_rng(45)
    prompt = [int(t) for t in rng.integers(0, 151936, 9)]
    max_new = 4
    plan = Plan(small_model, batch=2, capacity=64)
    plan.set_capture(layer)
    plan.set_intervention(1, layer, position, u, strength)
    if exact_prefill:
        plan.prefill(prompt)
        assert plan.read_intervention() == (0, 1)
    plan.generate(prompt, max_new)
    tokens, results = plan.collect()
    assert plan.read_intervention() == (0, 1)
    consumed = len(prompt) + max_new
    for seq in (0, 1):
        iv = (layer, position, u, strength) if seq == 1 else None
        stream, captures, logits, state = oracle_stream(oracle, w, prompt, max_new, layer, intervene=iv)
        assert results[seq]["status"] == 0 and results[seq]["reason"] == "limit", results[seq]
        assert tokens[seq].tolist() == stream, seq
        assert np.array_equal(plan.read_capture(seq, 0, consumed), np.stack(captures)), seq
        assert np.array_equal(plan.logits(seq), logits), seq
        if seq == 1:
            assert state.tolist() == [0, 1]


def test_intervention_through_device_direction(small_model, oracle, device, queue):
    """The direction region of a DeviceDirection feeds the plan directly; the
    intervention at the last prompt position (consumed by the selecting
    step) equals the oracle."""
    from dolittle_amd.interventions import DeviceDirection, Region
    from dolittle_amd.qwen3 import Plan
    w = oracle_weights(oracle, small_model)
    d = w.dims
    rng = np.random.default_rng(46)
    a = oracle.bf16_from_f32(rng.standard_normal(d.hidden).astype(np.float32))
    b = oracle.bf16_from_f32(rng.standard_normal(d.hidden).astype(np.float32))
    ba, bb = device.upload_array(queue, a), device.upload_array(queue, b)
    dd = DeviceDirection(device, queue, Region(ba, 0, a.nbytes), Region(bb, 0, b.nbytes), "bfloat16", d.hidden)
    dd.submit()
    region = dd.finish()
    _, u = oracle.direction(a, b, True)
    prompt = [int(t) for t in rng.integers(0, 151936, 6)]
    plan = Plan(small_model, batch=1, capacity=64)
    plan.set_intervention(0, 0, len(prompt) - 1, region, 1.5)
    plan.generate(prompt, 3)
    tokens, results = plan.collect()
    stream, _, logits, state = oracle_stream(oracle, w, prompt, 3, intervene=(0, len(prompt) - 1, u, 1.5))
    assert results[0]["status"] == 0 and tokens[0].tolist() == stream
    assert np.array_equal(plan.logits(0), logits)
    assert plan.read_intervention() == (0, 1) and state.tolist() == [0, 1]


def test_intervention_on_mfma_prefill(small_model, oracle):
    """MFMA prefill: the captured block output at the intervention position is
    the oracle's intervention applied to the same block output of a run
    without it, bit for bit; earlier positions are unchanged and the count
    is one through the resumed generation."""
    from dolittle_amd.qwen3 import Plan
    d = oracle_weights(oracle, small_model).dims
    layer, position, strength = 0, 11, 0.5
    u = unit_direction(oracle, d, 8)
    rng = np.random.default_rng(47)
    prompt = [int(t) for t in rng.integers(0, 151936, 24)]
    plan = Plan(small_model, batch=1, capacity=64)
    plan.set_capture(layer)
    plan.prefill(prompt, mfma=True)
    before = plan.read_capture(0, 0, position + 1)
    plan.set_intervention(0, layer, position, u, strength)
    plan.prefill(prompt, mfma=True)
    after = plan.read_capture(0, 0, position + 1)
    assert plan.read_intervention() == (0, 1)
    assert np.array_equal(after[:position], before[:position])
    expect = before[position].copy()
    state = np.zeros(2, np.uint32)
    assert oracle.intervene(expect, True, 1, d.hidden, u, position, position, strength, state)
    assert state.tolist() == [0, 1] and not np.array_equal(expect, before[position])
    assert np.array_equal(after[position], expect)
    plan.generate(prompt, 2)
    _, results = plan.collect()
    assert results[0]["status"] == 0 and results[0]["generated"] == 2
    assert plan.read_intervention() == (0, 1)


def test_intervention_failure_ends_the_loop(small_model, oracle):
    """A nonfinite beta latches the intervention status: the loop ends after
    the failing position with reason failure and status bit 16, selecting
    nothing; a later generation without the intervention runs normally."""
    from dolittle_amd.qwen3 import Plan
    d = oracle_weights(oracle, small_model).dims
    u = unit_direction(oracle, d, 9)
    prompt = [5, 17, 99, 1234, 77, 8]
    plan = Plan(small_model, batch=1, capacity=64)
    plan.set_intervention(0, 1, 2, u, 3.0e38)
    plan.generate(prompt, 4)
    _, results = plan.collect()
    r = results[0]
    assert r["reason"] == "failure" and r["status"] & 16 and r["generated"] == 0 and r["position"] == 3, r
    assert plan.read_intervention() == (1, 1)
    with pytest.raises(Exception):
        plan.set_intervention(0, 1, 2, u, float("nan"))
    with pytest.raises(Exception):  # the position must be a prompt row
        plan.set_intervention(0, 1, len(prompt), u, 1.0)
        plan.generate(prompt, 1)
    plan.set_intervention(0, 1, 0, None, 0.0)
    plan.generate(prompt, 2)
    _, results = plan.collect()
    assert results[0]["reason"] == "limit" and results[0]["status"] == 0 and results[0]["generated"] == 2


def injection(oracle, device, queue, d, seed, zero=False):
    from dolittle_amd.interventions import DeviceInjection, Region
    x = np.zeros(d.hidden, np.float32) if zero else np.random.default_rng(seed).standard_normal(d.hidden)
    x = oracle.bf16_from_f32(np.asarray(x, np.float32))
    buf = device.upload_array(queue, x)
    inj = DeviceInjection(device, queue, Region(buf, 0, x.nbytes), "bfloat16", "bfloat16", d.hidden, 150.0)
    inj.submit()
    inj._source_buffer = buf
    status, _, row = oracle.inject(x, True, True, 150.0)
    return inj, status, row


@pytest.mark.parametrize("exact_prefill", [False, True])
def test_injection_matches_oracle(small_model, oracle, device, queue, exact_prefill):
    """The normalized row replaces the embedding of prompt position 3 for
    sequence 1 only; streams and logits equal the oracle."""
    from dolittle_amd.qwen3 import Plan
    w = oracle_weights(oracle, small_model)
    d = w.dims
    inj, status, row = injection(oracle, device, queue, d, 11)
    assert status == 0
    rng = np.random.default_rng(48)
    prompt = [int(t) for t in rng.integers(0, 151936, 7)]
    max_new = 3
    plan = Plan(small_model, batch=2, capacity=64)
    plan.set_injection(inj, 3, seq_mask=0b10)
    if exact_prefill:
        plan.prefill(prompt)
    plan.generate(prompt, max_new)
    tokens, results = plan.collect()
    for seq in (0, 1):
        stream, _, logits, _ = oracle_stream(oracle, w, prompt, max_new, inject=(3, row) if seq else None)
        assert results[seq]["status"] == 0, results[seq]
        assert tokens[seq].tolist() == stream, seq
        assert np.array_equal(plan.logits(seq), logits), seq


def test_injection_status_gates_the_loop(small_model, oracle, device, queue):
    """A zero source row is an invalid injection: the loop ends before it
    consumes anything (status bit 8, reason failure, position 0).  An
    injection position past the prompt replaces nothing; removing the
    injection restores the plain run."""
    from dolittle_amd.qwen3 import Plan
    d = oracle_weights(oracle, small_model).dims
    bad, status, _ = injection(oracle, device, queue, d, 0, zero=True)
    assert status == 1
    prompt = [3, 1, 4, 1, 5]
    plan = Plan(small_model, batch=1, capacity=64)
    plan.set_injection(bad, 1)
    plan.generate(prompt, 3)
    _, results = plan.collect()
    r = results[0]
    assert r["reason"] == "failure" and r["status"] == 8 and r["generated"] == 0 and r["position"] == 0, r
    plan.set_injection(None, 0)
    plan.generate(prompt, 3)
    plain, results = plan.collect()
    assert results[0]["status"] == 0
    good, _, _ = injection(oracle, device, queue, d, 12)
    plan.set_injection(good, len(prompt) + 1)
    plan.generate(prompt, 3)
    late, results = plan.collect()
    assert results[0]["status"] == 0 and late[0].tolist() == plain[0].tolist()
    with pytest.raises(Exception):  # FP32 output does not match BF16 activations
        from dolittle_amd import _lib
        _lib.call("dl_plan_set_injection", plan.handle, 1, good.storage.ptr(), 2, 1)


@pytest.mark.parametrize("prefill", ["none", "exact", "mfma"])
def test_edge_positions(small_model, oracle, device, queue, prefill):
    """Edge positions: the injection at the last prompt position (always
    consumed by the selecting step, also after a prefill) and the
    intervention at position 0 (row 0 of the first chunk or prefill block).
    Bit-exact with the oracle on the exact paths; on the MFMA prefill the
    greedy stream must still follow (the intervened row is exact, later
    rows carry the MFMA tolerance, so the check there is count and status)."""
    from dolittle_amd.qwen3 import Plan
    w = oracle_weights(oracle, small_model)
    d = w.dims
    inj, status, row = injection(oracle, device, queue, d, 13)
    assert status == 0
    u = unit_direction(oracle, d, 14)
    p = [int(t) for t in np.random.default_rng(49).integers(0, 151936, 11)]
    max_new = 3
    plan = Plan(small_model, batch=1, capacity=64)
    plan.set_injection(inj, len(p) - 1, 1)
    plan.set_intervention(0, 1, 0, u, 0.25)
    if prefill == "exact":
        plan.prefill(p)
    elif prefill == "mfma":
        plan.prefill(p, mfma=True)
    if prefill != "none":
        assert plan.read_intervention() == (0, 1)
    plan.generate(p, max_new)
    tokens, results = plan.collect()
    assert results[0]["status"] == 0 and results[0]["generated"] == max_new
    assert plan.read_intervention() == (0, 1)
    if prefill != "mfma":
        stream, _, logits, state = oracle_stream(oracle, w, p, max_new, inject=(len(p) - 1, row),
                                                 intervene=(1, 0, u, 0.25))
        assert tokens[0].tolist() == stream and np.array_equal(plan.logits(0), logits)
