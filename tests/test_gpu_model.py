"""GPU parity of the Qwen3 token loop against the CPU contract mirror.

- the synthetic weight generator and the packed resident layout round-trip;
- one Qwen3-8B decoder block, decode at position 512
  over a seeded N(0,1) KV cache of 512 entries, output hidden state and
  appended K/V rows bit-exact;
- a multi-block Qwen3-8B-width model: greedy token stream and logits
  bit-exact over prefill + decode, plus loop semantics (stop ids, budget,
  positions) and batch invariance.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 20261201


def qwen_config(layers, vocab=151936, tied=True):
    from dolittle_amd.qwen3 import Qwen3Config
    return Qwen3Config(layers=layers, vocab=vocab, tied_embeddings=tied)


def oracle_weights(o, model):
    cfg = model.config
    dims = o.Dims(cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab, cfg.rms_eps,
                  cfg.rope_theta)
    blocks = []
    for layer in range(cfg.layers):
        blocks.append({name: np.ascontiguousarray(model.read(role, layer).reshape(-1)) for name, role in (
            ("input_norm", "input_norm"), ("wq", "q"), ("wk", "k"), ("wv", "v"), ("q_norm", "q_norm"),
            ("k_norm", "k_norm"), ("wo", "o"), ("post_norm", "post_norm"), ("wg", "gate"), ("wu", "up"),
            ("wd", "down"))})
    lm = np.ascontiguousarray(model.read("lm_head").reshape(-1))
    emb = lm if cfg.tied_embeddings else np.ascontiguousarray(model.read("embedding").reshape(-1))
    return o.Qwen3Weights(dims, blocks, np.ascontiguousarray(model.read("final_norm")), lm, emb)


class OracleRun:
    """The contract mirror composed in recipe order with its own KV cache."""

    def __init__(self, o, weights, capacity):
        self.o, self.w = o, weights
        d = weights.dims
        kw = d.kv_heads * d.head_dim
        self.k = [np.zeros(capacity * kw, np.uint16) for _ in weights.blocks]
        self.v = [np.zeros(capacity * kw, np.uint16) for _ in weights.blocks]
        self.pos = 0

    def step(self, token, logits=True, row=None):
        d = self.w.dims
        h = row.copy() if row is not None else self.w.embedding.reshape(d.vocab, d.hidden)[token].copy()
        for layer in range(len(self.w.blocks)):
            self.o.block_forward(self.w, layer, h, 1, self.pos, self.k[layer], self.v[layer])
        self.pos += 1
        self.h = h
        return self.o.logits(self.w, h) if logits else None


@pytest.fixture(scope="module")
def small_model(device, queue):
    from dolittle_amd.qwen3 import Qwen3Model
    model = Qwen3Model(device, queue, qwen_config(layers=2))
    model.fill_synthetic(SEED, 0.02)
    return model


def test_synthetic_weights_match_cpu_generator(small_model, oracle):
    """Element i of (role, layer) is dl_normal_bf16(seed, layer*16 + role, i)
    on host and device alike; this also round-trips the packed layouts."""
    from dolittle_amd.qwen3 import ROLE
    for role, layer in (("q", 0), ("k", 1), ("v", 0), ("o", 1), ("gate", 0), ("up", 1), ("down", 0)):
        got = small_model.read(role, layer).reshape(-1)
        n = min(got.size, 1 << 20)
        want = oracle.normal_bf16(n, SEED, layer * 16 + ROLE[role], 0.02)
        assert np.array_equal(got[:n], want), role
        tail = oracle.normal_bf16(4096, SEED, layer * 16 + ROLE[role], 0.02, got.size - 4096)
        assert np.array_equal(got[-4096:], tail), role
    lm = small_model.read("lm_head").reshape(-1)
    assert np.array_equal(lm[: 1 << 18], oracle.normal_bf16(1 << 18, SEED, ROLE["embedding"], 0.02))
    assert np.all(small_model.read("input_norm", 0) == 0x3F80)
    vals = oracle.f32_from_bf16(lm[: 1 << 20])
    assert abs(float(vals.std()) - 0.02) < 2e-4 and abs(float(vals.mean())) < 2e-4


def test_write_read_tensor_round_trip(device, queue, oracle):
    from dolittle_amd.qwen3 import Qwen3Model
    model = Qwen3Model(device, queue, qwen_config(layers=1, vocab=2048, tied=False))
    rng = np.random.default_rng(2)
    for role in ("q", "k", "v", "o", "gate", "up", "down", "lm_head", "embedding", "q_norm", "final_norm"):
        shape = model.config.shape(role)
        data = rng.integers(0, 65536, int(np.prod(shape)), dtype=np.uint16)
        model.write(role, 0, data)
        assert np.array_equal(model.read(role, 0).reshape(-1), data), role


def test_config1_single_block_decode(device, queue, oracle):
    """one Qwen3-8B block, token at position 512, seeded
    N(0,1) BF16 cache of 512 entries, N(0,1) input residual."""
    from dolittle_amd.qwen3 import Plan, Qwen3Model
    model = Qwen3Model(device, queue, qwen_config(layers=1, vocab=2048))
    model.fill_synthetic(SEED, 0.02)
    w = oracle_weights(oracle, model)
    plan = Plan(model, batch=1, capacity=513)
    kw = 8 * 128
    keys = oracle.normal_bf16(512 * kw, SEED + 1, 1000, 1.0)
    values = oracle.normal_bf16(512 * kw, SEED + 1, 1001, 1.0)
    plan.write_cache(0, 0, keys, values)
    x = oracle.normal_bf16(4096, SEED + 1, 1002, 1.0)
    plan.set_embedding_override(512, x, 1)
    plan.seek(512)
    plan.forward([0])
    got = plan.hidden(0)
    run = OracleRun(oracle, w, 513)
    run.k[0][: 512 * kw] = keys
    run.v[0][: 512 * kw] = values
    run.pos = 512
    run.step(0, logits=True, row=x)
    assert np.array_equal(got, run.h)
    k_row, v_row = plan.read_cache(0, 512, 1)
    assert np.array_equal(k_row, run.k[0][512 * kw: 513 * kw])
    assert np.array_equal(v_row, run.v[0][512 * kw: 513 * kw])
    k_old, _ = plan.read_cache(0, 0, 512)
    assert np.array_equal(k_old, keys)
    assert np.array_equal(plan.logits(0), oracle.logits(w, run.h))


@pytest.mark.parametrize("position", [1, 63, 64, 77, 383, 511, 512, 513, 777, 1023, 1024, 1089, 1500, 1535, 1536,
                                      1543, 4607])
def test_single_block_both_attention_paths(device, queue, oracle, position):
    """Positions below 1536 run the fused short-context attention kernel,
    positions from 1536 the three-kernel split; both equal the oracle, up to
    BASELINE config 3's last decode position (4607)."""
    from dolittle_amd.qwen3 import Plan, Qwen3Model
    model = Qwen3Model(device, queue, qwen_config(layers=1, vocab=2048))
    model.fill_synthetic(SEED + 7, 0.02)
    w = oracle_weights(oracle, model)
    capacity = max(1600, position + 1)
    plan = Plan(model, batch=1, capacity=capacity)
    kw = 8 * 128
    keys = oracle.normal_bf16(position * kw, SEED + 3, 2000, 1.0)
    values = oracle.normal_bf16(position * kw, SEED + 3, 2001, 1.0)
    plan.write_cache(0, 0, keys, values)
    x = oracle.normal_bf16(4096, SEED + 3, 2002, 1.0)
    plan.set_embedding_override(position, x, 1)
    plan.seek(position)
    plan.forward([0])
    run = OracleRun(oracle, w, capacity)
    run.k[0][: position * kw] = keys
    run.v[0][: position * kw] = values
    run.pos = position
    run.step(0, logits=False, row=x)
    assert np.array_equal(plan.hidden(0), run.h)


@pytest.mark.parametrize("position", [1535, 1536, 4607])
def test_eager_launches_pick_the_attention_path_by_position(device, queue, oracle, monkeypatch, position):
    """DL_EAGER=1 launches the step kernels directly (no graphs are
    captured); the attention path still follows the position, so a step at
    1536 keys or more runs the three-kernel split and equals the oracle."""
    from dolittle_amd.qwen3 import Plan, Qwen3Model
    monkeypatch.setenv("DL_EAGER", "1")
    model = Qwen3Model(device, queue, qwen_config(layers=1, vocab=2048))
    model.fill_synthetic(SEED + 7, 0.02)
    w = oracle_weights(oracle, model)
    capacity = position + 64
    plan = Plan(model, batch=1, capacity=capacity)
    kw = 8 * 128
    keys = oracle.normal_bf16(position * kw, SEED + 5, 2000, 1.0)
    values = oracle.normal_bf16(position * kw, SEED + 5, 2001, 1.0)
    plan.write_cache(0, 0, keys, values)
    x = oracle.normal_bf16(4096, SEED + 5, 2002, 1.0)
    plan.set_embedding_override(position, x, 1)
    plan.seek(position)
    plan.forward([0])
    run = OracleRun(oracle, w, capacity)
    run.k[0][: position * kw] = keys
    run.v[0][: position * kw] = values
    run.pos = position
    run.step(0, logits=False, row=x)
    assert np.array_equal(plan.hidden(0), run.h)


def test_greedy_stream_bit_exact(small_model, oracle):
    """Prefill + greedy decode through the device-owned loop equals the
    contract mirror token for token, and the final logits bit for bit."""
    from dolittle_amd.qwen3 import Plan
    w = oracle_weights(oracle, small_model)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, 151936, 12)]
    max_new = 20
    plan = Plan(small_model, batch=1, capacity=64)
    plan.generate(prompt, max_new)
    tokens, results = plan.collect()
    assert results[0]["generated"] == max_new and results[0]["reason"] == "limit"
    assert results[0]["position"] == len(prompt) + max_new
    run = OracleRun(oracle, w, 64)
    expected = []
    for i, t in enumerate(prompt):
        logits = run.step(t, logits=(i == len(prompt) - 1))
    for _ in range(max_new):
        status, nxt = oracle.greedy(logits)
        assert status == 0
        expected.append(nxt)
        logits = run.step(nxt)
    assert tokens[0].tolist() == expected


def test_forward_chunks_equal_generation(small_model, oracle):
    """Cached chunk forward (diagnostic path) gives the same logits as the
    oracle after each chunk, independent of chunking."""
    from dolittle_amd.qwen3 import Plan
    w = oracle_weights(oracle, small_model)
    prompt = [int(t) for t in np.random.default_rng(9).integers(0, 151936, 9)]
    plan = Plan(small_model, batch=1, capacity=32)
    plan.forward(prompt[:4])
    plan.forward(prompt[4:])
    run = OracleRun(oracle, w, 32)
    for i, t in enumerate(prompt):
        logits = run.step(t, logits=(i == len(prompt) - 1))
    assert np.array_equal(plan.logits(0), logits)
    assert plan.position() == len(prompt)


def test_stop_id_and_budget(small_model):
    from dolittle_amd.qwen3 import Plan
    prompt = [11, 22, 33]
    plan = Plan(small_model, batch=1, capacity=64)
    plan.generate(prompt, 10)
    tokens, _ = plan.collect()
    stream = tokens[0].tolist()
    stop = stream[3]
    plan.generate(prompt, 10, stop_ids=[stop])
    tokens2, res = plan.collect()
    first = stream.index(stop)
    assert res[0]["generated"] == first + 1 and res[0]["reason"] == "eos"
    assert tokens2[0][: first + 1].tolist() == stream[: first + 1]
    plan.generate(prompt, 0)
    _, res0 = plan.collect()
    assert res0[0]["generated"] == 0 and res0[0]["position"] == len(prompt)


def test_batch_two_equals_batch_one(small_model):
    """Two identical sequences in one batched plan reproduce the batch-1
    stream (batch invariance of every reduction)."""
    from dolittle_amd.qwen3 import Plan
    prompt = [5, 6, 7, 8]
    p1 = Plan(small_model, batch=1, capacity=32)
    p1.generate(prompt, 8)
    t1, _ = p1.collect()
    p2 = Plan(small_model, batch=2, capacity=32)
    p2.generate(prompt, 8)
    t2, _ = p2.collect()
    assert t2[0].tolist() == t1[0].tolist() and t2[1].tolist() == t1[0].tolist()


def test_batch_eight_equals_batch_one(small_model):
    """Batch 8 runs Q and K/V as two launches, the down projection with its
    inputs staged in 4096-wide blocks, and the 8-row gate/up, O and LM-head
    kernels; every sequence reproduces the batch-1 stream and its last
    logits bit for bit."""
    from dolittle_amd.qwen3 import Plan
    prompt = [9, 150000, 3, 77, 4096]
    p1 = Plan(small_model, batch=1, capacity=32)
    p1.generate(prompt, 10)
    t1, _ = p1.collect()
    l1 = p1.logits(0)
    p8 = Plan(small_model, batch=8, capacity=32)
    p8.generate(prompt, 10)
    t8, res = p8.collect()
    for b in range(8):
        assert t8[b].tolist() == t1[0].tolist(), b
        assert res[b]["generated"] == 10
        assert np.array_equal(p8.logits(b), l1), b


@pytest.mark.parametrize("batch", [3, 4, 5, 6, 7, 8])
def test_batched_rows_follow_their_own_sequences(small_model, batch):
    """Each sequence of a batched plan samples with its own MT19937-64 seed,
    so the rows diverge; every row's token stream and last logits equal a
    batch-1 run with that seed.  Covers the 4- and 8-row kernels over all
    their rows and over fewer rows (3 rows on the 4-row kernels, 5 to 7 on
    the 8-row kernels, which read and write only the rows that exist),
    where a row read from or written to the wrong sequence would show."""
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    prompt = [11, 4242, 90000, 7]
    settings = SamplingSettings("categorical", 1.0, 0, 0.95)
    seeds = [1000 + 17 * b for b in range(batch)]
    pb = Plan(small_model, batch=batch, capacity=24)
    pb.generate(prompt, 12, settings, seeds)
    tb, res = pb.collect()
    streams = set()
    for b in range(batch):
        p1 = Plan(small_model, batch=1, capacity=24)
        p1.generate(prompt, 12, settings, [seeds[b]])
        t1, _ = p1.collect()
        assert tb[b].tolist() == t1[0].tolist(), b
        assert res[b]["generated"] == 12
        assert np.array_equal(pb.logits(b), p1.logits(0)), b
        streams.add(tuple(t1[0].tolist()))
    assert len(streams) > 1  # the rows really differ


@pytest.mark.parametrize("batch,grids", [
    (2, [(5, 768), (7, 256), (6, 256)]),   # gate/up, LM head and down off their 2-row defaults
    (3, [(5, 96), (4, 512)]),              # 3 rows on the 4-row kernels
    (8, [(0, 96), (6, 128), (7, 320)]),    # the 8-row Q and K/V parts on fewer workgroups
])
def test_workgroup_counts_do_not_change_results(small_model, batch, grids):
    """Every output is the same FMA chain whichever workgroup runs its tile,
    so a plan whose decode kernels are launched with other workgroup counts
    (dl_plan_set_grid) produces the same tokens and logits as one with the
    defaults."""
    from dolittle_amd import _lib
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    prompt = [5, 17, 91000, 4242, 7]
    settings = SamplingSettings("categorical", 1.0, 0, 0.95)
    seeds = [300 + 11 * b for b in range(batch)]
    runs = []
    for custom in (False, True):
        plan = Plan(small_model, batch=batch, capacity=24)
        if custom:
            for which, blocks in grids:
                _lib.call("dl_plan_set_grid", plan.handle, which, blocks)
        plan.generate(prompt, 10, settings, seeds)
        tokens, _ = plan.collect()
        runs.append((tokens, [plan.logits(b) for b in range(batch)]))
    assert np.array_equal(runs[0][0], runs[1][0])
    for b in range(batch):
        assert np.array_equal(runs[0][1][b], runs[1][1][b]), b


def _categorical_run(plan, prompt, max_new, settings, seeds, override=None, stop_ids=None):
    """Drives the loop one step at a time; returns the per-step logits rows
    and the emitted tokens of every sequence."""
    plan.prepare_generation(prompt, max_new, settings, seeds, stop_ids=stop_ids)
    plan.decode_steps(len(prompt))
    logits = []
    for step in range(max_new):
        logits.append([plan.logits(b) for b in range(plan.batch)])
        if step + 1 < max_new:
            plan.decode_steps(1)
    plan.decode_steps(1)
    tokens, results = plan.collect()
    return logits, tokens, results


def test_categorical_loop_ids_follow_the_law(small_model, oracle):
    """Interpretation-sampling shape at reduced length: 8 sequences share a
    prompt with one injected embedding row (BF16 N(0,1) x 40), top-p 0.95 at
    T 1 with per-sequence MT19937-64 seeds.  Every sampled id equals the host
    law applied to that step's device logits with the sequence's draws."""
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    prompt = [int(t) for t in np.random.default_rng(21).integers(0, 151936, 24)]
    plan = Plan(small_model, batch=8, capacity=64)
    row = oracle.normal_bf16(4096, SEED + 5, 3000, 40.0)
    plan.set_embedding_override(7, row, 0xFF)
    seeds = [1000 + 17 * b for b in range(8)]
    settings = SamplingSettings("categorical", 1.0, 0, 0.95)
    max_new = 6
    logits, tokens, results = _categorical_run(plan, prompt, max_new, settings, seeds)
    for b in range(8):
        assert results[b]["generated"] == max_new, results[b]
        rng = oracle.MT19937_64(seeds[b])
        for i in range(max_new):
            status, want = oracle.categorical_bits(oracle.f32_from_bf16(logits[i][b]), 1, 1.0, 0, 0.95, rng())
            assert status == 0
            assert tokens[b][i] == want, (b, i)
    assert len({tuple(t) for t in tokens.tolist()}) > 1


def test_categorical_stop_id_ends_one_sequence(small_model, oracle):
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    prompt = [5, 6, 7, 8, 9]
    seeds = [3, 4, 5, 6]
    settings = SamplingSettings("categorical", 1.0, 0, 0.95)
    plan = Plan(small_model, batch=4, capacity=32)
    plan.generate(prompt, 6, settings, seeds)
    base, _ = plan.collect()
    stop = int(base[2][1])
    plan.generate(prompt, 6, settings, seeds, stop_ids=[stop])
    tokens, results = plan.collect()
    for b in range(4):
        stream = base[b].tolist()
        if stop in stream:
            first = stream.index(stop)
            assert results[b]["generated"] == first + 1 and results[b]["reason"] == "eos"
            assert tokens[b][: first + 1].tolist() == stream[: first + 1]
        else:
            assert results[b]["generated"] == 6
            assert tokens[b].tolist() == stream


def test_categorical_then_greedy_recaptures(small_model):
    """Switching the law re-records the step graphs; greedy afterwards equals
    a fresh greedy plan."""
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    prompt = [11, 12, 13]
    plan = Plan(small_model, batch=2, capacity=32)
    plan.generate(prompt, 4, SamplingSettings("categorical", 0.8, 10, 0.9), [1, 2])
    plan.collect()
    plan.generate(prompt, 4)
    t, _ = plan.collect()
    fresh = Plan(small_model, batch=2, capacity=32)
    fresh.generate(prompt, 4)
    t2, _ = fresh.collect()
    assert t.tolist() == t2.tolist()


def test_capture_and_steering_batch_two(small_model, oracle):
    """Config-4 semantics at two blocks: both sequences capture block 0's
    output at every consumed position; sequence 1 is steered there by a unit
    FP32 vector times 8 (h <- BF16(FP32(h) + v)) and the capture sees the
    steered row.  Streams, captures and final logits equal the oracle."""
    from dolittle_amd.qwen3 import Plan
    w = oracle_weights(oracle, small_model)
    d = w.dims
    layer = 0
    rng = np.random.default_rng(44)
    v = rng.standard_normal(d.hidden).astype(np.float32)
    v = (v / np.float32(np.linalg.norm(v.astype(np.float64)))).astype(np.float32) * np.float32(8.0)
    prompt = [int(t) for t in rng.integers(0, 151936, 10)]
    max_new = 6
    plan = Plan(small_model, batch=2, capacity=64)
    plan.set_capture(layer)
    plan.set_steering(1, layer, v)
    plan.generate(prompt, max_new)
    tokens, results = plan.collect()
    consumed = len(prompt) + max_new
    for seq in (0, 1):
        assert results[seq]["generated"] == max_new
        kw = d.kv_heads * d.head_dim
        k = [np.zeros(64 * kw, np.uint16) for _ in w.blocks]
        vv = [np.zeros(64 * kw, np.uint16) for _ in w.blocks]
        stream, captures, logits = list(prompt), [], None
        for pos in range(consumed):
            h = w.embedding.reshape(d.vocab, d.hidden)[stream[pos]].copy()
            for l in range(len(w.blocks)):
                oracle.block_forward(w, l, h, 1, pos, k[l], vv[l])
                if l == layer:
                    if seq == 1:
                        oracle.steer(h, v)
                    captures.append(h.copy())
            if pos >= len(prompt) - 1 and len(stream) < consumed:
                logits = oracle.logits(w, h)
                status, nxt = oracle.greedy(logits)
                assert status == 0
                stream.append(nxt)
        assert tokens[seq].tolist() == stream[len(prompt):], seq
        got = plan.read_capture(seq, 0, consumed)
        assert np.array_equal(got, np.stack(captures)), seq
        assert np.array_equal(plan.logits(seq), logits), seq
    assert tokens[0].tolist() != tokens[1].tolist()
