"""Full-depth parity of BASELINE configs 2 and 3 against the CPU oracle.

- Config 2 at its real depth: Qwen3-8B (36 blocks, tied 151,936-row head,
  seeded N(0, 0.02) BF16 weights), a 128-id seeded prompt and 64 greedy
  tokens.  The token stream and the last selection's logits are bit-exact
  with the oracle, both when the loop consumes the prompt one position per
  step and after the exact chunked prompt pass (the bench's path).  This is
  the north star's "greedy token streams identical for the first 64 tokens"
  at full size.
- Config 3's 4096-id prompt at 2 blocks against the oracle: the exact
  chunked prompt pass is bit-exact (caches, logits, tokens).  The MFMA
  prefill is as close to the exact pass as the exact pass with one-ulp flips
  on 0.1% of block 0's cached K/V entries (the sensitivity floor), and both
  miss the north star's logits bound (2e-2 absolute + 1e-2 relative, every
  logit): an expected failure, kept below.
- Config 3 at 36 blocks: the same floor comparison against the
  oracle-pinned exact pass; the floor and the MFMA pass both exceed the
  reference's own 36-block acceptance budget
  (scripts/validation/README.md:128-142: max |d| <= max(1e-4, peak / 16),
  relative L2 <= 0.03), an expected failure; and greedy decode grown to
  4608 keys, where the exact prompt pass then 512 tokens equals consuming
  all 4096 prompt ids through the loop (tokens, logits, caches of blocks 0,
  24, 35).
- Config 4 at 36 blocks with its 256-id prompt (16 tokens): batch 2,
  block-24 capture at every position, sequence 1 steered there by the unit
  vector times 8; tokens, all 272 captured rows and the last logits of both
  sequences bit-exact with the oracle.
- Config 5 at 36 blocks with its 192-id prefix (8 tokens per sample): the
  x40 injected embedding slot, batch 8, top-p 0.95; the first selection's
  logits bit-exact with the oracle for every sample and every sampled id
  equal to the host law on that step's device logits.
"""
import numpy as np
import pytest

from parity_helpers import OracleLoop, logit_errors, read_weights

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

SEED = 20261201


def prompt(seed, n):
    return [int(t) for t in np.random.default_rng(seed).integers(0, 151936, n)]


@pytest.fixture(scope="module")
def full_model(device, queue):
    from dolittle_amd.qwen3 import Qwen3Config, Qwen3Model
    model = Qwen3Model(device, queue, Qwen3Config())
    model.fill_synthetic(SEED, 0.02)
    return model


@pytest.fixture(scope="module")
def full_weights(full_model, oracle):
    """The 36-block model's weights read back into the oracle's layout
    (checked against the seeded generator)."""
    return read_weights(oracle, full_model, seed=SEED)


@pytest.mark.timeout(900)
def test_config2_full_depth_matches_oracle(full_model, full_weights, oracle):
    from dolittle_amd.qwen3 import Plan
    p, new = prompt(128, 128), 64
    loop = Plan(full_model, batch=1, capacity=len(p) + new + 1)
    loop.generate(p, new)
    loop_tokens, results = loop.collect()
    assert results[0]["generated"] == new and results[0]["status"] == 0
    pre = Plan(full_model, batch=1, capacity=len(p) + new + 1)
    pre.prefill(p)
    pre.generate(p, new)
    pre_tokens, pre_results = pre.collect()
    assert pre_results[0]["generated"] == new and pre_results[0]["status"] == 0

    run = OracleLoop(oracle, full_weights, len(p) + new + 1)
    want_tokens, want_logits = run.generate(p, new)
    assert loop_tokens[0].tolist() == want_tokens
    assert np.array_equal(loop.logits(0), want_logits)
    assert pre_tokens[0].tolist() == want_tokens
    assert np.array_equal(pre.logits(0), want_logits)
    for layer in (0, 35):
        k, v = pre.read_cache(layer, 0, len(p) + new - 1)
        wk, wv = run.cache_rows(layer, len(p) + new - 1)
        assert np.array_equal(k, wk) and np.array_equal(v, wv), layer


@pytest.fixture(scope="module")
def two_blocks(device, queue):
    from dolittle_amd.qwen3 import Qwen3Config, Qwen3Model
    model = Qwen3Model(device, queue, Qwen3Config(layers=2))
    model.fill_synthetic(SEED + 3, 0.02)
    return model


@pytest.fixture(scope="module")
def config3_oracle(two_blocks, oracle):
    """The oracle over config 3's 4096-id prompt at 2 blocks: the prompt
    positions before the last as one chunk, then 4 greedy steps."""
    p, new = prompt(4096, 4096), 4
    w = read_weights(oracle, two_blocks, seed=SEED + 3)
    run = OracleLoop(oracle, w, len(p) + new + 1)
    run.prompt(p[:-1])
    first_logits = None
    seq, tokens, logits = list(p), [], None
    for position in range(len(p) - 1, len(p) - 1 + new):
        logits = run.step(seq[position], position)
        first_logits = logits if first_logits is None else first_logits
        status, token = oracle.greedy(logits)
        assert status == 0
        tokens.append(token)
        seq.append(token)
    return p, new, run, tokens, first_logits, logits


@pytest.mark.timeout(900)
def test_config3_exact_prefill_4096_two_blocks_matches_oracle(two_blocks, config3_oracle):
    from dolittle_amd.qwen3 import Plan
    p, new, run, tokens, _, logits = config3_oracle
    plan = Plan(two_blocks, batch=1, capacity=len(p) + new + 1)
    plan.prefill(p)
    plan.generate(p, new)
    got, results = plan.collect()
    assert results[0]["generated"] == new and results[0]["status"] == 0
    assert got[0].tolist() == tokens
    assert np.array_equal(plan.logits(0), logits)
    for layer in (0, 1):
        k, v = plan.read_cache(layer, 0, len(p) + new - 1)
        wk, wv = run.cache_rows(layer, len(p) + new - 1)
        assert np.array_equal(k, wk) and np.array_equal(v, wv), layer


def one_ulp_flips(bits, fraction, rng):
    """bits with +-1 in the last place on a seeded random `fraction` of its
    nonzero finite entries (never producing a zero, infinity or NaN)."""
    out = bits.copy()
    mag = out & 0x7FFF
    candidates = np.nonzero((mag != 0) & (mag < 0x7F00))[0]
    idx = candidates[rng.random(candidates.size) < fraction]
    step = np.where(rng.random(idx.size) < 0.5, 1, -1)
    out[idx] = (out[idx].astype(np.int64) + step).astype(np.uint16)
    return out, idx.size


def exact_mfma_and_floor(model, p, fraction):
    """First logits of config 3's prompt three ways: the exact pass, the
    exact pass with one-ulp flips on `fraction` of block 0's cached K and V
    entries (the floor), and the MFMA pass."""
    from dolittle_amd.qwen3 import Plan
    n = len(p) - 1

    def first_logits(mfma=False, perturb=False):
        plan = Plan(model, batch=1, capacity=len(p) + 2)
        plan.prefill(p, mfma=mfma)
        flipped = 0
        if perturb:
            k, v = plan.read_cache(0, 0, n)
            rng = np.random.default_rng(7)
            k2, fk = one_ulp_flips(k, fraction, rng)
            v2, fv = one_ulp_flips(v, fraction, rng)
            plan.write_cache(0, 0, k2, v2)
            flipped = fk + fv
        plan.generate(p, 1)
        plan.collect()
        return plan.logits(0), flipped

    exact, _ = first_logits()
    floor, flipped = first_logits(perturb=True)
    mfma, _ = first_logits(mfma=True)
    return exact, floor, flipped, mfma


# The MFMA pass cannot meet the north star's logits bound or the reference's
# 36-block budget on this synthetic model, and neither can any other path
# that is not bit-exact: +-1 BF16 ulp on a handful of block 0's cached K/V
# entries of the exact pass already moves the first logits outside both
# (measured on MI355X with the prompts below: 9 flipped entries of 8.4
# million give max |d| 0.041 and 99.75% of logits inside at 2 blocks, and
# relative L2 0.039 at 36 blocks; 8,503 flips, 0.1%, give 0.047 / 98.8% and
# 0.041).  The MFMA GEMMs flip about that fraction of every projection's
# outputs.  The tests below assert that the bound cannot tell the MFMA pass
# from a one-ulp perturbation of the exact pass, and keep the bounds
# themselves as strict expected failures (a pass would report as a failure,
# so a change that meets a bound shows).  Config 3's parity path is the exact
# prompt pass (test_config3_exact_prefill_4096_two_blocks_matches_oracle).
FLOOR_FRACTION = 1e-3


@pytest.mark.timeout(900)
def test_config3_mfma_prefill_within_the_one_ulp_floor_two_blocks(two_blocks, config3_oracle, oracle):
    p, _, _, _, first_logits, _ = config3_oracle
    exact, floor, flipped, mfma = exact_mfma_and_floor(two_blocks, p, FLOOR_FRACTION)
    assert np.array_equal(exact, first_logits)  # the exact pass is the oracle's
    f = logit_errors(floor, exact, oracle)
    e = logit_errors(mfma, exact, oracle)
    print(f"2 blocks, first logits vs the oracle: {flipped} one-ulp K/V flips in block 0 {f}; MFMA pass {e}")
    assert flipped > 0 and f["north_star_frac"] < 1.0, f  # the floor already misses the bound
    assert e["rel_l2"] <= 1.5 * f["rel_l2"] and e["max_abs"] <= 1.5 * f["max_abs"], (e, f)


@pytest.mark.xfail(strict=True, reason="no path that is not bit-exact meets the north star's bound on this model: "
                                       "one-ulp flips in block 0's cache of the exact pass already miss it")
@pytest.mark.timeout(900)
def test_config3_mfma_prefill_4096_two_blocks_north_star_bound(two_blocks, config3_oracle, oracle):
    from dolittle_amd.qwen3 import Plan
    p, _, _, _, first_logits, _ = config3_oracle
    plan = Plan(two_blocks, batch=1, capacity=len(p) + 2)
    plan.prefill(p, mfma=True)
    plan.generate(p, 1)
    plan.collect()
    e = logit_errors(plan.logits(0), first_logits, oracle)
    print(f"MFMA prefill, 4096 ids, 2 blocks, first logits vs oracle: {e}")
    assert e["north_star_frac"] == 1.0, e


@pytest.mark.timeout(900)
def test_config3_mfma_prefill_within_the_one_ulp_floor_full_depth(full_model, oracle):
    exact, floor, flipped, mfma = exact_mfma_and_floor(full_model, prompt(4097, 4096), FLOOR_FRACTION)
    f = logit_errors(floor, exact, oracle)
    e = logit_errors(mfma, exact, oracle)
    print(f"36 blocks, first logits vs the exact pass: {flipped} one-ulp K/V flips in block 0 {f}; MFMA pass {e}")
    assert flipped > 0 and f["rel_l2"] > 0.03, f  # the floor already exceeds the reference's budget
    assert e["rel_l2"] <= 1.5 * f["rel_l2"] and e["max_abs"] <= 1.5 * f["max_abs"], (e, f)


@pytest.mark.xfail(strict=True, reason="no path that is not bit-exact meets the reference's 36-block budget on "
                                       "this model: one-ulp flips in block 0's cache of the exact pass exceed it")
@pytest.mark.timeout(900)
def test_config3_mfma_prefill_full_depth_against_exact(full_model, oracle):
    from dolittle_amd.qwen3 import Plan
    p = prompt(4097, 4096)
    exact = Plan(full_model, batch=1, capacity=len(p) + 2)
    exact.prefill(p)
    exact.generate(p, 1)
    exact.collect()
    mfma = Plan(full_model, batch=1, capacity=len(p) + 2)
    mfma.prefill(p, mfma=True)
    mfma.generate(p, 1)
    mfma.collect()
    e = logit_errors(mfma.logits(0), exact.logits(0), oracle)
    print(f"MFMA prefill, 4096 ids, 36 blocks, first logits vs the exact pass: {e}")
    assert e["max_abs"] <= max(1e-4, e["peak"] * 0.0625) and e["rel_l2"] <= 0.03, e


@pytest.mark.timeout(900)
def test_config3_decode_to_4608_keys_exact_prefill_equals_loop(full_model):
    from dolittle_amd.qwen3 import Plan
    p, new = prompt(4098, 4096), 512
    loop = Plan(full_model, batch=1, capacity=len(p) + new)
    loop.generate(p, new)
    want, results = loop.collect()
    assert results[0]["generated"] == new and results[0]["status"] == 0
    assert results[0]["position"] == len(p) + new
    pre = Plan(full_model, batch=1, capacity=len(p) + new)
    pre.prefill(p)
    pre.generate(p, new)
    got, results = pre.collect()
    assert results[0]["generated"] == new and results[0]["status"] == 0
    assert got[0].tolist() == want[0].tolist()
    assert np.array_equal(pre.logits(0), loop.logits(0))
    for layer in (0, 24, 35):
        k0, v0 = loop.read_cache(layer, 0, len(p) + new - 1)
        k1, v1 = pre.read_cache(layer, 0, len(p) + new - 1)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1), layer


@pytest.mark.timeout(900)
def test_config4_full_depth_capture_and_steering_match_oracle(full_model, full_weights, oracle):
    """BASELINE config 4 at its depth and prompt, reduced generation: 36
    blocks, batch 2, a 256-id prompt through the exact prompt pass, block-24
    capture at every consumed position, sequence 1 steered there at every
    position by a seeded N(0,1) FP32 vector normalised to unit length times
    8.0 (h <- BF16(FP32(h) + v)), 16 greedy tokens.  Tokens, the 272 captured
    rows of both sequences and their last logits equal the oracle's."""
    from dolittle_amd.qwen3 import Plan
    w, d = full_weights, full_weights.dims
    p, new, layer = prompt(4104, 256), 16, 24
    rng = np.random.default_rng(4105)
    v = rng.standard_normal(d.hidden).astype(np.float32)
    v = (v / np.float32(np.linalg.norm(v.astype(np.float64)))).astype(np.float32) * np.float32(8.0)
    plan = Plan(full_model, batch=2, capacity=len(p) + new + 1)
    plan.set_capture(layer)
    plan.set_steering(1, layer, v)
    plan.prefill(p)
    plan.generate(p, new)
    tokens, results = plan.collect()
    consumed = len(p) + new
    print(f"config 4: GPU done, {results}", flush=True)

    # Oracle: blocks 0..24 of the 255 prompt rows are shared; sequence 1 is
    # steered after block 24 and both continue through blocks 25..35.
    kw, cap, rows = d.kv_heads * d.head_dim, consumed + 1, len(p) - 1
    emb = w.embedding.reshape(d.vocab, d.hidden)
    caches = [([np.zeros(cap * kw, np.uint16) for _ in w.blocks], [np.zeros(cap * kw, np.uint16) for _ in w.blocks])
              for _ in range(2)]
    h = np.ascontiguousarray(emb[np.asarray(p[:-1], np.int64)].reshape(-1))
    for l in range(layer + 1):
        oracle.block_forward(w, l, h, rows, 0, caches[0][0][l], caches[0][1][l])
    hs = [h, h.copy()]
    for l in range(layer + 1):
        caches[1][0][l][:] = caches[0][0][l]
        caches[1][1][l][:] = caches[0][1][l]
    for r in range(rows):
        oracle.steer(hs[1][r * d.hidden:(r + 1) * d.hidden], v)
    captures = [hs[0].reshape(rows, d.hidden).copy(), hs[1].reshape(rows, d.hidden).copy()]
    for seq in (0, 1):
        for l in range(layer + 1, len(w.blocks)):
            oracle.block_forward(w, l, hs[seq], rows, 0, caches[seq][0][l], caches[seq][1][l])
    print("config 4: oracle prompt done", flush=True)
    for seq in (0, 1):
        stream, caps, logits = list(p), [captures[seq]], None
        for pos in range(rows, consumed):
            x = emb[stream[pos]].copy()
            for l in range(len(w.blocks)):
                oracle.block_forward(w, l, x, 1, pos, caches[seq][0][l], caches[seq][1][l])
                if l == layer:
                    if seq == 1:
                        oracle.steer(x, v)
                    caps.append(x.reshape(1, d.hidden).copy())
            if pos + 1 < consumed:
                logits = oracle.logits(w, x)
                status, nxt = oracle.greedy(logits)
                assert status == 0
                stream.append(nxt)
        assert results[seq]["generated"] == new and results[seq]["status"] == 0
        assert tokens[seq].tolist() == stream[len(p):], seq
        assert np.array_equal(plan.read_capture(seq, 0, consumed), np.concatenate(caps)), seq
        assert np.array_equal(plan.logits(seq), logits), seq
    assert tokens[0].tolist() != tokens[1].tolist()


@pytest.mark.timeout(900)
def test_config5_full_depth_injected_prefix_and_top_p_follow_the_law(full_model, full_weights, oracle):
    """BASELINE config 5 at its depth, batch and prefix, reduced generation:
    36 blocks, 8 samples sharing a 192-id prefix (exact prompt pass) whose
    embedding slot 57 is replaced by a BF16 N(0,1) x 40 row, then 8 tokens
    per sample at T 1.0, top-p 0.95 with per-sample MT19937-64 seeds.  The
    first selection's logits of every sample equal the oracle's (36 blocks
    over the injected prefix), and every sampled id equals the host law
    (categorical.cpp:146-201) applied to that step's device logits with the
    sample's k-th draw."""
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    w, d = full_weights, full_weights.dims
    p, new, slot = prompt(4106, 192), 8, 57
    row = oracle.normal_bf16(d.hidden, SEED + 11, 3000, 40.0)
    seeds = [1000 + 17 * b for b in range(8)]
    settings = SamplingSettings("categorical", 1.0, 0, 0.95)
    plan = Plan(full_model, batch=8, capacity=len(p) + new + 1)
    plan.set_embedding_override(slot, row, 0xFF)
    plan.prefill(p)
    plan.prepare_generation(p, new, settings, seeds)
    plan.decode_steps(1)  # consumes the last prefix position, selects token 0
    logits = []
    for step in range(new):
        logits.append([plan.logits(b) for b in range(8)])
        plan.decode_steps(1)
    tokens, results = plan.collect()
    print(f"config 5: GPU done, {[r['generated'] for r in results]}", flush=True)

    emb = w.embedding.reshape(d.vocab, d.hidden)
    kw, cap, rows = d.kv_heads * d.head_dim, len(p) + 1, len(p) - 1
    h = np.ascontiguousarray(emb[np.asarray(p[:-1], np.int64)])
    h[slot] = row
    h = h.reshape(-1)
    k = [np.zeros(cap * kw, np.uint16) for _ in w.blocks]
    vv = [np.zeros(cap * kw, np.uint16) for _ in w.blocks]
    for l in range(len(w.blocks)):
        oracle.block_forward(w, l, h, rows, 0, k[l], vv[l])
    x = emb[p[-1]].copy()
    for l in range(len(w.blocks)):
        oracle.block_forward(w, l, x, 1, rows, k[l], vv[l])
    first = oracle.logits(w, x)
    for b in range(8):
        assert np.array_equal(logits[0][b], first), b
    for b in range(8):
        assert results[b]["generated"] == new and results[b]["status"] == 0, results[b]
        draws = oracle.MT19937_64(seeds[b])
        for i in range(new):
            status, want = oracle.categorical_bits(oracle.f32_from_bf16(logits[i][b]), 1, 1.0, 0, 0.95, draws())
            assert status == 0 and tokens[b][i] == want, (b, i)
    assert len({tuple(t) for t in tokens.tolist()}) > 1
