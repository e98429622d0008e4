"""The acceptance-fixture runner (dolittle_amd/fixtures.py) on a bundle in
the reference's fixture.json format (scripts/validation/forward_reference.py,
schema_version 1): a two-block Qwen3-8B-width checkpoint (vocabulary 2048,
untied) whose reference rows come from the CPU contract mirror.  The runner
opens the bundle through the verified archive path, replays the three cases
and the generation case through the token loop, and must pass every output
with zero error; a perturbed logit and a wrong generated ID must fail.  The
real Qwen3-8B bundles need the downloaded checkpoint, which this image lacks."""
import copy
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CONFIG = {"model_type": "qwen3", "architectures": ["Qwen3ForCausalLM"], "hidden_act": "silu",
          "num_hidden_layers": 2, "hidden_size": 4096, "num_attention_heads": 32, "num_key_value_heads": 8,
          "head_dim": 128, "intermediate_size": 12288, "vocab_size": 2048, "max_position_embeddings": 64,
          "rms_norm_eps": 1e-06, "rope_theta": 1000000, "torch_dtype": "bfloat16", "attention_bias": False,
          "tie_word_embeddings": False, "rope_scaling": None, "sliding_window": None,
          "use_sliding_window": False, "use_cache": False}
ROLES = ["input_norm", "q", "k", "v", "q_norm", "k_norm", "o", "post_norm", "gate", "up", "down"]
ORACLE_NAMES = {"input_norm": "input_norm", "q": "wq", "k": "wk", "v": "wv", "q_norm": "q_norm",
                "k_norm": "k_norm", "o": "wo", "post_norm": "post_norm", "gate": "wg", "up": "wu", "down": "wd"}


def bf16_bits(x):
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def tolerance(values):
    # forward_reference.py tolerance() for a BF16 model of at most three blocks.
    peak = max((abs(v) for v in values), default=0.0)
    return {"max_absolute_error": max(1e-4, peak * 0.03125), "max_relative_l2": 0.02}


def rows_entry(rows, positions):
    values = np.concatenate([rows[p] for p in positions]).astype(np.float64).tolist()
    return {"positions": list(positions), "width": int(rows[0].size), "original_storage_type": "bfloat16",
            "values": values, "tolerance": tolerance(values)}


def evaluate(o, w, name, tokens, all_rows=False):
    """The mirror's forward of `tokens` with the fixture's output selection."""
    d = w.dims
    blocks = len(w.blocks)
    kw = d.kv_heads * d.head_dim
    k = [np.zeros(64 * kw, np.uint16) for _ in w.blocks]
    v = [np.zeros(64 * kw, np.uint16) for _ in w.blocks]
    n = len(tokens)
    observed = sorted({0, blocks // 2, blocks - 1})
    positions = list(range(n)) if all_rows else sorted({0, n // 2, n - 1})
    logit_positions = list(range(n)) if all_rows else sorted({0, n - 1})
    inputs = {b: {} for b in observed}
    outputs = {b: {} for b in observed}
    logits = {}
    f32 = lambda bits: (bits.astype(np.uint32) << 16).view(np.float32)
    for pos, token in enumerate(tokens):
        h = w.embedding.reshape(d.vocab, d.hidden)[token].copy()
        for layer in range(blocks):
            if layer in inputs:
                inputs[layer][pos] = f32(h.copy())
            o.block_forward(w, layer, h, 1, pos, k[layer], v[layer])
            if layer in outputs:
                outputs[layer][pos] = f32(h.copy())
        if pos in logit_positions:
            logits[pos] = f32(o.logits(w, h))
    captures = []
    for b in observed:
        captures.append({"boundary": "block_input", "block": b, **rows_entry(inputs[b], positions)})
        captures.append({"boundary": "block_output", "block": b, **rows_entry(outputs[b], positions)})
    return {"name": name, "token_ids": list(tokens), "logit_positions": logit_positions,
            "logits": rows_entry(logits, logit_positions), "captures": captures}


@pytest.fixture(scope="module")
def bundle(tmp_path_factory, oracle):
    from dolittle_amd import checkpoint as ck
    from dolittle_amd.qwen3 import Qwen3Config
    root = str(tmp_path_factory.mktemp("bundle"))
    cfg = Qwen3Config(layers=2, vocab=2048, tied_embeddings=False)
    rng = np.random.default_rng(11)
    tensors, blocks = {}, []
    for layer in range(cfg.layers):
        block = {}
        for role in ROLES:
            scale = 1.0 if role.endswith("norm") else 0.02
            bits = bf16_bits(rng.standard_normal(cfg.shape(role), np.float32) * scale)
            tensors[ck.tensor_name(role, layer)] = ("BF16", bits)
            block[ORACLE_NAMES[role]] = np.ascontiguousarray(bits.reshape(-1))
        blocks.append(block)
    glob = {}
    for role in ("embedding", "lm_head", "final_norm"):
        scale = 1.0 if role == "final_norm" else 0.02
        glob[role] = bf16_bits(rng.standard_normal(cfg.shape(role), np.float32) * scale)
        tensors[ck.tensor_name(role)] = ("BF16", glob[role])
    names = sorted(tensors)
    shards = {"model-00001-of-00002.safetensors": names[:12], "model-00002-of-00002.safetensors": names[12:]}
    for shard, members in shards.items():
        ck.write_safetensors(os.path.join(root, shard), {n: tensors[n] for n in members})
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": {n: s for s, m in shards.items() for n in m}}, f)
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump(CONFIG, f)
    o = oracle
    dims = o.Dims(cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab, cfg.rms_eps,
                  cfg.rope_theta)
    w = o.Qwen3Weights(dims, blocks, np.ascontiguousarray(glob["final_norm"]),
                       np.ascontiguousarray(glob["lm_head"].reshape(-1)),
                       np.ascontiguousarray(glob["embedding"].reshape(-1)))
    tokens = [(i * 7 + 3) % 2048 for i in range(8)]
    cases = [evaluate(o, w, "full", tokens), evaluate(o, w, "prefix", tokens[:3]),
             evaluate(o, w, "alternate", [(t + 5) % 2048 for t in tokens])]
    prompt = [3, 10, 17, 24, 31]
    trace = list(prompt)
    run = evaluate  # greedy IDs from the mirror's logits of the growing prefix
    for _ in range(4):
        last = run(o, w, "step", trace)["logits"]
        row = np.asarray(last["values"][-2048:], np.float32)
        status, nxt = o.greedy(bf16_bits(row))
        assert status == 0
        trace.append(int(nxt))
    generation = {"prompt_tokens": len(prompt), "max_new_tokens": 4, "text": None,
                  "reference": evaluate(o, w, "generation", trace, all_rows=True)}
    paths = ["config.json", "model.safetensors.index.json", *shards]
    artifacts = [ck.ArtifactSpec.of(root, p).__dict__ for p in paths]
    fixture = {"schema_version": 1, "repository": "test/tiny-width-qwen3", "revision": "seed-11",
               "config_artifact": "config.json", "dtype": "bfloat16", "artifacts": artifacts,
               "shards": sorted(shards), "index": "model.safetensors.index.json", "reference": {},
               "tolerances": {}, "cases": cases, "generation": generation}
    with open(os.path.join(root, "fixture.json"), "w") as f:
        json.dump(fixture, f)
    return root, fixture


def test_bundle_passes_with_zero_error(device, queue, bundle):
    from dolittle_amd.fixtures import run_bundle
    root, _ = bundle
    report = run_bundle(device, queue, root)
    assert report["passed"], report
    outputs = [o for c in report["cases"].values() for o in c.values()]
    outputs += [v for k, v in report["generation"].items() if k != "generated_ids"]
    assert len(outputs) == 3 * 5 + 5
    assert all(o["errors"]["max_absolute_error"] == 0.0 for o in outputs)
    assert report["generation"]["generated_ids"]["passed"]


def test_bundle_failures_are_reported(device, queue, bundle):
    from dolittle_amd.fixtures import run_bundle
    root, fixture = bundle
    bad = copy.deepcopy(fixture)
    bad["cases"][0]["logits"]["values"][5] += 10.0
    report = run_bundle(device, queue, root, bad)
    assert not report["passed"] and not report["cases"]["full"]["logits"]["passed"]
    assert report["cases"]["prefix"]["logits"]["passed"]
    bad = copy.deepcopy(fixture)
    ids = bad["generation"]["reference"]["token_ids"]
    ids[-1] = (ids[-1] + 1) % 2048
    report = run_bundle(device, queue, root, bad)
    assert not report["generation"]["generated_ids"]["passed"] and not report["passed"]
