"""GPU upload of a safetensors checkpoint (dl_qwen3_load): a one-block
Qwen3-8B-width checkpoint (vocabulary 2048, untied, BF16) in two shards with
an index is opened with SHA-256 verification, bound as bind_causal_lm does
(src/models/qwen3/checkpoint.cpp) and streamed into the packed resident
layout; every parameter read back from the device equals the file's bytes.
A model whose config differs from the archive's is rejected."""
import json
import os
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CONFIG = {"model_type": "qwen3", "architectures": ["Qwen3ForCausalLM"], "hidden_act": "silu",
          "num_hidden_layers": 1, "hidden_size": 4096, "num_attention_heads": 32, "num_key_value_heads": 8,
          "head_dim": 128, "intermediate_size": 12288, "vocab_size": 2048, "max_position_embeddings": 40960,
          "rms_norm_eps": 1e-06, "rope_theta": 1000000, "torch_dtype": "bfloat16", "attention_bias": False,
          "tie_word_embeddings": False, "rope_scaling": None, "sliding_window": None,
          "use_sliding_window": False, "use_cache": True, "bos_token_id": 151643, "eos_token_id": 151645}

ROLES = ["embedding", "lm_head", "final_norm", "input_norm", "q", "k", "v", "q_norm", "k_norm", "o",
         "post_norm", "gate", "up", "down"]


def bf16_bits(x):
    return (np.asarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.fixture(scope="module")
def checkpoint_dir(tmp_path_factory):
    from dolittle_amd import checkpoint as ck
    from dolittle_amd.qwen3 import Qwen3Config
    root = str(tmp_path_factory.mktemp("qwen3"))
    cfg = Qwen3Config(layers=1, vocab=2048, tied_embeddings=False)
    rng = np.random.default_rng(7)
    arrays = {}
    for role in ROLES:
        layer = 0
        shape = cfg.shape(role)
        scale = 1.0 if role.endswith("norm") else 0.02
        arrays[ck.tensor_name(role, layer)] = (role, bf16_bits(rng.standard_normal(shape, np.float32) * scale))
    names = sorted(arrays)
    half = len(names) // 2
    shards = {"model-00001-of-00002.safetensors": names[:half], "model-00002-of-00002.safetensors": names[half:]}
    weight_map = {}
    for shard, members in shards.items():
        ck.write_safetensors(os.path.join(root, shard), {n: ("BF16", arrays[n][1]) for n in members},
                             {"format": "pt"})
        weight_map.update({n: shard for n in members})
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, f)
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump(CONFIG, f)
    return root, arrays, list(shards)


def test_load_reads_back_bit_exact(device, queue, checkpoint_dir):
    from dolittle_amd import checkpoint as ck
    root, arrays, shards = checkpoint_dir
    paths = ["config.json", "model.safetensors.index.json", *shards]
    artifacts = [ck.ArtifactSpec.of(root, p) for p in paths]
    t0 = time.perf_counter()
    archive = ck.open_archive(root, "Qwen/Qwen3-8B-test", "rev", artifacts, shards,
                              "model.safetensors.index.json", verification_workers=2)
    t1 = time.perf_counter()
    model = ck.load_qwen3(device, queue, archive)
    t2 = time.perf_counter()
    total = sum(a.nbytes for _, a in arrays.values())
    print(f"open+verify {t1 - t0:.2f} s, bind+upload {total / (t2 - t1) / 1e9:.2f} GB/s ({total / 1e6:.0f} MB)",
          flush=True)
    assert model.config.vocab == 2048 and not model.config.tied_embeddings
    for name, (role, array) in arrays.items():
        got = model.read(role, 0).reshape(array.shape)
        assert np.array_equal(got, array), name


def test_load_rejects_a_different_model(device, queue, checkpoint_dir):
    from dolittle_amd import _lib
    from dolittle_amd import checkpoint as ck
    from dolittle_amd.qwen3 import Qwen3Config, Qwen3Model
    root, _, shards = checkpoint_dir
    artifacts = [ck.ArtifactSpec.of(root, p) for p in ["config.json", *shards]]
    archive = ck.open_archive(root, "r", "v", artifacts, shards, integrity="prepared_setup")
    for cfg in (Qwen3Config(layers=1, vocab=2048, tied_embeddings=True),
                Qwen3Config(layers=1, vocab=4096, tied_embeddings=False)):
        model = Qwen3Model(device, queue, cfg)
        with pytest.raises(_lib.InvalidArgument):
            _lib.call("dl_qwen3_load", model.handle, queue.handle, archive.handle, b"config.json")
