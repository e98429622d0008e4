"""Checkpoint archives and the Qwen3 binding (host code of libdlhip.so; no
GPU).  The cases follow the reference's own contract tests,
tests/core/test_safetensors.cpp (valid_headers, invalid_headers,
limits_and_overflow) and tests/core/test_qwen3_checkpoint.cpp
(config_contracts, binding_contracts), with their JSON inputs; archive
opening is checked on temporary files, and SHA-256 against Python's
hashlib (an independent implementation)."""
import hashlib
import json
import os

import numpy as np
import pytest

from dolittle_amd import _lib
from dolittle_amd import checkpoint as ck

LIMITS = dict(max_header_bytes=1 << 20, max_metadata_bytes=1 << 20, max_tensor_count=100)


def parse(text, data_bytes, **limits):
    return ck.parse_header(text.encode() if isinstance(text, str) else text, data_bytes, **{**LIMITS, **limits})


# ------------------------------------------------ test_safetensors.cpp cases
def test_valid_headers():
    text = ('{"z":{"dtype":"BF16","shape":[2,3],"data_offsets":[4,16]},"a":{"dtype":"F32","shape":[],'
            '"data_offsets":[0,4]},"empty":{"dtype":"U32","shape":[9,0],"data_offsets":[16,16]},'
            '"__metadata__":{"format":"pt"}}   ')
    entries = {e.name: e for e in parse(text, 16).tensors()}
    assert set(entries) == {"a", "z", "empty"}
    assert entries["a"].shape == () and entries["a"].byte_count == 4 and entries["a"].dtype == "F32"
    assert entries["z"].dtype == "BF16" and entries["z"].shape == (2, 3) and entries["z"].data_offset == 4
    assert entries["empty"].byte_count == 0 and entries["empty"].dtype == "U32"
    assert sum(e.byte_count for e in entries.values()) == 16
    assert [e.name for e in parse(text, 16).tensors()] == ["a", "empty", "z"]  # name order
    assert parse("{}", 0).tensors() == []


@pytest.mark.parametrize("text", [
    '{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}',
    '{"x":{"dtype":"F32","dtype":"BF16","shape":[2],"data_offsets":[0,4]}}',
    '{"__metadata__":{"a":"one","a":"two"}}',
    '{"__metadata__":{"a":3}}',
    '{"x":{"dtype":"F16","shape":[2],"data_offsets":[0,4]}}',
    '{"x":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}',
    '{"x":{"dtype":"F32","shape":[1.0],"data_offsets":[0,4]}}',
    '{"x":{"dtype":"F32","shape":[1],"data_offsets":[-1,3]}}',
    '{"x":{"dtype":"F32","shape":[1],"data_offsets":[4,0]}}',
    '{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}',
    '{"x":{"dtype":"F32","shape":[1],"data_offsets":[1,5]}}',
    '{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4],"extra":true}}',
    '{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"y":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}',
    '{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}} trailing',
    " {}", "[]", "{", "{}",
])
def test_invalid_headers(text):
    with pytest.raises(_lib.InvalidArgument):
        parse(text, 4)


def test_gap_is_invalid():
    with pytest.raises(_lib.InvalidArgument):
        parse('{"x":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}', 8)


@pytest.mark.parametrize("limits", [dict(max_header_bytes=4, max_tensor_count=10),
                                    dict(max_metadata_bytes=4, max_tensor_count=10),
                                    dict(max_tensor_count=0)])
def test_limits(limits):
    with pytest.raises(_lib.LengthError):
        parse('{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', 4, **limits)


def test_overflow_and_nesting():
    overflow = '{"x":{"dtype":"F32","shape":[%d],"data_offsets":[0,4]}}' % (2 ** 64 - 1)
    with pytest.raises(_lib.LengthError):
        parse(overflow, 4)
    nested = '{"x":' + "[" * 65 + "0" + "]" * 65 + "}"
    with pytest.raises(_lib.LengthError):
        parse(nested, 0)
    # 63 arrays under the root object is the deepest accepted nesting; the
    # descriptor is then malformed, not over the limit.
    with pytest.raises(_lib.InvalidArgument):
        parse('{"x":' + "[" * 63 + "0" + "]" * 63 + "}", 0)


def test_json_text_rules():
    ok = '{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"__metadata__":{"k":"%s"}}'
    for s in ["\\u00e9", "\\ud83d\\ude00", "café", "tab\\t"]:
        parse((ok % s).encode("utf-8"), 4)
    for s in ["\\ud83d", "\\ude00", "\x01", "\\x"]:
        with pytest.raises(_lib.InvalidArgument):
            parse((ok % s).encode("utf-8"), 4)
    with pytest.raises(_lib.InvalidArgument):  # invalid UTF-8
        parse((ok % "A").encode().replace(b"A", b"\xc3\x28"), 4)
    with pytest.raises(_lib.InvalidArgument):  # nonfinite number
        parse('{"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"y":1e999}', 4)


# ------------------------------------------------ test_qwen3_checkpoint.cpp
CONFIG = ('{"model_type":"qwen3","architectures":["Qwen3ForCausalLM"],"hidden_act":"silu","num_hidden_layers":1,'
          '"hidden_size":4,"num_attention_heads":2,"num_key_value_heads":1,"head_dim":2,"intermediate_size":6,'
          '"vocab_size":7,"max_position_embeddings":16,"rms_norm_eps":0.000001,"rope_theta":10000,'
          '"torch_dtype":"float32","attention_bias":false,"tie_word_embeddings":false,"rope_scaling":null,'
          '"sliding_window":null,"use_sliding_window":false,"use_cache":true}')


def test_config_contracts():
    cfg, context = ck.parse_config(CONFIG.encode(), "float32", 1 << 20)
    assert (cfg.layers, cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab, context) == \
        (1, 4, 2, 1, 2, 6, 7, 16)
    assert not cfg.tied_embeddings and cfg.rope_theta == 10000 and cfg.rms_eps == np.float32(1e-6)
    ck.parse_config(CONFIG.replace("float32", "bfloat16").encode(), "bfloat16", 1 << 20)
    for before, after in [
            ('"qwen3"', '"qwen2"'), ('"silu"', '"gelu"'), ('"attention_bias":false', '"attention_bias":true'),
            ('"tie_word_embeddings":false', '"tie_word_embeddings":true'),
            ('"rope_scaling":null', '"rope_scaling":{"rope_type":"yarn"}'),
            ('"sliding_window":null', '"sliding_window":8'), ('"head_dim":2', '"head_dim":3'),
            ('"num_key_value_heads":1', '"num_key_value_heads":3'),
            ('"num_hidden_layers":1', '"num_hidden_layers":-1'), ('"hidden_size":4', '"hidden_size":4.0'),
            ('"rope_theta":10000', '"rope_theta":0'), ('"rms_norm_eps":0.000001', '"rms_norm_eps":-1'),
            ('"float32"', '"bfloat16"'), ('"use_cache":true', '"use_cache":true,"unknown_behavior":true'),
            ('"use_cache":true', '"use_cache":true,"head_dim":2'),
            ('"use_cache":true', '"use_cache":true,"layer_types":["sliding_attention"]'),
            ('"use_cache":true', '"use_cache":true,"_name_or_path":{"x":1,"x":2}')]:
        assert before in CONFIG
        with pytest.raises(_lib.InvalidArgument):
            ck.parse_config(CONFIG.replace(before, after, 1).encode(), "float32", 1 << 20)
    with pytest.raises(_lib.LengthError):
        ck.parse_config(CONFIG.encode(), "float32", 1)
    with pytest.raises(_lib.LengthError):
        ck.parse_config(CONFIG.replace('"num_hidden_layers":1', '"num_hidden_layers":100000000').encode(),
                        "float32", 1 << 20)


SHAPES = [("model.embed_tokens.weight", (7, 4)), ("model.norm.weight", (4,)), ("lm_head.weight", (7, 4)),
          ("model.layers.0.input_layernorm.weight", (4,)),
          ("model.layers.0.post_attention_layernorm.weight", (4,)),
          ("model.layers.0.self_attn.q_proj.weight", (4, 4)), ("model.layers.0.self_attn.k_proj.weight", (2, 4)),
          ("model.layers.0.self_attn.v_proj.weight", (2, 4)), ("model.layers.0.self_attn.o_proj.weight", (4, 4)),
          ("model.layers.0.self_attn.q_norm.weight", (2,)), ("model.layers.0.self_attn.k_norm.weight", (2,)),
          ("model.layers.0.mlp.gate_proj.weight", (6, 4)), ("model.layers.0.mlp.up_proj.weight", (6, 4)),
          ("model.layers.0.mlp.down_proj.weight", (4, 6))]


def catalog(entries, dtype="F32"):
    """A decoded header holding `entries` (name, shape) in that member order."""
    header, offset = {}, 0
    for name, shape in entries:
        n = int(np.prod(shape, dtype=np.int64)) * (2 if dtype == "BF16" else 4)
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + n]}
        offset += n
    return parse(json.dumps(header), offset)


def test_binding_contracts():
    cfg, _ = ck.parse_config(CONFIG.encode(), "float32", 1 << 20)
    ck.bind_parameters(cfg, "float32", catalog(SHAPES))
    ck.bind_parameters(cfg, "float32", catalog(SHAPES[::-1]))  # order independent
    assert ck.tensor_name("embedding") == "model.embed_tokens.weight"
    assert ck.tensor_name("lm_head") == "lm_head.weight"
    assert ck.tensor_name("q_norm", 0) == "model.layers.0.self_attn.q_norm.weight"
    assert ck.tensor_name("down", 35) == "model.layers.35.mlp.down_proj.weight"
    invalid = [SHAPES[:-1], SHAPES + [("model.extra.weight", (1,))], [("unexpected.weight", (7, 4))] + SHAPES[1:],
               [("model.embed_tokens.weight", (4, 7))] + SHAPES[1:]]
    for entries in invalid:
        with pytest.raises(_lib.InvalidArgument):
            ck.bind_parameters(cfg, "float32", catalog(entries))
    with pytest.raises(_lib.InvalidArgument):  # BF16 payloads under an FP32 config
        ck.bind_parameters(cfg, "float32", catalog(SHAPES, "BF16"))


# ------------------------------------------------------------- SHA-256
@pytest.mark.parametrize("n", [0, 1, 3, 55, 56, 63, 64, 65, 119, 1000, 1 << 20])
def test_sha256_matches_hashlib(n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert ck.sha256_hex(data) == hashlib.sha256(data).hexdigest()
    assert ck.sha256_hex(b"abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"


# ---------------------------------------------------------- archive open
def make_archive(root, dtype="F32"):
    """Two shards, an index and the test config; returns (artifacts, arrays)."""
    rng = np.random.default_rng(1)
    arrays = {}
    for name, shape in SHAPES:
        if dtype == "F32":
            arrays[name] = rng.standard_normal(shape).astype(np.float32)
        else:
            arrays[name] = rng.integers(0, 1 << 16, shape, dtype=np.uint16)
    names = sorted(arrays)
    first, second = names[:7], names[7:]
    ck.write_safetensors(os.path.join(root, "model-1.safetensors"), {n: (dtype, arrays[n]) for n in first},
                         {"format": "pt"})
    ck.write_safetensors(os.path.join(root, "model-2.safetensors"), {n: (dtype, arrays[n]) for n in second})
    index = {"metadata": {"total_size": 0}, "weight_map": {
        **{n: "model-1.safetensors" for n in first}, **{n: "model-2.safetensors" for n in second}}}
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump(index, f)
    config = CONFIG if dtype == "F32" else CONFIG.replace("float32", "bfloat16")
    with open(os.path.join(root, "config.json"), "w") as f:
        f.write(config)
    paths = ["config.json", "model-1.safetensors", "model-2.safetensors", "model.safetensors.index.json"]
    return [ck.ArtifactSpec.of(root, p) for p in paths], arrays


SHARDS = ["model-1.safetensors", "model-2.safetensors"]


def manifest_digest(artifacts):
    h = hashlib.sha256(b"dolittle-artifacts-v1")
    for a in sorted(artifacts, key=lambda a: a.relative_path.encode()):
        p = a.relative_path.encode()
        h.update(len(p).to_bytes(8, "little") + p + a.byte_size.to_bytes(8, "little") + a.sha256.lower().encode())
    return h.hexdigest()


@pytest.mark.parametrize("workers", [1, 3])
def test_open_archive(tmp_path, workers):
    root = str(tmp_path)
    artifacts, arrays = make_archive(root)
    archive = ck.open_archive(root, "test/repository", "revision", artifacts, SHARDS,
                              "model.safetensors.index.json", verification_workers=workers)
    entries = archive.tensors()
    assert [e.name for e in entries] == sorted(arrays)[:7] + sorted(arrays)[7:]
    for e in entries:
        assert archive.payload(e.name) == arrays[e.name].tobytes()
        assert e.shape == arrays[e.name].shape
    assert archive.identity() == ("test/repository", "revision", manifest_digest(artifacts))
    assert archive.artifact("config.json") == CONFIG.encode()
    cfg, context, total = ck.bind_archive(archive)
    assert (cfg.layers, cfg.hidden, cfg.vocab, context) == (1, 4, 7, 16)
    assert total == sum(a.nbytes for a in arrays.values())


def test_open_archive_rejections(tmp_path):
    root = str(tmp_path)
    artifacts, _ = make_archive(root)
    index = "model.safetensors.index.json"

    def attempt(arts=artifacts, shards=SHARDS, idx=index, **kw):
        return ck.open_archive(root, "r", "v", arts, shards, idx, **kw)

    def replace(path, **changes):
        return [ck.ArtifactSpec(**{**a.__dict__, **changes}) if a.relative_path == path else a for a in artifacts]

    wrong = replace("config.json", sha256="0" * 64)
    with pytest.raises(_lib.DeviceError):  # digest mismatch is a runtime error
        attempt(wrong)
    attempt(wrong, integrity="prepared_setup")  # sizes only
    with pytest.raises(_lib.InvalidArgument):
        attempt(replace("config.json", sha256="z" * 64), integrity="prepared_setup")
    with pytest.raises(_lib.DeviceError):
        attempt(replace("config.json", byte_size=artifacts[0].byte_size + 1))
    for path in ["../config.json", "a//b", "./config.json", "/etc/passwd", "a\\b", "dir/"]:
        with pytest.raises(_lib.InvalidArgument):
            attempt(artifacts + [ck.ArtifactSpec(path, 0, "0" * 64)])
    with pytest.raises(_lib.InvalidArgument):  # shard not declared
        attempt(shards=SHARDS + ["other.safetensors"])
    with pytest.raises(_lib.InvalidArgument):  # index may not be a shard
        attempt(shards=SHARDS + [index])
    with pytest.raises(_lib.InvalidArgument):
        attempt(verification_workers=0)
    with pytest.raises(_lib.InvalidArgument):  # the index names the tensors of both shards
        attempt(shards=SHARDS[:1])
    with pytest.raises(_lib.LengthError):
        attempt(max_header_bytes=16)
    os.symlink("/etc/hostname", os.path.join(root, "escape"))
    with pytest.raises(_lib.InvalidArgument):
        attempt(artifacts + [ck.ArtifactSpec("escape", os.path.getsize("/etc/hostname"), "0" * 64)],
                integrity="prepared_setup")


def test_index_and_shard_mismatches(tmp_path):
    root = str(tmp_path)
    artifacts, arrays = make_archive(root)
    with open(os.path.join(root, "model.safetensors.index.json")) as f:
        index = json.load(f)
    for change in ["shard", "extra"]:
        bad = json.loads(json.dumps(index))
        if change == "shard":
            name = next(iter(bad["weight_map"]))
            bad["weight_map"][name] = "model-2.safetensors" if bad["weight_map"][name] != "model-2.safetensors" \
                else "model-1.safetensors"
        else:
            bad["extra"] = 1
        with open(os.path.join(root, "bad.json"), "w") as f:
            json.dump(bad, f)
        arts = artifacts + [ck.ArtifactSpec.of(root, "bad.json")]
        with pytest.raises(_lib.InvalidArgument):
            ck.open_archive(root, "r", "v", arts, SHARDS, "bad.json")
    # The same tensor in two shards.
    name = sorted(arrays)[0]
    ck.write_safetensors(os.path.join(root, "dup.safetensors"), {name: ("F32", arrays[name])})
    arts = artifacts + [ck.ArtifactSpec.of(root, "dup.safetensors")]
    with pytest.raises(_lib.InvalidArgument):
        ck.open_archive(root, "r", "v", arts, SHARDS + ["dup.safetensors"])
    # A truncated header.
    with open(os.path.join(root, "cut.safetensors"), "wb") as f:
        f.write((1000).to_bytes(8, "little") + b"{}")
    arts = artifacts + [ck.ArtifactSpec.of(root, "cut.safetensors")]
    with pytest.raises(_lib.InvalidArgument):
        ck.open_archive(root, "r", "v", arts, ["cut.safetensors"])


def test_bind_archive_bf16(tmp_path):
    root = str(tmp_path)
    artifacts, _ = make_archive(root, dtype="BF16")
    archive = ck.open_archive(root, "r", "v", artifacts, SHARDS, "model.safetensors.index.json")
    cfg, _, total = ck.bind_archive(archive)
    assert total == sum(int(np.prod(s)) * 2 for _, s in SHAPES)
    with pytest.raises(_lib.InvalidArgument):  # unknown configuration artifact
        ck.bind_archive(archive, "missing.json")
