"""Shared helpers of the GPU parity tests (imported by tests/test_gpu_*.py):
the resident model's weights read back into the oracle's row-major layout,
and the oracle's token loop in the Qwen3 recipe order
(src/models/qwen3/model.cpp:343-409)."""
import numpy as np

ROLES = (("input_norm", "input_norm"), ("wq", "q"), ("wk", "k"), ("wv", "v"), ("q_norm", "q_norm"),
         ("k_norm", "k_norm"), ("wo", "o"), ("post_norm", "post_norm"), ("wg", "gate"), ("wu", "up"),
         ("wd", "down"))


def read_weights(o, model, seed=None, std=0.02):
    """Row-major weights of every block read back from the device.  With a
    seed, a slice at the start and one at the end of every projection of
    every block is checked against the CPU generator (element i of (role,
    layer) is dl_normal_bf16(seed, 16 * layer + role, i)), so the weights the
    oracle uses are the seeded ones, not only what the device holds."""
    from dolittle_amd.qwen3 import ROLE
    cfg = model.config
    dims = o.Dims(cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab, cfg.rms_eps,
                  cfg.rope_theta)
    blocks = []
    for layer in range(cfg.layers):
        block = {name: np.ascontiguousarray(model.read(role, layer).reshape(-1)) for name, role in ROLES}
        if seed is not None:
            for name, role in ROLES:
                if not name.startswith("w"):
                    assert np.all(block[name] == 0x3F80), (layer, name)
                    continue
                a = block[name]
                stream = 16 * layer + ROLE[role]
                assert np.array_equal(a[:2048], o.normal_bf16(2048, seed, stream, std)), (layer, name)
                assert np.array_equal(a[-2048:], o.normal_bf16(2048, seed, stream, std, a.size - 2048)), (layer, name)
        blocks.append(block)
    lm = np.ascontiguousarray(model.read("lm_head").reshape(-1))
    if seed is not None and cfg.tied_embeddings:
        stream = ROLE["embedding"]
        assert np.array_equal(lm[:2048], o.normal_bf16(2048, seed, stream, std))
        assert np.array_equal(lm[-2048:], o.normal_bf16(2048, seed, stream, std, lm.size - 2048))
    emb = lm if cfg.tied_embeddings else np.ascontiguousarray(model.read("embedding").reshape(-1))
    return o.Qwen3Weights(dims, blocks, np.ascontiguousarray(model.read("final_norm")), lm, emb)


class OracleLoop:
    """The oracle composed as the reference's generation runs it: the prompt
    positions before the last as one chunk per block, then one position per
    step with the LM head and greedy selection."""

    def __init__(self, o, weights, capacity):
        self.o, self.w = o, weights
        d = weights.dims
        self.kw = d.kv_heads * d.head_dim
        self.k = [np.zeros(capacity * self.kw, np.uint16) for _ in weights.blocks]
        self.v = [np.zeros(capacity * self.kw, np.uint16) for _ in weights.blocks]
        self.emb = weights.embedding.reshape(d.vocab, d.hidden)

    def prompt(self, ids):
        """Positions [0, len(ids)) as one chunk per block."""
        h = np.ascontiguousarray(self.emb[np.asarray(ids, np.int64)].reshape(-1))
        for layer in range(len(self.w.blocks)):
            self.o.block_forward(self.w, layer, h, len(ids), 0, self.k[layer], self.v[layer])
        return h

    def step(self, token, position):
        h = self.emb[token].copy()
        for layer in range(len(self.w.blocks)):
            self.o.block_forward(self.w, layer, h, 1, position, self.k[layer], self.v[layer])
        return self.o.logits(self.w, h)

    def generate(self, ids, new):
        """Greedy tokens and the logits row of the last selection."""
        self.prompt(ids[:-1])
        seq, tokens, logits = list(ids), [], None
        for position in range(len(ids) - 1, len(ids) - 1 + new):
            logits = self.step(seq[position], position)
            status, token = self.o.greedy(logits)
            assert status == 0
            tokens.append(token)
            seq.append(token)
        return tokens, logits

    def cache_rows(self, layer, count):
        return self.k[layer][: count * self.kw], self.v[layer][: count * self.kw]


def logit_errors(got_bits, want_bits, o):
    """Deviation of a logits row from a reference row: max |d|, peak |want|,
    relative L2, and the fraction of entries inside |d| <= 2e-2 + 1e-2 |want|
    (the north star's absolute / relative bound)."""
    got = o.f32_from_bf16(got_bits).astype(np.float64)
    want = o.f32_from_bf16(want_bits).astype(np.float64)
    d = np.abs(got - want)
    return {
        "max_abs": float(d.max()),
        "peak": float(np.abs(want).max()),
        "rel_l2": float(np.linalg.norm(got - want) / np.linalg.norm(want)),
        "north_star_frac": float(np.mean(d <= 2e-2 + 1e-2 * np.abs(want))),
    }
