"""Pins of the oracle's composed Qwen3 block and head
(orc_qwen3_block_forward, orc_qwen3_logits), which restate the recipe of
src/models/qwen3/model.cpp:343-409:

    x = RMSNorm(h, input_norm); q, k, v = x Wq, x Wk, x Wv;
    q, k = RoPE(RMSNorm_head(q, q_norm)), RoPE(RMSNorm_head(k, k_norm));
    cache append; a = attention; h = h + a Wo;
    x = RMSNorm(h, post_norm); h = h + (SiLU(x Wg) * (x Wu)) Wd
    logits = RMSNorm(h_last, final_norm) W_lm

Every operator under the composition is pinned on its own
(test_oracle_ops.py, test_oracle_kat.py).  These tests pin the wiring with
weights chosen so that the block's output has a closed form, and so that a
plausible composition mistake changes it: gate and up exchanged, a norm fed
the wrong input or the wrong gains, the GQA group mapping transposed, V
taken before the norm, the final norm skipped.  Gains differ per role
(1.5, 0.75, 1.25, 3.0, 2.0) so a role mix-up moves the values.
"""
import numpy as np

D, HQ, HKV, HD, F, V = 256, 4, 2, 128, 512, 300
QW, KW = HQ * HD, HKV * HD
EPS, THETA = 1e-6, 1e6


def bf16_const(value, n):
    from oracle import bf16_from_f32
    return bf16_from_f32(np.full(n, value, np.float32))


def dims(o):
    return o.Dims(D, HQ, HKV, HD, F, V, EPS, THETA)


def block(o, rng_seed, **override):
    """Random BF16 weights N(0, 0.05) with distinct norm gains per role."""
    b = {
        "input_norm": bf16_const(1.5, D), "q_norm": bf16_const(0.75, HD), "k_norm": bf16_const(1.25, HD),
        "post_norm": bf16_const(3.0, D),
        "wq": o.normal_bf16(QW * D, rng_seed, 1, 0.05), "wk": o.normal_bf16(KW * D, rng_seed, 2, 0.05),
        "wv": o.normal_bf16(KW * D, rng_seed, 3, 0.05), "wo": o.normal_bf16(D * QW, rng_seed, 4, 0.05),
        "wg": o.normal_bf16(F * D, rng_seed, 5, 0.05), "wu": o.normal_bf16(F * D, rng_seed, 6, 0.05),
        "wd": o.normal_bf16(D * F, rng_seed, 7, 0.05),
    }
    b.update(override)
    return {k: np.ascontiguousarray(v, np.uint16) for k, v in b.items()}


def weights(o, blk, final_gain=2.0, lm=None):
    lm = np.zeros(V * D, np.uint16) if lm is None else lm
    return o.Qwen3Weights(dims(o), [blk], bf16_const(final_gain, D), lm, lm)


def run_block(o, w, h, first, k_cache, v_cache, rows=1):
    h = np.ascontiguousarray(h.copy(), np.uint16)
    o.block_forward(w, 0, h, rows, first, k_cache, v_cache)
    return h


def test_zero_output_projections_make_the_block_the_identity(oracle):
    """Wo = Wd = 0: the block leaves h unchanged (both residual additions add
    +0), while the cache rows at the position still equal
    K = RoPE(RMSNorm_head(RMSNorm(h) Wk)) and V = RMSNorm(h) Wv: V from the
    normalized row, not from h, and each with its own gains."""
    o = oracle
    zero_o, zero_d = np.zeros(D * QW, np.uint16), np.zeros(D * F, np.uint16)
    w = weights(o, block(o, 11, wo=zero_o, wd=zero_d))
    first = 5
    h = o.normal_bf16(D, 12, 0, 1.0)
    k = np.zeros(8 * KW, np.uint16)
    v = np.zeros(8 * KW, np.uint16)
    k[: first * KW] = o.normal_bf16(first * KW, 13, 0, 1.0)
    v[: first * KW] = o.normal_bf16(first * KW, 13, 1, 1.0)
    k0, v0 = k.copy(), v.copy()
    out = run_block(o, w, h, first, k, v)
    assert np.array_equal(out, h)

    b = w.blocks[0]
    x = o.rms_norm(h, b["input_norm"], 1, D, EPS)
    kraw = o.projection(x, b["wk"], 1, D, KW)
    knorm = o.rms_norm(kraw, b["k_norm"], HKV, HD, EPS)
    want_k = o.rotary(knorm, 1, HKV, HD, first, THETA)
    want_v = o.projection(x, b["wv"], 1, D, KW)
    assert np.array_equal(k[first * KW:(first + 1) * KW], want_k)
    assert np.array_equal(v[first * KW:(first + 1) * KW], want_v)
    # Rows before the position are untouched; the rows after stay empty.
    assert np.array_equal(k[: first * KW], k0[: first * KW]) and np.array_equal(v[: first * KW], v0[: first * KW])
    assert not k[(first + 1) * KW:].any() and not v[(first + 1) * KW:].any()
    # The mistakes this rules out produce other rows.
    assert not np.array_equal(want_v, o.projection(h, b["wv"], 1, D, KW))
    assert not np.array_equal(want_k, o.rotary(o.rms_norm(kraw, b["q_norm"], HKV, HD, EPS), 1, HKV, HD, first,
                                               THETA))


def test_one_visible_key_attends_to_its_own_value_row(oracle):
    """At position 0 the only visible key is the token's own: p = e/l = 1,
    so query head j's attention output is V row of kv head j // (HQ / HKV),
    and with Wd = 0 the block output is h + round(att Wo)."""
    o = oracle
    w = weights(o, block(o, 21, wd=np.zeros(D * F, np.uint16)))
    b = w.blocks[0]
    h = o.normal_bf16(D, 22, 0, 1.0)
    k = np.zeros(4 * KW, np.uint16)
    v = np.zeros(4 * KW, np.uint16)
    out = run_block(o, w, h, 0, k, v)

    x = o.rms_norm(h, b["input_norm"], 1, D, EPS)
    vrow = o.projection(x, b["wv"], 1, D, KW).reshape(HKV, HD)
    group = HQ // HKV
    att = np.concatenate([vrow[j // group] for j in range(HQ)])
    want = o.add(h, o.projection(att, b["wo"], 1, QW, D))
    assert np.array_equal(out, want)
    # A transposed group mapping (j % HKV) gives another row.
    wrong = np.concatenate([vrow[j % HKV] for j in range(HQ)])
    assert not np.array_equal(want, o.add(h, o.projection(wrong, b["wo"], 1, QW, D)))


def test_silu_gate_times_up_with_selector_rows(oracle):
    """Wo = 0; gate row j is c * e_m with x[m] the largest positive
    normalized feature, so gate_j = BF16(c x[m]) is about 32 and SiLU(gate_j)
    rounds to gate_j exactly (sigma = 1.0f); up row j selects feature j and
    down row i selects activation i.  The block output is then
    h_i + BF16(gate_i * x_i) with x = RMSNorm(h, post_norm): exchanging gate
    and up, or normalizing with the input gains, gives other values."""
    from oracle import bf16_from_f32, f32_from_bf16
    o = oracle
    h = o.normal_bf16(D, 32, 0, 1.0)
    post = bf16_const(3.0, D)
    x = o.rms_norm(h, post, 1, D, EPS)
    xf = f32_from_bf16(x)
    m = int(np.argmax(xf))
    assert xf[m] > 0
    c = bf16_from_f32(np.array([32.0 / xf[m]], np.float32))[0]
    wg = np.zeros((F, D), np.uint16)
    wu = np.zeros((F, D), np.uint16)
    wd = np.zeros((D, F), np.uint16)
    for j in range(D):
        wg[j, m] = c
        wu[j, j] = 0x3F80
        wd[j, j] = 0x3F80
    w = weights(o, block(o, 31, wo=np.zeros(D * QW, np.uint16), wg=wg.reshape(-1), wu=wu.reshape(-1),
                         wd=wd.reshape(-1)))
    k = np.zeros(4 * KW, np.uint16)
    v = np.zeros(4 * KW, np.uint16)
    out = run_block(o, w, h, 0, k, v)

    gate = f32_from_bf16(bf16_from_f32(np.array([f32_from_bf16(np.array([c]))[0] * xf[m]], np.float32)))[0]
    assert gate > 20.0
    act = f32_from_bf16(bf16_from_f32((np.float32(gate) * xf).astype(np.float32)))
    want = bf16_from_f32((f32_from_bf16(h) + act).astype(np.float32))
    assert np.array_equal(out, want)
    # gate and up exchanged: SiLU(x_j) * gate.
    swapped = f32_from_bf16(o.silu_multiply(x, bf16_from_f32(np.full(D, gate, np.float32))))
    assert not np.array_equal(want, bf16_from_f32((f32_from_bf16(h) + swapped).astype(np.float32)))
    # the input norm's gains instead of the post-attention norm's.
    x_in = f32_from_bf16(o.rms_norm(h, bf16_const(1.5, D), 1, D, EPS))
    act_in = f32_from_bf16(bf16_from_f32((np.float32(gate) * x_in).astype(np.float32)))
    assert not np.array_equal(want, bf16_from_f32((f32_from_bf16(h) + act_in).astype(np.float32)))


def test_logits_are_the_head_applied_to_the_final_norm(oracle):
    """Zero blocks: logits = RMSNorm(h, final_norm) W_lm.  With final gains
    2.0 (an exact doubling) and LM head row j selecting feature j mod D,
    logit j = BF16(2 BF16(h_{j mod D} * inverse)), inverse from the pinned
    reduction."""
    from oracle import bf16_from_f32, f32_from_bf16
    o = oracle
    lm = np.zeros((V, D), np.uint16)
    lm[np.arange(V), np.arange(V) % D] = 0x3F80
    w = weights(o, block(o, 41), final_gain=2.0, lm=np.ascontiguousarray(lm.reshape(-1)))
    h = o.normal_bf16(D, 42, 0, 1.0)
    got = o.logits(w, h)
    inverse = np.float32(o.lib().orc_rms_inverse(h, D, EPS))
    normalized = f32_from_bf16(bf16_from_f32((f32_from_bf16(h) * inverse).astype(np.float32)))
    want = bf16_from_f32((normalized * np.float32(2.0)).astype(np.float32))[np.arange(V) % D]
    assert np.array_equal(got, want)
    # Skipping the final norm returns the raw features.
    assert not np.array_equal(got, h[np.arange(V) % D])


def test_rows_at_once_equal_one_position_at_a_time(oracle):
    """A chunk of consecutive positions (the prompt-pass form used as the
    oracle for prefill) equals consuming them one position per call: causal
    masking and absolute positions inside a chunk."""
    o = oracle
    w = weights(o, block(o, 51))
    rows, first = 5, 3
    k1 = np.zeros(16 * KW, np.uint16)
    v1 = np.zeros(16 * KW, np.uint16)
    k1[: first * KW] = o.normal_bf16(first * KW, 52, 0, 1.0)
    v1[: first * KW] = o.normal_bf16(first * KW, 52, 1, 1.0)
    k2, v2 = k1.copy(), v1.copy()
    h = o.normal_bf16(rows * D, 53, 0, 1.0)
    chunk = run_block(o, w, h, first, k1, v1, rows=rows)
    step = np.concatenate([run_block(o, w, h[r * D:(r + 1) * D], first + r, k2, v2) for r in range(rows)])
    assert np.array_equal(chunk, step)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)

