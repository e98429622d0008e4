"""GPU checks of the MFMA prefill path (BASELINE config 3's prompt pass).

MFMA units accumulate in their own order, so this path is compared with
tolerances rather than bit for bit:
- the MFMA projection against an FP64 product of the same BF16 operands
  (at most one BF16 ulp after rounding) at the Qwen3-8B projection shapes;
- a multi-block model: KV rows written by the prefill against the CPU
  contract restatement, and the first decoded logits against the oracle's
  exact logits within 2e-2 absolute / 1e-2 relative (the north-star logits
  tolerance), at a prompt length that is not a multiple of the 128-row tile.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 7701


def bf16_ulp(x):
    """Spacing of BF16 numbers at |x| (2^(e-7))."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


# (4096, 4096, 4096) has 256 output tiles of 256 x 256: the 256 x 256 tile
# GEMM; the smaller shapes run the 128 x 256 and 128 x 128 tile GEMMs.
@pytest.mark.parametrize("rows,in_w,out_w", [(256, 4096, 4096), (128, 4096, 1024), (128, 12288, 4096),
                                             (384, 4096, 6144), (512, 12288, 4096), (512, 4096, 6144),
                                             (4096, 4096, 4096)])
def test_prefill_projection_within_one_ulp(device, queue, oracle, rows, in_w, out_w):
    from dolittle_amd import _lib
    x = oracle.normal_bf16(rows * in_w, SEED, 1, 1.0)
    w = oracle.normal_bf16(out_w * in_w, SEED, 2, 0.02)
    bx, bw = device.upload_array(queue, x), device.upload_array(queue, w)
    nbytes = C.c_uint64()
    _lib.call("dl_projection_packed_bytes", out_w, in_w, C.byref(nbytes))
    packed = device.allocate(nbytes.value)
    by, work = device.allocate(rows * out_w * 2), device.allocate(rows * in_w * 2)
    _lib.call("dl_projection_pack", queue.handle, bw.ptr(), packed.ptr(), out_w, in_w)
    _lib.call("dl_prefill_projection", queue.handle, bx.ptr(), packed.ptr(), by.ptr(), work.ptr(), rows, in_w, out_w)
    queue.drain()
    got = oracle.f32_from_bf16(queue.read(by, np.uint16, rows * out_w)).reshape(rows, out_w).astype(np.float64)
    xf = oracle.f32_from_bf16(x).reshape(rows, in_w).astype(np.float64)
    wf = oracle.f32_from_bf16(w).reshape(out_w, in_w).astype(np.float64)
    exact = xf @ wf.T
    # One BF16 ulp of rounding plus the FP32 accumulation error of K / 16
    # sequential MFMA steps (random-walk bound on the absolute-value sum),
    # which dominates only for outputs near zero.
    scale = np.abs(xf) @ np.abs(wf).T
    bound = bf16_ulp(exact) + 4.0 * np.sqrt(in_w / 16) * 2.0 ** -24 * scale + 1e-6
    err = np.abs(got - exact)
    assert np.all(err <= bound), float((err / bound).max())
    # A misplaced operand piece would show as errors of many ulps at
    # ordinary magnitudes; the bulk stays within one ulp.
    assert np.mean(err <= bf16_ulp(exact)) > 0.9999


def permuted_np(k, P):
    """Position of input k in the P-permuted order (prefill.h `permuted`)."""
    block = 8 * P
    return (k // block) * block + (k % P) * 8 + (k % block) // P


def test_prefill_gate_up_silu_of_every_bf16_gate(device, queue, oracle):
    """The gate/up GEMM's SiLU * up against the oracle's SiluMultiply for
    every BF16 gate value that is +0 or finite and normal (65,025 bit
    patterns).  Rows of x carry the patterns in inputs 0-127 and 1.0 in input
    128; gate row f selects input f % 128 and up row f input 128, each with
    weight 1.0, so every MFMA sum is exact and act[m][f] = SiLU(x[m][f % 128])
    rounded as the contract rounds it.  512 rows x 65,536 gate/up columns is
    512 tiles of 256 x 256: the 256 x 256 tile kernel, whose SiLU comes from
    the table built per device, and its P32-permuted activation order."""
    from dolittle_amd import _lib
    K, F, rows = 256, 32768, 512
    patterns = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exponent = (patterns >> 7) & 0xFF
    # -0 is left out: a dot product adds +0 terms to it, so its gate is +0.
    usable = ((exponent != 0) | ((patterns & 0x7F) == 0)) & (exponent != 0xFF) & (patterns != 0x8000)
    x = np.zeros((rows, K), np.uint16)
    x[:, :128] = np.where(usable, patterns, 0).reshape(rows, 128)
    x[:, 128] = 0x3F80
    f = np.arange(F)
    w = np.zeros((2 * F, K), np.uint16)
    w[4 * (f // 2) + f % 2, f % 128] = 0x3F80       # gate rows: g 2j, g 2j+1
    w[4 * (f // 2) + 2 + f % 2, 128] = 0x3F80       # up rows: u 2j, u 2j+1
    bx, bw = device.upload_array(queue, x.reshape(-1)), device.upload_array(queue, w.reshape(-1))
    nbytes = C.c_uint64()
    _lib.call("dl_projection_packed_bytes", 2 * F, K, C.byref(nbytes))
    packed = device.allocate(nbytes.value)
    _lib.call("dl_projection_pack", queue.handle, bw.ptr(), packed.ptr(), 2 * F, K)
    out, work = device.allocate(rows * F * 2), device.allocate(rows * K * 2)
    _lib.call("dl_prefill_gate_up", queue.handle, bx.ptr(), packed.ptr(), out.ptr(), work.ptr(), rows, K, F)
    queue.drain()
    act = queue.read(out, np.uint16, rows * F).reshape(rows, F)[:, permuted_np(f, 32)]
    gate = x[:, f % 128]
    want = oracle.silu_multiply(gate.reshape(-1), np.full(gate.size, 0x3F80, np.uint16)).reshape(rows, F)
    check = usable.reshape(rows, 128)[:, f % 128]
    assert int(usable.sum()) == 65536 - 256 - 254 - 1 and int(check.sum()) == int(usable.sum()) * (F // 128)
    assert np.array_equal(act[check], want[check])


def test_prefill_projection_rejects_ragged_shapes(device, queue):
    from dolittle_amd import InvalidArgument, _lib
    buf = device.allocate(1 << 20)
    with pytest.raises(InvalidArgument):
        _lib.call("dl_prefill_projection", queue.handle, buf.ptr(), buf.ptr(), buf.ptr(), buf.ptr(), 100, 4096, 4096)
    with pytest.raises(InvalidArgument):
        _lib.call("dl_prefill_projection", queue.handle, buf.ptr(), buf.ptr(), buf.ptr(), buf.ptr(), 128, 4096, 100)


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
    return o.Qwen3Weights(dims, blocks, np.ascontiguousarray(model.read("final_norm")), lm, lm)


@pytest.fixture(scope="module")
def prefill_model(device, queue):
    from dolittle_amd.qwen3 import Qwen3Config, Qwen3Model
    model = Qwen3Model(device, queue, Qwen3Config(layers=2))
    model.fill_synthetic(SEED, 0.02)
    return model


@pytest.mark.parametrize("n", [300, 500])
def test_prefill_cache_and_first_logits_within_tolerance(prefill_model, oracle, n):
    """The first block's prefilled K/V rows equal the oracle's except for
    rare flips (MFMA accumulation order), and the first logits after a
    two-block prefill stay within 0.06 of the exact ones (98% of them within
    2e-2 absolute + 1e-2 relative).
    Deeper models drift further (every order-dependent rounding flip
    propagates through the following blocks); the exact path remains the
    parity path.  Prompts of 300 and 500 ids (384 and 512 GEMM rows)."""
    from dolittle_amd.qwen3 import Plan
    cfg = prefill_model.config
    w = oracle_weights(oracle, prefill_model)
    cap = n + 20
    prompt = [int(t) for t in np.random.default_rng(31).integers(0, cfg.vocab, n)]
    plan = Plan(prefill_model, batch=1, capacity=cap)
    plan.prefill(prompt, mfma=True)
    plan.generate(prompt, 1)
    tokens, results = plan.collect()
    assert results[0]["generated"] == 1 and results[0]["position"] == n + 1

    kw = cfg.kv_heads * cfg.head_dim
    k = [np.zeros(cap * kw, np.uint16) for _ in range(cfg.layers)]
    v = [np.zeros(cap * kw, np.uint16) for _ in range(cfg.layers)]
    emb = w.embedding.reshape(cfg.vocab, cfg.hidden)
    h = np.ascontiguousarray(emb[prompt].reshape(-1))
    for layer in range(cfg.layers):
        oracle.block_forward(w, layer, h, n, 0, k[layer], v[layer])
    kg, vg = plan.read_cache(0, 0, n - 1)
    for got, ref in ((kg, k[0][: (n - 1) * kw]), (vg, v[0][: (n - 1) * kw])):
        g = oracle.f32_from_bf16(got).astype(np.float64)
        r = oracle.f32_from_bf16(ref).astype(np.float64)
        assert np.mean(g == r) > 0.999
        # A flipped projection output moves its whole head through the QK
        # norm: a couple of ulps at most (values are O(1) after the norm).
        assert np.all(np.abs(g - r) <= 2 * bf16_ulp(r) + 2.0 ** -9)
    logits_ref = oracle.f32_from_bf16(oracle.logits(w, h.reshape(n, cfg.hidden)[-1].copy())).astype(np.float64)
    logits = oracle.f32_from_bf16(plan.logits(0)).astype(np.float64)
    diff = np.abs(logits - logits_ref)
    # The perturbation reaches the logits as absolute noise of a few
    # hundredths (two blocks), independent of the logit's magnitude.
    assert diff.max() <= 0.06, float(diff.max())
    assert np.mean(diff <= 2e-2 + 1e-2 * np.abs(logits_ref)) > 0.98
    # The first token is the exact greedy selection over the device logits.
    assert oracle.greedy(plan.logits(0)) == (0, int(tokens[0][0]))


def test_prefill_attention_matches_contract(device, queue, oracle):
    """Causal MFMA attention (FP32 softmax, probabilities split exactly into
    three BF16 parts) against the exact attention contract; flips only where
    the output is a cancelling sum."""
    from dolittle_amd import _lib
    rows, cap, H, G = 200, 256, 32, 8
    qr = oracle.normal_bf16(rows * H * 128, 5, 1, 1.0)
    k_ref = oracle.normal_bf16(cap * G * 128, 5, 2, 1.0)
    v_ref = oracle.normal_bf16(cap * G * 128, 5, 3, 1.0)
    k_plan = np.ascontiguousarray(k_ref.reshape(cap, G, 128).transpose(1, 0, 2))
    v_plan = np.ascontiguousarray(v_ref.reshape(cap, G * 128).T)
    bq, bk, bv = device.upload_array(queue, qr), device.upload_array(queue, k_plan), device.upload_array(queue, v_plan)
    bo = device.allocate(rows * H * 128 * 2)
    _lib.call("dl_prefill_attention", queue.handle, bq.ptr(), bk.ptr(), bv.ptr(), bo.ptr(), rows, H, G, cap, 0)
    queue.drain()
    out = queue.read(bo, np.uint16, rows * H * 128).reshape(rows, H * 128)
    k = np.arange(H * 128)
    nat = out[:, (k // 128) * 128 + (k % 16) * 8 + (k % 128) // 16]
    ref = oracle.attention(qr, k_ref, v_ref, rows, H, G, 128, 0).reshape(rows, H * 128)
    g = oracle.f32_from_bf16(nat).astype(np.float64)
    r = oracle.f32_from_bf16(ref).astype(np.float64)
    assert np.mean(g == r) > 0.999
    assert np.all(np.abs(g - r) <= 2 * bf16_ulp(r) + 1e-4)


def test_prefill_then_decode_continues(prefill_model):
    """A different prompt after a prefill runs the exact path from 0; the
    same prompt resumes after the prefilled positions."""
    from dolittle_amd.qwen3 import Plan
    prompt = list(range(1000, 1000 + 130))
    plan = Plan(prefill_model, batch=2, capacity=160)
    plan.prefill(prompt, mfma=True)
    plan.generate(prompt, 6)
    t1, res = plan.collect()
    assert all(r["generated"] == 6 and r["position"] == 136 for r in res)
    assert t1[0].tolist() == t1[1].tolist()
    other = list(range(2000, 2000 + 20))
    plan.generate(other, 3)
    _, res2 = plan.collect()
    assert res2[0]["position"] == 23
