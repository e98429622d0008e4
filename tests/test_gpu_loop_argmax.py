"""The token loop's own greedy selection (k_lm_head's per-block argmax keys
merged in k_step_end) at its edges, against the pinned greedy oracle.

The reference's loop selects greedily on the device with the law of
categorical.cpp:168-173 (maximum finite logit, lowest id on ties; NaN or
+inf anywhere is status 1, no finite logit status 2: sampling.cu:158,274).
To put chosen logits into the loop, a one-block model with an untied
embedding gets a crafted final norm and LM head: the final norm keeps one
feature k0 (gain 1, every other gain 0), so the normalized row is x at k0
and zero elsewhere, and LM-head row v holds c_v * sign(x) at k0 and zeros
elsewhere.  Logit v is then BF16(|x| c_v) with the sign of c_v: equal c_v
give bit-equal logits, c_v = -inf gives -inf, +inf gives +inf, NaN gives NaN,
and +-0 give +0.  Each case runs the loop for one selection and checks the
selected id, or the failure status, against orc_greedy_bf16 on the logits
the loop wrote, and against the case's construction.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V = 4096
SEED = 20261202
PROMPT = [3, 17]
NAN_BITS, NEG_ZERO = 0x7FC0, 0x8000


@pytest.fixture(scope="module")
def crafted(device, queue, oracle):
    from dolittle_amd.qwen3 import Plan, Qwen3Config, Qwen3Model
    cfg = Qwen3Config(layers=1, vocab=V, tied_embeddings=False)
    model = Qwen3Model(device, queue, cfg)
    model.fill_synthetic(SEED, 0.02)
    plan = Plan(model, batch=1, capacity=8)
    plan.generate(PROMPT, 1)
    plan.collect()
    h = oracle.f32_from_bf16(plan.hidden(0))
    k0 = int(np.argmax(np.abs(h)))
    assert h[k0] != 0
    gains = np.zeros(cfg.hidden, np.uint16)
    gains[k0] = 0x3F80
    model.write("final_norm", 0, gains)
    return model, k0, float(np.sign(h[k0]))


def run_case(model, k0, sign, oracle, column):
    """column: V multipliers (float, +-inf or nan; the string '-0' for a
    negative zero weight).  Returns (loop result, tokens, logits bits)."""
    from dolittle_amd.qwen3 import Plan
    col = np.empty(V, np.uint16)
    for i, c in enumerate(column):
        if isinstance(c, str):
            col[i] = NEG_ZERO
        elif np.isnan(c):
            col[i] = NAN_BITS
        else:
            col[i] = oracle.bf16_from_f32(np.array([c * sign], np.float32))[0]
    w = np.zeros((V, model.config.hidden), np.uint16)
    w[:, k0] = col
    model.write("lm_head", 0, w)
    plan = Plan(model, batch=1, capacity=8)
    plan.generate(PROMPT, 1)
    tokens, results = plan.collect()
    return results[0], tokens[0], plan.logits(0)


def check(oracle, result, tokens, logits, want):
    status, got = oracle.greedy(logits)
    if want[0] == 0:
        assert (status, got) == want, (status, got, want)
        assert result["status"] == 0 and result["generated"] == 1, result
        assert int(tokens[0]) == want[1], (tokens, want)
    else:
        assert status == want[0], (status, want)
        assert result["status"] == want[0] and result["reason"] == "failure", result
        assert result["generated"] == 0, result


def test_ties_select_the_lowest_id(crafted, oracle):
    model, k0, sign = crafted
    col = [-1.0] * V
    for i in (3000, 77, 1000):
        col[i] = 2.0
    res, tok, logits = run_case(model, k0, sign, oracle, col)
    assert logits[77] == logits[1000] == logits[3000] and logits[77] < 0x7F80
    check(oracle, res, tok, logits, (0, 77))
    col = [-1.0] * V
    col[0] = col[V - 1] = 3.0
    res, tok, logits = run_case(model, k0, sign, oracle, col)
    check(oracle, res, tok, logits, (0, 0))
    col = [-1.0] * V
    col[V - 1] = 0.5
    res, tok, logits = run_case(model, k0, sign, oracle, col)
    check(oracle, res, tok, logits, (0, V - 1))


def test_zero_logits_tie_across_signs(crafted, oracle):
    model, k0, sign = crafted
    col = [-1.0] * V
    col[9], col[5], col[3] = 0.0, 0.0, "-0"
    res, tok, logits = run_case(model, k0, sign, oracle, col)
    assert logits[3] & 0x7FFF == 0 and logits[5] & 0x7FFF == 0 and logits[9] & 0x7FFF == 0, logits[[3, 5, 9]]
    check(oracle, res, tok, logits, (0, 3))


def test_negative_infinity_is_skipped(crafted, oracle):
    model, k0, sign = crafted
    col = [-np.inf] * V
    col[2], col[4000] = -5.0, -3.0
    res, tok, logits = run_case(model, k0, sign, oracle, col)
    assert logits[0] == 0xFF80 and logits[1] == 0xFF80
    check(oracle, res, tok, logits, (0, 4000))


def test_all_negative_infinity_fails_with_no_candidate(crafted, oracle):
    model, k0, sign = crafted
    res, tok, logits = run_case(model, k0, sign, oracle, [-np.inf] * V)
    assert np.all(logits == 0xFF80)
    check(oracle, res, tok, logits, (2, None))


@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_nan_or_positive_infinity_fails(crafted, oracle, bad):
    model, k0, sign = crafted
    col = [-1.0] * V
    col[100] = 4.0
    col[2048] = bad
    res, tok, logits = run_case(model, k0, sign, oracle, col)
    assert (logits[2048] & 0x7FFF) >= 0x7F80
    check(oracle, res, tok, logits, (1, None))
