"""The plan's DeviceSequence event journal and stop semantics on the GPU.

Each case restates a scenario of the reference's device test
(tests/gpu/test_device.cpp:356-470, the autonomous sequence over
DeviceSequence of src/kernels/cuda/decode.cu) on the Qwen3 token loop, and
every journal is checked with the rules the reference's generate() applies
to the events it consumes (src/inference/generation.cpp:160-200): a
selected event's position is the number of tokens so far and its token is
in the vocabulary; a consumed event starts where the previous consumption
ended and covers tokens already known; the journal ends with one terminal
event.

- limit: prompt 3, 8 tokens; events consumed x3, then (selected,
  consumed) x8, terminal limit at position 11 with count 8; the selected
  tokens are the collected stream.
- cancel before start: nothing is consumed; terminal cancelled at 0.
- eos: the first token is a stop id; terminal eos at position 4, count 1.
- invalid injection (zero, NaN and FLT_MAX source rows): an injection event
  with a nonzero status, then terminal failure at 0 with count 0; a valid
  one (2.0) publishes status 0 and its norm, then the normal limit journal.
- cancel while decoding (ADVICE: a selection is still consumed): with a
  step window the host stops enqueuing, so the request lands mid-run; the
  terminal event is cancelled with position = prompt + generated.
- bounded window: an eos at token k of 100 leaves at most 2 windows of
  steps enqueued past the stop.
- idle steps past a capacity below the one-kernel attention limit replay
  the short-context graph and change nothing.
- batch 2 where one sequence stops early: per-sequence terminal events.
- a resumed prompt pass opens the journal with one consumed event
  covering the prefilled positions.
"""
import numpy as np
import pytest

from test_gpu_model import small_model  # noqa: F401  (module fixture)

pytestmark = pytest.mark.gpu

V = 151936


def check_journal(events, prompt_len, tokens=None):
    """generation.cpp's publication checks; returns (selected ids, terminal)."""
    assert events and events[-1]["kind"] == "terminal", events[-3:]
    assert all(e["kind"] != "terminal" for e in events[:-1])
    known, consumed, selected = prompt_len, 0, []
    for e in events[:-1]:
        if e["kind"] == "selected":
            assert e["position"] == known and e["token"] < V, e
            selected.append(e["token"])
            known += 1
        elif e["kind"] == "consumed":
            assert e["position"] == consumed and 0 < e["count"] <= known - consumed, (e, consumed, known)
            consumed += e["count"]
        else:
            assert e["kind"] == "injection", e
    term = events[-1]
    assert term["position"] == consumed and term["count"] == len(selected), (term, consumed, len(selected))
    if tokens is not None:
        assert selected == list(tokens[: len(selected)])
    return selected, term


REASONS = {0: "limit", 1: "eos", 2: "cancelled", 3: "failure"}


def test_limit_journal(small_model):
    from dolittle_amd.qwen3 import Plan
    p, new = [11, 22, 33], 8
    plan = Plan(small_model, batch=1, capacity=32)
    plan.generate(p, new)
    tokens, results = plan.collect()
    events = plan.events(0)
    selected, term = check_journal(events, len(p), tokens[0].tolist())
    assert len(selected) == new and REASONS[term["status"]] == "limit" and term["position"] == len(p) + new
    kinds = [e["kind"] for e in events]
    assert kinds == ["consumed"] * 3 + ["selected", "consumed"] * new + ["terminal"]
    assert [e["position"] for e in events if e["kind"] == "selected"] == list(range(3, 3 + new))
    assert results[0]["reason"] == "limit" and results[0]["position"] == len(p) + new


def test_cancel_before_start(small_model):
    from dolittle_amd.qwen3 import Plan
    p, new = [11, 22, 33], 8
    plan = Plan(small_model, batch=1, capacity=32)
    plan.prepare_generation(p, new)
    plan.request_stop()
    plan.decode_steps(len(p) + new)
    _, results = plan.collect()
    events = plan.events(0)
    assert [e["kind"] for e in events] == ["terminal"]
    assert REASONS[events[0]["status"]] == "cancelled" and events[0]["position"] == 0 and events[0]["count"] == 0
    assert results[0]["reason"] == "cancelled" and results[0]["generated"] == 0 and results[0]["position"] == 0


def test_eos_journal(small_model):
    from dolittle_amd.qwen3 import Plan
    p = [11, 22, 33]
    plan = Plan(small_model, batch=1, capacity=32)
    plan.generate(p, 8)
    first = int(plan.collect()[0][0][0])
    plan.generate(p, 8, stop_ids=[first])
    tokens, results = plan.collect()
    events = plan.events(0)
    selected, term = check_journal(events, len(p))
    assert selected == [first]
    assert REASONS[term["status"]] == "eos" and term["position"] == 4 and term["count"] == 1
    assert results[0]["reason"] == "eos" and results[0]["position"] == 4


@pytest.mark.parametrize("value", ["zero", "nan", "flt_max", "two"])
def test_injection_status_events(small_model, device, queue, oracle, value):
    from dolittle_amd.interventions import DeviceInjection, Region
    from dolittle_amd.qwen3 import Plan
    x = np.zeros(4096, np.float32)
    x[0] = {"zero": 0.0, "nan": np.nan, "flt_max": np.finfo(np.float32).max, "two": 2.0}[value]
    buf = device.upload_array(queue, x)
    inj = DeviceInjection(device, queue, Region(buf, 0, x.nbytes), "float32", "bfloat16", 4096, 150.0)
    inj.submit()
    status, norm, _ = oracle.inject(x, False, True, 150.0)
    p, new = [11, 22, 33], 4
    plan = Plan(small_model, batch=1, capacity=32)
    plan.set_injection(inj, 1)
    plan.generate(p, new)
    _, results = plan.collect()
    events = plan.events(0)
    assert events[0]["kind"] == "injection" and events[0]["status"] == status
    _, term = check_journal(events, len(p))
    if value == "two":
        assert status == 0 and events[0]["norm"] == np.float32(norm) == np.float32(2.0)
        assert REASONS[term["status"]] == "limit" and term["count"] == new
    else:
        assert status != 0
        assert [e["kind"] for e in events] == ["injection", "terminal"]
        assert REASONS[term["status"]] == "failure" and term["position"] == 0 and term["count"] == 0
        assert term["token"] & 8
        assert results[0]["reason"] == "failure" and results[0]["position"] == 0


def test_cancel_while_decoding_consumes_the_selection(small_model):
    """The host stops after the fifth selected event and requests a stop.
    With a two-step window at most four more steps are enqueued, so the
    device sees the request mid-run; the last selection is consumed:
    terminal cancelled with position = prompt + generated."""
    from dolittle_amd.qwen3 import Plan
    p, new = [5, 6, 7, 8], 200
    plan = Plan(small_model, batch=1, capacity=256)
    plan.set_step_window(2)
    plan.generate(p, new)
    events, selected = [], 0
    while selected < 5:
        e = plan.collect_event(0, len(events))
        events.append(e)
        selected += e["kind"] == "selected"
    plan.request_stop()
    while events[-1]["kind"] != "terminal":
        events.append(plan.collect_event(0, len(events)))
    tokens, results = plan.collect()
    chosen, term = check_journal(events, len(p), tokens[0].tolist())
    assert REASONS[term["status"]] == "cancelled", term
    assert 5 <= term["count"] < new and term["position"] == len(p) + term["count"]
    assert events[-2]["kind"] == "consumed" and events[-2]["position"] == term["position"] - 1
    assert results[0]["reason"] == "cancelled" and results[0]["position"] == len(p) + results[0]["generated"]
    assert plan.steps_enqueued() <= len(p) + term["count"] + 2 * 2


def test_window_bounds_the_steps_after_a_stop(small_model):
    from dolittle_amd.qwen3 import Plan
    p, new, window = [9, 8, 7], 100, 4
    plan = Plan(small_model, batch=1, capacity=128)
    plan.generate(p, 12)
    stream = plan.collect()[0][0].tolist()
    k = next(i for i in range(2, 12) if stream[i] not in stream[:i])
    plan.set_step_window(window)
    plan.generate(p, new, stop_ids=[stream[k]])
    tokens, results = plan.collect()
    assert results[0]["reason"] == "eos" and results[0]["generated"] == k + 1
    assert tokens[0][: k + 1].tolist() == stream[: k + 1]
    consumed = len(p) + k + 1
    assert plan.steps_enqueued() <= consumed + 2 * window, (plan.steps_enqueued(), consumed)
    _, term = check_journal(plan.events(0), len(p), stream)
    assert term["position"] == consumed
    # Without a window every step of the budget is enqueued.
    plan.set_step_window(0)
    plan.generate(p, new, stop_ids=[stream[k]])
    plan.collect()
    assert plan.steps_enqueued() == len(p) + new


def test_idle_steps_past_a_short_capacity(small_model):
    """A plan whose cache ends below the one-kernel attention limit has
    only the short-context step graph; replaying steps past its capacity
    (beyond that limit) finds the loop stopped and changes nothing."""
    from dolittle_amd.qwen3 import Plan
    p = [9, 8, 7]
    plan = Plan(small_model, batch=1, capacity=64)
    plan.generate(p, 8)
    tokens, results = plan.collect()
    plan.decode_steps(1600)
    again, results_again = plan.collect()
    assert again.tolist() == tokens.tolist() and results_again == results


def test_batch_two_sequence_stops_early(small_model):
    """Sequence 1 is steered so the two streams differ; a stop id from
    sequence 0's stream that sequence 1 never produces ends sequence 0
    early: its terminal event is eos at its own position while sequence 1
    runs to the limit."""
    from dolittle_amd.qwen3 import Plan
    p, new = [21, 22, 23, 24], 10
    v = np.random.default_rng(5).standard_normal(4096).astype(np.float32) * np.float32(4.0)
    plan = Plan(small_model, batch=2, capacity=32)
    plan.set_steering(1, 1, v)
    plan.generate(p, new)
    streams, _ = plan.collect()
    s0, s1 = streams[0].tolist(), streams[1].tolist()
    k = next((i for i in range(1, new - 1) if s0[i] not in s1 and s0[i] not in s0[:i]), None)
    if k is None:
        pytest.skip("the streams share every candidate stop id")
    plan.generate(p, new, stop_ids=[s0[k]])
    tokens, results = plan.collect()
    e0, e1 = plan.events(0), plan.events(1)
    sel0, t0 = check_journal(e0, len(p), s0)
    sel1, t1 = check_journal(e1, len(p), s1)
    assert REASONS[t0["status"]] == "eos" and t0["count"] == k + 1 and t0["position"] == len(p) + k + 1
    assert REASONS[t1["status"]] == "limit" and t1["count"] == new and t1["position"] == len(p) + new
    assert results[0]["reason"] == "eos" and results[1]["reason"] == "limit"


def test_prefilled_positions_open_the_journal(small_model):
    from dolittle_amd.qwen3 import Plan
    p, new = [int(t) for t in np.random.default_rng(3).integers(0, V, 12)], 3
    plan = Plan(small_model, batch=1, capacity=32)
    plan.prefill(p)
    plan.generate(p, new)
    tokens, _ = plan.collect()
    events = plan.events(0)
    assert events[0] == {"kind": "consumed", "status": 0, "position": 0, "count": len(p) - 1, "token": 0,
                         "norm": 0.0}
    _, term = check_journal(events, len(p), tokens[0].tolist())
    assert REASONS[term["status"]] == "limit" and term["position"] == len(p) + new


def test_an_index_past_the_terminal_event_fails_instead_of_waiting(small_model):
    """decode.cu:579-600: a sequence that ended without the asked event is an
    error, for the non-blocking read as for the blocking one."""
    from dolittle_amd import DeviceError
    from dolittle_amd.qwen3 import Plan
    plan = Plan(small_model, batch=1, capacity=32)
    plan.generate([1, 2, 3], 4)
    plan.collect()
    events = plan.events(0)
    assert events[-1]["kind"] == "terminal"
    for wait in (False, True):
        with pytest.raises(DeviceError, match="ended without event"):
            plan.collect_event(0, len(events), wait=wait)


def test_window_change_is_rejected_while_a_windowed_generation_is_live(small_model):
    """Switching the window to 0 mid-run would leave the remaining steps
    unenqueued: the plan refuses it until the generation has ended."""
    from dolittle_amd import InvalidArgument
    from dolittle_amd.qwen3 import Plan
    plan = Plan(small_model, batch=1, capacity=256)
    plan.set_step_window(2)
    plan.generate([1, 2, 3], 200)
    with pytest.raises(InvalidArgument):
        plan.set_step_window(0)
    tokens, results = plan.collect()
    assert results[0]["generated"] == 200 and results[0]["reason"] == "limit"
    plan.set_step_window(0)  # the generation has ended
