"""The binding's destruction order (dolittle_amd._lib.Native): a native
handle is destroyed only after every handle created from it, in whatever
order Python finalizes the owners (the objects of one garbage cycle are
finalized in no particular order).  Pure host logic: the destroy calls are
recorded instead of made."""
import itertools

import pytest


@pytest.fixture
def recorder(monkeypatch):
    from dolittle_amd import _lib
    calls = []
    monkeypatch.setattr(_lib, "call", lambda name, handle: calls.append((name, handle)))
    return calls


def test_dependents_are_destroyed_first_in_every_release_order(recorder):
    from dolittle_amd._lib import Native
    names = ["device", "queue", "model", "plan", "buffer"]
    for order in itertools.permutations(names):
        recorder.clear()
        device = Native("dl_device_close", "device")
        queue = Native("dl_queue_destroy", "queue", device)
        model = Native("dl_qwen3_destroy", "model", device, queue)
        plan = Native("dl_plan_destroy", "plan", model)
        buffer = Native("dl_buffer_free", "buffer", device)
        records = {"device": device, "queue": queue, "model": model, "plan": plan, "buffer": buffer}
        for name in order:
            records[name].release()
        done = [h for _, h in recorder]
        assert sorted(done) == sorted(names), (order, done)
        pos = {h: i for i, h in enumerate(done)}
        assert pos["plan"] < pos["model"] < pos["queue"] < pos["device"], (order, done)
        assert pos["buffer"] < pos["device"], (order, done)


def test_release_is_idempotent_and_waits_for_dependents(recorder):
    from dolittle_amd._lib import Native
    device = Native("dl_device_close", "device")
    queue = Native("dl_queue_destroy", "queue", device)
    device.release()
    device.release()
    assert recorder == []
    queue.release()
    queue.release()
    assert recorder == [("dl_queue_destroy", "queue"), ("dl_device_close", "device")]
