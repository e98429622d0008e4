"""The reference-side adapter (integration/hip_backend.cpp) executed on the
GPU through the reference's own interfaces, every result checked against the
CPU oracle by tests/adapter_driver.cpp:

- Queue upload / copy / download, and DeviceCategorical's borrowed result
  and current-token regions downloaded after submit_next (the reference's
  own use, executor.cpp:1021);
- kernels::prepare / PreparedOperation for all eight operations: Projection,
  RmsNorm, Rotary, CausalAttention (full forward, and the incremental form
  over a ContiguousLayerView with dynamic rows), Embedding, Add,
  SiluMultiply, GatherRows (fixed rows and the last-active-row policy),
  bit-exact against the contract mirror;
- DeviceSequence recorded stage by stage as the executor records it
  (executor.cpp:1595-1657), over a toy recipe (Embedding with captures, then
  the last row's logits projection and the device sampler): the journal's
  events, the greedy tokens and the captured rows against the oracle's
  Markov chain, for a limit run (two chunks and a remainder), an eos run,
  a run cancelled before start and a prompt of whole chunks;
- DeviceInjection, DeviceDirection and DeviceIntervention against the NLA
  oracle.

The driver is built here, where the reference headers are, by
integration/Makefile (build() runs it); the GPU box runs the built binary."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "integration", "_build", "adapter_driver")

CHECKS = {
    "transfers": ["queue upload, copy and download", "DeviceCategorical::submit_next result region downloaded",
                  "DeviceCategorical::current_token region downloaded"],
    "operations": ["prepared Projection", "prepared RmsNorm", "prepared Rotary",
                   "prepared CausalAttention (full forward)",
                   "prepared CausalAttention (cache view, dynamic rows)", "prepared Embedding", "prepared Add",
                   "prepared SiluMultiply", "prepared GatherRows", "prepared GatherRows (last active row)"],
    "sequence": ["DeviceSequence limit: events, tokens and captures against the oracle",
                 "DeviceSequence eos: the stop token is selected and consumed",
                 "DeviceSequence cancelled before start", "DeviceSequence prompt of whole chunks"],
    "nla": ["DeviceInjection output, status and norm", "DeviceDirection", "DeviceIntervention row and state"],
}


@pytest.mark.skipif(not os.path.exists(DRIVER), reason="adapter driver not built (needs the reference headers)")
@pytest.mark.parametrize("part", list(CHECKS))
def test_adapter_on_the_gpu(part):
    print(f"adapter driver: {part}", flush=True)
    r = subprocess.run([DRIVER, part], capture_output=True, text=True, timeout=120)
    print(r.stdout[-4000:], r.stderr[-2000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    lines = r.stdout.splitlines()
    assert lines[-1] == "done"
    for check in CHECKS[part]:
        assert f"ok {check}" in lines, check
