"""Reference acceptance fixtures run against this backend.

The reference's validation bundles (scripts/validation/forward_reference.py,
fixture.json schema_version 1; bounds in scripts/validation/README.md:128-142)
hold a checkpoint, its declared artifacts and reference outputs of an
independent FP32-accumulation forward: per case, logits rows at
`logit_positions` and block-input / block-output rows of a few blocks at
`positions`, each output with its own tolerance; and a generation case whose
four greedy IDs follow the prompt, with every row of the full trace.

`run_bundle` opens the bundle through the verified archive path
(dl_safetensors_open with SHA-256), uploads the checkpoint, replays every
case through the exact token loop and compares each output as the reference
does (forward_reference.py:212-220): both the maximum absolute error and the
relative L2 error must be within that output's bounds, and the generated IDs
must equal the reference's.

    python -m dolittle_amd.fixtures <bundle directory>
"""
from __future__ import annotations

import json
import math
import os
import sys
from typing import Optional

import numpy as np


def error(reference, actual) -> dict:
    """forward_reference.py error(): max |a - b| and sqrt(sum (a-b)^2 / sum a^2)."""
    ref = np.asarray(reference, np.float64)
    act = np.asarray(actual, np.float64)
    if ref.shape != act.shape:
        raise ValueError("output shape mismatch")
    diff = ref - act
    squared_reference = math.fsum((ref * ref).tolist())
    return {"max_absolute_error": float(np.max(np.abs(diff))) if diff.size else 0.0,
            "relative_l2": math.sqrt(math.fsum((diff * diff).tolist()) / squared_reference)
            if squared_reference else None}


def within(errors: dict, tolerance: dict) -> bool:
    """Both bounds must hold (README.md:128-142); an all-zero reference has
    no relative error."""
    if not errors["max_absolute_error"] <= tolerance["max_absolute_error"]:
        return False
    return errors["relative_l2"] is None or errors["relative_l2"] <= tolerance["max_relative_l2"]


def f32_from_bf16(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


class Trace:
    """Logits and block outputs of one token sequence through the exact loop
    (one position per step, so every row is the token loop's own row)."""

    def __init__(self, model, tokens, blocks, logit_positions):
        from .qwen3 import Plan
        self.tokens = list(tokens)
        n = len(self.tokens)
        self.logits, self.outputs = {}, {}
        plan = Plan(model, batch=1, capacity=n + 1)
        layers = sorted(set(blocks)) or [-1]
        for i, layer in enumerate(layers):
            plan.reset()
            plan.set_capture(layer)
            for p, token in enumerate(self.tokens):
                plan.forward([token])
                if i == 0 and p in logit_positions:
                    self.logits[p] = f32_from_bf16(plan.logits(0))
            if layer >= 0:
                self.outputs[layer] = f32_from_bf16(plan.read_capture(0, 0, n))
        plan.set_capture(-1)


def _rows(matrix_rows, positions):
    return np.concatenate([matrix_rows[p] for p in positions]) if positions else np.zeros(0, np.float32)


def run_case(model, case: dict, embedding: np.ndarray) -> dict:
    """Replays one fixture case; returns {output name: {errors, tolerance, passed}}."""
    tokens = case["token_ids"]
    captures = case["captures"]
    needed = set()
    for c in captures:
        needed.add(c["block"] if c["boundary"] == "block_output" else c["block"] - 1)
    logit_positions = set(case["logits"]["positions"])
    trace = Trace(model, tokens, [b for b in needed if b >= 0], logit_positions)
    report = {}
    got = _rows(trace.logits, case["logits"]["positions"])
    e = error(case["logits"]["values"], got)
    report["logits"] = {"errors": e, "tolerance": case["logits"]["tolerance"],
                        "passed": within(e, case["logits"]["tolerance"])}
    for c in captures:
        block = c["block"] if c["boundary"] == "block_output" else c["block"] - 1
        if block >= 0:
            rows = trace.outputs[block]
        else:  # the input of block 0 is the embedding row
            rows = f32_from_bf16(embedding[np.asarray(tokens)])
        got = np.concatenate([rows[p] for p in c["positions"]])
        e = error(c["values"], got)
        report[f'block_{c["block"]}_{c["boundary"]}'] = {"errors": e, "tolerance": c["tolerance"],
                                                          "passed": within(e, c["tolerance"])}
    return report


def run_generation(model, generation: dict, embedding: np.ndarray) -> dict:
    """The generation case: the engine's greedy IDs after the prompt must
    equal the reference's, and every row of the full trace must pass."""
    from .qwen3 import Plan
    reference = generation["reference"]
    tokens = reference["token_ids"]
    prompt_length, new = generation["prompt_tokens"], generation["max_new_tokens"]
    plan = Plan(model, batch=1, capacity=len(tokens) + 1)
    plan.generate(tokens[:prompt_length], new)
    ids, results = plan.collect()
    report = run_case(model, reference, embedding)
    report["generated_ids"] = {"reference": tokens[prompt_length:], "engine": ids[0].tolist()[:results[0]["generated"]],
                               "passed": ids[0].tolist()[:results[0]["generated"]] == tokens[prompt_length:]}
    return report


def run_bundle(device, queue, root: str, fixture: Optional[dict] = None) -> dict:
    """Opens the bundle at `root` (fixture.json plus the declared artifacts)
    and returns the full report with an overall `passed`."""
    from . import checkpoint as ck
    if fixture is None:
        with open(os.path.join(root, "fixture.json")) as f:
            fixture = json.load(f)
    if fixture.get("schema_version") != 1:
        raise ValueError("unsupported fixture schema")
    artifacts = [ck.ArtifactSpec(a["relative_path"], a["byte_size"], a["sha256"]) for a in fixture["artifacts"]]
    archive = ck.open_archive(root, fixture["repository"], fixture["revision"], artifacts, fixture["shards"],
                              fixture.get("index"))
    model = ck.load_qwen3(device, queue, archive, fixture.get("config_artifact", "config.json"))
    embedding = model.read("embedding").reshape(model.config.vocab, model.config.hidden)
    report = {"cases": {}, "identity": archive.identity()}
    for case in fixture["cases"]:
        report["cases"][case["name"]] = run_case(model, case, embedding)
    if fixture.get("generation"):
        report["generation"] = run_generation(model, fixture["generation"], embedding)
    outputs = [o for c in report["cases"].values() for o in c.values()]
    outputs += list(report.get("generation", {}).values())
    report["passed"] = all(o["passed"] for o in outputs)
    return report


def main(argv=None) -> int:
    from .runtime import Device
    args = argv if argv is not None else sys.argv[1:]
    if len(args) != 1:
        print("usage: python -m dolittle_amd.fixtures <bundle directory>", file=sys.stderr)
        return 2
    device = Device(0)
    queue = device.create_queue()
    report = run_bundle(device, queue, args[0])
    print(json.dumps(report, indent=1, default=str))
    return 0 if report["passed"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
