#!/usr/bin/env python3
"""Qwen3-8B batch-1 decode tokens/s on one MI355X.

Workload: the full Qwen3-8B architecture (36 blocks, tied 151,936-row LM
head) with seeded random BF16 weights ~N(0, 0.02) generated on the device,
a prompt of 128 seeded uniform-random token ids, fresh KV cache, greedy
decoding of 256 tokens through the device-owned token loop.  One "step" is
one decode token (one full forward of the last token + LM head + greedy
selection).  The first token comes from the prompt pass; `--warmup` more
steps run untimed; exactly `--steps` steps are timed with HIP events on the
plan's stream.  Inputs are resident in HBM for the whole timed region.

Also reported: prefill tokens/s of the 128-token prompt (the exact chunked
prompt pass), the whole-step HBM
roofline fraction, a live HIP-event roofline of the dominant kernel (the
fused RMSNorm + gate/up GEMV + SiLU), and the CPU baseline: the CPU contract
restatement (oracle/) timed on this host's cores on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense BF16 MFMA, MI355X
METRIC = "Qwen3-8B batch-1 decode tokens/s on 1 MI355X; % HBM roofline; prefill tok/s"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_bytes(cfg, which):
    """Algorithmic bytes of one launch of a decode-step kernel at batch 1."""
    D, QW, KW, F, V = cfg.hidden, cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim, cfg.ffn, cfg.vocab
    return {
        0: (QW + 2 * KW) * D * 2 + 2 * D * 2 + QW * 2 + KW * 2 + KW * 2,  # weights, norm+h, q/k out, v append
        4: D * QW * 2 + QW * 2 + 2 * D * 2,                                 # weights, att in, h in/out
        5: 2 * F * D * 2 + 2 * D * 2 + F * 2,                               # weights, norm+h, act out
        6: D * F * 2 + F * 2 + 2 * D * 2,                                   # weights, act in, h in/out
        7: V * D * 2 + 2 * D * 2 + V * 2,                                   # weights, norm+h, logits out
    }[which]


def step_bytes(cfg, context, batch=1):
    """Algorithmic bytes of one decode step of `batch` sequences with
    `context` visible keys each: projection weights incl. LM head and norm
    gains (read once per step), and per sequence the embedding row, KV read
    and append, and the BF16 logits row."""
    weights = cfg.projection_bytes_per_token() + (cfg.layers * (2 * cfg.hidden + 2 * cfg.head_dim) + cfg.hidden) * 2
    per_seq = cfg.hidden * 2 + cfg.layers * 2 * cfg.kv_heads * cfg.head_dim * 2 * (context + 1) + cfg.vocab * 2
    return weights + batch * per_seq


def bf16_bits(x):
    """Round-to-nearest-even BF16 bits of float32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def timed_loop(device, queue, plan, prompt, max_new, consume_steps, sampling=None, seeds=None):
    """Runs one device-owned generation: `consume_steps` steps take the
    prompt (and select token 1), then tokens 2..max_new are timed with HIP
    events on the plan's stream; returns (ms per step, tokens, results)."""
    from dolittle_amd import Event
    plan.prepare_generation(prompt, max_new, sampling, seeds)
    plan.decode_steps(consume_steps)
    queue.drain()
    ea, eb = Event(device), Event(device)
    ea.record(queue)
    plan.decode_steps(max_new - 1)
    eb.record(queue)
    queue.drain()
    plan.decode_steps(1)
    tokens, results = plan.collect()
    assert all(r["generated"] == max_new for r in results), results
    return ea.elapsed_ms(eb) / (max_new - 1), tokens, results


def other_configs(device, queue, model, cfg, seed, pplan, long_prompt):
    """Decode-side measurements of BASELINE configs 3, 4 and 5 (the token
    loop as the bench's main line runs it, at their batch and context)."""
    from dolittle_amd import Event
    from dolittle_amd.qwen3 import Plan, SamplingSettings
    out = {}
    if pplan is not None:
        # Config 3: greedy decode of 512 tokens after the exact prompt pass
        # of a 4096-id prompt; visible keys grow from 4097 to 4607.
        n, max_new = len(long_prompt), 512
        pplan.prefill(long_prompt)  # warm: allocates the exact pass's chunk buffers
        ea, eb = Event(device), Event(device)
        queue.drain()
        ea.record(queue)
        pplan.prefill(long_prompt)
        eb.record(queue)
        queue.drain()
        exact_ms = ea.elapsed_ms(eb)
        out["config3_exact_prefill"] = {"positions": n - 1, "ms": round(exact_ms, 2),
                                        "tokens_per_s": round((n - 1) / (exact_ms * 1e-3), 1)}
        log(f"config 3: exact prefill of {n - 1} positions in {exact_ms:.1f} ms = "
            f"{(n - 1) / (exact_ms * 1e-3):.0f} tok/s")
        ms, _, _ = timed_loop(device, queue, pplan, long_prompt, max_new, 1)
        mean_ctx = n + 1 + (max_new - 2) / 2.0
        gbs = step_bytes(cfg, mean_ctx) / (ms * 1e-3) / 1e9
        out["config3_decode"] = {"prompt": n, "new_tokens": max_new, "timed_positions": [n + 1, n + max_new - 1],
                                 "ms_per_step": round(ms, 4), "tokens_per_s": round(1000.0 / ms, 2),
                                 "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"config 3: decode at {n + 1}..{n + max_new - 1} keys {ms * 1e3:.1f} us/token = {1000.0 / ms:.1f} tok/s "
            f"({gbs / HBM_PEAK_GBS:.1%} of HBM peak)")
        # The long-context attention kernels, live, at the last decode
        # position (4608 visible keys), cycling layers.
        from dolittle_amd import _lib
        _lib.call("dl_plan_bench_prepare", pplan.handle)
        keys = n + max_new
        kv = keys * 2 * cfg.kv_heads * cfg.head_dim * 2
        attn, total = {}, 0.0
        for which, name in ((1, "k_attn_qk"), (2, "k_attn_softmax"), (3, "k_attn_pv")):
            _lib.call("dl_plan_launch_kernel", pplan.handle, which, 0, 2)
            ea, eb = Event(device), Event(device)
            queue.drain()
            ea.record(queue)
            _lib.call("dl_plan_launch_kernel", pplan.handle, which, 0, 72)
            eb.record(queue)
            us = ea.elapsed_ms(eb) * 1e3 / 72
            alg = attention_bytes(cfg, which, keys)
            gbs = alg / (us * 1e-6) / 1e9
            attn[name] = {"us": round(us, 2), "algorithmic_bytes": alg, "GB/s": round(gbs, 1),
                          "frac": round(gbs / HBM_PEAK_GBS, 4)}
            if keys == TRAFFIC_KEYS["long"]:
                attn[name]["traffic"] = load_traffic(name)[0]
            total += us
        attn.update({"keys": keys, "kv_bytes": kv, "total_us": round(total, 2),
                     "hbm_frac": round(kv / (total * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        out["config3_attention"] = attn
        log(f"config 3: attention at {keys} keys: {attn}")

    # The north star's 1K-context point: batch-1 greedy decode of 64 tokens
    # after the exact prompt pass of a 1024-id prompt (visible keys 1025 to
    # 1087 in the timed steps).
    prompt1k = np.random.default_rng(seed + 10).integers(0, cfg.vocab, 1024).astype(np.uint32)
    plan1k = Plan(model, batch=1, capacity=1024 + 64 + 2)
    plan1k.prefill(prompt1k)
    ms1k, _, _ = timed_loop(device, queue, plan1k, prompt1k, 64, 1)
    del plan1k
    ctx1k = 1024 + 1 + 62 / 2.0
    out["decode_1k_context"] = {
        "prompt": 1024, "new_tokens": 64, "timed_positions": [1024, 1086], "ms_per_step": round(ms1k, 4),
        "tokens_per_s": round(1000.0 / ms1k, 2),
        "hbm_frac": round(step_bytes(cfg, ctx1k) / (ms1k * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "north_star_tokens_per_s": 330}
    log(f"1K context: decode at 1025..1087 keys {ms1k * 1e3:.1f} us/token = {1000.0 / ms1k:.1f} tok/s "
        f"({out['decode_1k_context']['hbm_frac']:.1%} of HBM peak)")

    # Config 4: batch 2, 256-id prompt, 256 tokens; plain, then capture of
    # block 24 at every position for both sequences plus an FP32 steering
    # vector (unit N(0,1) direction x 8.0) added at block 24 of sequence 1.
    rng = np.random.default_rng(seed + 4)
    prompt4 = rng.integers(0, cfg.vocab, 256).astype(np.uint32)
    plan4 = Plan(model, batch=2, capacity=256 + 256 + 2)
    plain_ms, _, _ = timed_loop(device, queue, plan4, prompt4, 256, 256)
    u = rng.standard_normal(cfg.hidden)
    steer = (8.0 * u / np.linalg.norm(u)).astype(np.float32)
    plan4.set_capture(24)
    plan4.set_steering(1, 24, steer)
    hook_ms, _, _ = timed_loop(device, queue, plan4, prompt4, 256, 256)
    del plan4
    ctx4 = 256 + 1 + 254 / 2.0
    out["config4_capture_steering"] = {
        "batch": 2, "prompt": 256, "new_tokens": 256, "plain_ms_per_step": round(plain_ms, 4),
        "hooked_ms_per_step": round(hook_ms, 4), "overhead_frac": round(hook_ms / plain_ms - 1.0, 4),
        "tokens_per_s": round(2000.0 / hook_ms, 2),
        "hbm_frac": round(step_bytes(cfg, ctx4, 2) / (hook_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"config 4: batch 2 plain {plain_ms * 1e3:.1f} us/step, capture+steering {hook_ms * 1e3:.1f} us/step "
        f"({hook_ms / plain_ms - 1.0:+.2%})")

    # Config 5: batch 8 over one 192-id prefix with a BF16 N(0,1) x 40 row
    # replacing the embedding at position 96 of every sequence; 128 tokens
    # each, temperature 1.0, top-p 0.95, per-sequence MT19937-64 seeds.
    prompt5 = rng.integers(0, cfg.vocab, 192).astype(np.uint32)
    plan5 = Plan(model, batch=8, capacity=192 + 128 + 2)
    plan5.set_embedding_override(96, bf16_bits(40.0 * rng.standard_normal(cfg.hidden)), 0xFF)
    sampling = SamplingSettings("categorical", 1.0, 0, 0.95)
    ms5, _, _ = timed_loop(device, queue, plan5, prompt5, 128, 192, sampling, list(range(8)))
    del plan5
    ctx5 = 192 + 1 + 126 / 2.0
    out["config5_topp_batch8"] = {
        "batch": 8, "prompt": 192, "new_tokens": 128, "temperature": 1.0, "top_p": 0.95,
        "ms_per_step": round(ms5, 4), "tokens_per_s": round(8000.0 / ms5, 2),
        "hbm_frac": round(step_bytes(cfg, ctx5, 8) / (ms5 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"config 5: batch 8 top-p {ms5 * 1e3:.1f} us/step = {8000.0 / ms5:.1f} tok/s")
    return out


def cpu_info():
    """This host's logical CPU count, the CPUs this process may run on and
    the CPU model."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "model": name}


def cpu_threads():
    """Every CPU this job is given: OMP_NUM_THREADS where the host sets it
    (the GPU host gives each one-GPU job a share of its cores that way), else
    the CPUs of this process's affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else len(os.sched_getaffinity(0))


def cpu_baseline(model, plan, context, threads, seconds=10.0):
    """Times the CPU contract restatement on a bounded sample of the decode
    workload: whole tokens (the 36 block steps, each with its own block's
    weights and KV rows copied from the device, then the final norm + LM
    head) from `context` cached keys, repeated for at least `seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as o
    lib = o.lib()
    lib.or_set_threads(threads)
    cfg = model.config
    dims = o.Dims(cfg.hidden, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.ffn, cfg.vocab, cfg.rms_eps,
                  cfg.rope_theta)
    roles = (("input_norm", "input_norm"), ("wq", "q"), ("wk", "k"), ("wv", "v"), ("q_norm", "q_norm"),
             ("k_norm", "k_norm"), ("wo", "o"), ("post_norm", "post_norm"), ("wg", "gate"), ("wu", "up"),
             ("wd", "down"))
    blocks = [{name: np.ascontiguousarray(model.read(role, layer).reshape(-1)) for name, role in roles}
              for layer in range(cfg.layers)]
    lm = np.ascontiguousarray(model.read("lm_head").reshape(-1))
    weights = o.Qwen3Weights(dims, blocks, np.ascontiguousarray(model.read("final_norm")), lm, lm)
    kw = cfg.kv_heads * cfg.head_dim
    max_tokens = 512
    capacity = context + max_tokens + 1
    caches = []
    for layer in range(cfg.layers):
        k = np.zeros(capacity * kw, np.uint16)
        v = np.zeros(capacity * kw, np.uint16)
        keys, values = plan.read_cache(layer, 0, context)
        k[: context * kw] = keys
        v[: context * kw] = values
        caches.append((k, v))
    h0 = np.ascontiguousarray(plan.hidden(0))
    tokens, position = 0, context
    t0 = time.perf_counter()
    while tokens < max_tokens and (tokens == 0 or time.perf_counter() - t0 < seconds):
        h = h0.copy()
        for layer in range(cfg.layers):
            o.block_forward(weights, layer, h, 1, position, *caches[layer])
        o.logits(weights, h)
        position += 1
        tokens += 1
    elapsed = time.perf_counter() - t0
    info = cpu_info()
    return {
        "value": round(tokens / elapsed, 4),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "nproc": info["nproc"],
        "affinity_cpus": info["affinity"],
        "cpu_model": info["model"],
        "sample": (f"CPU contract restatement (oracle/, C, -O3, {threads} OpenMP threads = every CPU this job is "
                   f"given; host nproc {info['nproc']}, {info['model']}): {tokens} whole decode tokens "
                   f"({cfg.layers} block steps with each block's own weights and KV rows + final norm + LM head) "
                   f"from {context} cached keys, {elapsed:.1f} s"),
    }


# The decode kernels the HBM-traffic counter runs measure, in launch order:
# (hook index of dl_plan_launch_kernel, kernel name as rocprofv3 reports it
# with the namespace stripped (a prefix), launches, plan).  The "short" plan
# sits at 384 visible keys (the bench's last decode position), the "long" one
# at 4608 (config 3's last).
TRAFFIC_KERNELS = (
    (0, "k_qkv<1, 0, 1>", 8, "short"),
    (4, "k_residual<16, 1, 1>", 8, "short"),
    (5, "k_gateup<1>", 8, "short"),
    (6, "k_residual<32, 1, 1>", 8, "short"),
    (7, "k_lm_head<1>", 4, "short"),
    (8, "k_attn_fused", 8, "short"),
    (10, "k_attn_o", 8, "short"),
    (12, "k_qkv_attn_o", 8, "short"),
    (1, "k_attn_qk", 8, "long"),
    (2, "k_attn_softmax", 8, "long"),
    (3, "k_attn_pv", 8, "long"),
)
TRAFFIC_KEYS = {"short": 384, "long": 4608}
TRAFFIC_COPY_BYTES = 256 << 20
TRAFFIC_LAYERS = 4
TRAFFIC_PATH = os.path.join(ROOT, "profiles", "traffic.json")


def attention_bytes(cfg, which, keys):
    """Algorithmic bytes of one attention launch at batch 1 over `keys`
    visible keys: BF16 K and V rows of one layer, FP32 scores and
    probabilities of the 32 query heads, the BF16 query / key / output rows."""
    KW, QW = cfg.kv_heads * cfg.head_dim, cfg.q_heads * cfg.head_dim
    rows, scores = keys * KW * 2, cfg.q_heads * keys * 4
    return {
        1: rows + scores + QW * 2 + 2 * KW * 2,      # K rows, scores out, q / k in, k append
        2: 2 * scores,                               # scores in, probabilities out
        3: rows + scores + QW * 2,                   # V rows, probabilities in, att out
        8: 2 * rows + QW * 2 + 2 * KW * 2 + QW * 2,  # K and V rows, q / k in, k append, att out
    }[which]


def launch_bytes(cfg, which, keys):
    if which == 10:  # fused attention + O projection
        return attention_bytes(cfg, 8, keys) + kernel_bytes(cfg, 4)
    if which == 12:  # fused QKV + attention + O projection
        return kernel_bytes(cfg, 0) + attention_bytes(cfg, 8, keys) + kernel_bytes(cfg, 4)
    return attention_bytes(cfg, which, keys) if which in (1, 2, 3, 8) else kernel_bytes(cfg, which)


def sources_digest():
    """SHA-256 over the backend's sources and build script: counter results
    are valid only for the kernels they were measured on."""
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "dolittle_amd", "csrc")
    paths = sorted(os.path.join(csrc, n) for n in os.listdir(csrc) if n.endswith((".hip", ".h", ".cpp")))
    for path in paths + [os.path.join(ROOT, "dolittle_amd", "build.py")]:
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def traffic_driver(device, queue, seed):
    """The program the two counter runs profile (rocprofv3 --pmc FETCH_SIZE,
    then WRITE_SIZE): Qwen3-8B blocks (4 of them; every block has the same
    shapes) with the full 151,936-row LM head, two plans brought to 384 and
    4608 visible keys, then TRAFFIC_KERNELS' launches, then three copies of
    256 MiB device to device, the calibration of known size."""
    from dolittle_amd import _lib
    from dolittle_amd.qwen3 import Plan, Qwen3Config, Qwen3Model
    cfg = Qwen3Config(layers=TRAFFIC_LAYERS)
    model = Qwen3Model(device, queue, cfg)
    model.fill_synthetic(seed, 0.02)
    rng = np.random.default_rng(seed)
    plans = {}
    for name, keys in TRAFFIC_KEYS.items():
        prompt = rng.integers(0, cfg.vocab, keys - 2).astype(np.uint32)
        plan = Plan(model, batch=1, capacity=keys + 1)
        plan.prefill(prompt)
        plan.generate(prompt, 2)
        _, results = plan.collect()
        assert results[0]["position"] == keys, results
        _lib.call("dl_plan_bench_prepare", plan.handle)
        plans[name] = plan
    queue.drain()
    log("traffic driver: measured launches")
    for which, _, count, plan in TRAFFIC_KERNELS:
        _lib.call("dl_plan_launch_kernel", plans[plan].handle, which, 0, count)
    a, b = device.allocate(TRAFFIC_COPY_BYTES), device.allocate(TRAFFIC_COPY_BYTES)
    for _ in range(3):
        queue.copy(b, a, TRAFFIC_COPY_BYTES)
    queue.drain()
    log("traffic driver done")


def traffic_summary(fetch_csv, write_csv):
    """Reads the counter CSVs of the two runs of traffic_driver and writes
    profiles/traffic.json: per kernel the mean FETCH_SIZE / WRITE_SIZE (KiB
    per dispatch) of its measured launches (the last dispatches of that
    name), each scaled by what the counter reads for the 256 MiB copy."""
    import csv
    from dolittle_amd.qwen3 import Qwen3Config
    cfg = Qwen3Config()
    per = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        got = []
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    name = r["Kernel_Name"].replace("void ", "").replace("dl::(anonymous namespace)::", "")
                    got.append((int(r["Dispatch_Id"]), name, float(r["Counter_Value"])))
        got.sort()
        per[counter] = got

    def last(counter, match, count):
        vals = [v for _, n, v in per[counter] if match(n)][-count:]
        if len(vals) != count:
            raise SystemExit(f"{counter}: found {len(vals)} of {count} dispatches")
        return sum(vals) / count

    copy = lambda n: "copyBuffer" in n  # noqa: E731
    kib = TRAFFIC_COPY_BYTES / 1024
    fetch_copy, write_copy = last("FETCH_SIZE", copy, 3), last("WRITE_SIZE", copy, 3)
    ff, wf = kib / fetch_copy, kib / write_copy
    kernels = {}
    for which, prefix, count, plan in TRAFFIC_KERNELS:
        match = lambda n, p=prefix: n.startswith(p)  # noqa: E731
        fetch, write = last("FETCH_SIZE", match, count), last("WRITE_SIZE", match, count)
        hbm = round((fetch * ff + write * wf) * 1024)
        alg = launch_bytes(cfg, which, TRAFFIC_KEYS[plan])
        kernels[prefix] = {"hook": which, "keys": TRAFFIC_KEYS[plan], "dispatches": count,
                           "fetch_size_kib": round(fetch, 2), "write_size_kib": round(write, 2),
                           "hbm_bytes_per_launch": hbm, "algorithmic_bytes_per_launch": alg,
                           "traffic_over_algorithmic": round(hbm / alg, 4)}
        log(f"{prefix:<24} fetch {fetch:12.2f} KiB  write {write:10.2f} KiB  -> {hbm:>12,} B  "
            f"({hbm / alg:.3f} x algorithmic)")
    out = {"sources_sha256": sources_digest(),
           "copy_calibration": {"bytes": TRAFFIC_COPY_BYTES, "fetch_size_kib": round(fetch_copy, 2),
                                "write_size_kib": round(write_copy, 2), "fetch_factor": round(ff, 5),
                                "write_factor": round(wf, 5)},
           "kernels": kernels,
           "command": "rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) -- python3 bench.py --traffic-driver; "
                      "python3 bench.py --traffic-summary FETCH.csv WRITE.csv"}
    with open(TRAFFIC_PATH, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    log(f"wrote {TRAFFIC_PATH}")


def load_traffic(prefix):
    """HBM bytes per launch of one kernel from profiles/traffic.json, or
    (None, reason) when absent or measured on other sources."""
    if not os.path.exists(TRAFFIC_PATH):
        return None, "no counter measurement"
    with open(TRAFFIC_PATH) as f:
        data = json.load(f)
    if data.get("sources_sha256") != sources_digest():
        return None, "stale: counters were measured on other kernel sources"
    entry = data["kernels"].get(prefix)
    return (entry["hbm_bytes_per_launch"], "rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated") if entry \
        else (None, "kernel not measured")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=250)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--kernel-iters", type=int, default=72)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-driver", action="store_true",
                    help="only launch the decode kernels a few times each and copy 256 MiB three times "
                         "(the program run under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic.json from the two counter runs' CSVs (no GPU)")
    ap.add_argument("--mfma-prompt", type=int, default=4096,
                    help="prompt length of the MFMA prefill measurement (0 skips it)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the decode measurements of configs 3 (4.6K context), 4 and 5")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (PMC scaling reference)")
    args = ap.parse_args()
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary)
        return 0
    if args.gpus != 1:
        print("bench.py measures one MI355X: this backend has no multi-GPU path; run with --gpus 1",
              file=sys.stderr)
        return 2

    from dolittle_amd import Device, Event, _lib
    from dolittle_amd.qwen3 import Plan, Qwen3Config, Qwen3Model

    device = Device(0)
    queue = device.create_queue()
    if args.traffic_driver:
        traffic_driver(device, queue, args.seed)
        return 0
    cfg = Qwen3Config()
    t0 = time.perf_counter()
    model = Qwen3Model(device, queue, cfg)
    model.fill_synthetic(args.seed, 0.02)
    queue.drain()
    log(f"model resident: {model.resident_bytes() / 2**30:.2f} GiB in {time.perf_counter() - t0:.1f}s")
    max_new = 1 + args.warmup + args.steps
    capacity = args.prompt + max_new + 1
    plan = Plan(model, batch=1, capacity=capacity)
    prompt = np.random.default_rng(args.seed).integers(0, cfg.vocab, args.prompt).astype(np.uint32)
    # Warm: the first pass over the prompt allocates the chunk's row buffers
    # (sized to the longest chunk a pass has needed); the timed pass below
    # recomputes every position into the same caches.
    plan.prefill(prompt)
    e_p0, e_p1, e_a, e_b = Event(device), Event(device), Event(device), Event(device)
    queue.drain()
    e_p0.record(queue)
    plan.prefill(prompt)  # exact prompt pass over positions [0, prompt - 1)
    e_p1.record(queue)
    queue.drain()
    plan.prepare_generation(prompt, max_new)  # resumes at the last prompt position
    plan.decode_steps(1)  # consumes the last prompt position, selects token 1
    plan.decode_steps(args.warmup)
    queue.drain()
    e_a.record(queue)
    plan.decode_steps(args.steps)
    e_b.record(queue)
    queue.drain()
    plan.decode_steps(1)  # consumes the last selection (completes the loop)
    tokens, results = plan.collect()
    prefill_ms = e_p0.elapsed_ms(e_p1)
    prefill_positions = args.prompt - 1
    decode_ms = e_a.elapsed_ms(e_b)
    ms_per_step = decode_ms / args.steps
    tok_s = 1000.0 / ms_per_step
    assert results[0]["generated"] == max_new, results
    first_ctx = args.prompt + 1 + args.warmup
    mean_context = first_ctx + (args.steps - 1) / 2.0
    bytes_step = step_bytes(cfg, mean_context)
    step_gbs = bytes_step / (ms_per_step * 1e-3) / 1e9
    log(f"exact prefill {prefill_positions} positions in {prefill_ms:.2f} ms; decode {ms_per_step * 1e3:.1f} us/token "
        f"= {tok_s:.1f} tok/s; step {step_gbs:.0f} GB/s ({step_gbs / HBM_PEAK_GBS:.1%} of HBM peak)")

    # Live per-kernel timing on the plan's stream, cycling layers so every
    # launch streams distinct weights.
    _lib.call("dl_plan_bench_prepare", plan.handle)
    kernels = {}
    prefixes = {which: prefix for which, prefix, _, _ in TRAFFIC_KERNELS}
    names = {0: "k_qkv", 4: "k_residual<16> (O)", 5: "k_gateup", 6: "k_residual<32> (down)", 7: "k_lm_head",
             8: "k_attn_fused", 10: "k_attn_o (attention + O)",
             12: "k_qkv_attn_o (QKV + attention + O)"}
    # The bench control sits at the last consumed position: every position
    # so far is a visible key.
    attn_keys = args.prompt + max_new
    for which in (5, 7, 0, 6, 4, 8, 10, 12):
        iters = args.kernel_iters if which != 7 else max(8, args.kernel_iters // 8)
        _lib.call("dl_plan_launch_kernel", plan.handle, which, 0, 2)  # warm
        ea, eb = Event(device), Event(device)
        queue.drain()
        ea.record(queue)
        _lib.call("dl_plan_launch_kernel", plan.handle, which, 0, iters)
        eb.record(queue)
        us = ea.elapsed_ms(eb) * 1e3 / iters
        alg = launch_bytes(cfg, which, attn_keys)
        gbs = alg / (us * 1e-6) / 1e9
        entry = {"us": round(us, 2), "algorithmic_bytes": alg, "GB/s": round(gbs, 1),
                 "frac": round(gbs / HBM_PEAK_GBS, 4)}
        if which in (8, 10, 12):
            # The four query heads of a group share their K and V rows
            # through L2: the bytes count each row once.
            entry["keys"] = attn_keys
        if which in prefixes and (which != 8 or attn_keys == TRAFFIC_KEYS["short"]):
            entry["traffic"] = load_traffic(prefixes[which])[0]
        kernels[names[which]] = entry
        log(f"  {names[which]:<24} {us:8.2f} us  {gbs:7.0f} GB/s  {gbs / HBM_PEAK_GBS:.1%}")
    dominant = kernels["k_gateup"]

    # Replay cost of the step graph with the loop stopped: every kernel
    # exits at entry, leaving launch and dispatch overhead.
    queue.drain()
    ea, eb = Event(device), Event(device)
    ea.record(queue)
    plan.decode_steps(20)
    eb.record(queue)
    idle_us = ea.elapsed_ms(eb) * 1e3 / 20
    log(f"  idle step graph           {idle_us:8.2f} us")

    if args.copy_calibration_mib:
        n = args.copy_calibration_mib << 20
        a, b = device.allocate(n), device.allocate(n)
        queue.copy(b, a, n)
        queue.drain()

    # BASELINE config 3's prompt pass on the MFMA prefill path (tolerance
    # path, not bit-exact): 4096 prompt ids, positions 0..4094 as GEMMs.
    mfma, pplan, long_prompt = None, None, None
    if args.mfma_prompt:
        n = args.mfma_prompt
        pplan = Plan(model, batch=1, capacity=n + 512 + 1)
        long_prompt = np.random.default_rng(args.seed + 3).integers(0, cfg.vocab, n).astype(np.uint32)
        pplan.prefill(long_prompt, mfma=True)  # warm (allocates the row buffers)
        queue.drain()
        runs = 3
        ea, eb = Event(device), Event(device)
        ea.record(queue)
        for _ in range(runs):
            pplan.prefill(long_prompt, mfma=True)
        eb.record(queue)
        queue.drain()
        ms = ea.elapsed_ms(eb) / runs
        rows = n - 1
        proj = 2 * rows * cfg.layers * (cfg.hidden * (cfg.q_heads + 2 * cfg.kv_heads) * cfg.head_dim
                                        + cfg.q_heads * cfg.head_dim * cfg.hidden + 3 * cfg.hidden * cfg.ffn)
        pairs = rows * (rows + 1) // 2
        attn = 4 * pairs * cfg.head_dim * cfg.q_heads * cfg.layers
        tflops = (proj + attn) / (ms * 1e-3) / 1e12
        mfma = {"prompt": n, "positions": rows, "ms": round(ms, 2), "tokens_per_s": round(rows / (ms * 1e-3), 1),
                "flop": proj + attn, "achieved_tflops": round(tflops, 1), "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                "parity": "non-conforming tolerance path (MFMA accumulation order; as far from the exact pass as one-ulp "
                          "flips in block 0's cache); the parity path is prefill_tokens_per_s"}
        log(f"MFMA prefill {rows} positions in {ms:.1f} ms = {rows / (ms * 1e-3):.0f} tok/s, "
            f"{tflops:.0f} TFLOP/s ({tflops / MFMA_BF16_PEAK_TFLOPS:.1%} of BF16 peak)")

    others = {}
    if not args.no_other_configs:
        others = other_configs(device, queue, model, cfg, args.seed, pplan, long_prompt)
        del pplan

    cpu = None
    if not args.no_cpu_baseline:
        threads = cpu_threads()
        t0 = time.perf_counter()
        cpu = cpu_baseline(model, plan, int(mean_context), threads)
        log(f"cpu baseline: {cpu['value']} tok/s ({time.perf_counter() - t0:.1f}s)")

    gateup_bytes = kernel_bytes(cfg, 5)
    gateup_traffic, gateup_traffic_source = load_traffic(prefixes[5])
    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) BF16 weights generated on device, seeded uniform prompt ids)",
        "config": {
            "workload": "BASELINE config 2: Qwen3-8B, 36 blocks, tied 151936-row LM head, batch 1, "
                        f"{args.prompt}-id prompt, greedy decode of {max_new} tokens",
            "timed_decode_positions": [first_ctx, first_ctx + args.steps - 1],
            "parallelism": "single-gpu",
        },
        "prefill_tokens_per_s": round(prefill_positions / (prefill_ms * 1e-3), 1),
        "prefill_exact": {"positions": prefill_positions, "ms": round(prefill_ms, 3),
                          "path": "dl_plan_prefill: chunks of up to 512 positions through many-row "
                                  "exact GEMMs and row-block attention, caches bit-identical to the token loop"},
        "prefill_mfma": mfma,
        "hbm_roofline_step": {"bytes_per_step": int(bytes_step), "achieved_GBs": round(step_gbs, 1),
                              "peak_GBs": HBM_PEAK_GBS, "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": {
            "kernel": "k_gateup (RMSNorm + gate/up GEMV + SiLU*up, one block)",
            "bound": "hbm",
            "achieved": dominant["GB/s"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dominant["frac"],
            "traffic": gateup_traffic,
            "traffic_source": gateup_traffic_source,
            "algorithmic_bytes_per_launch": gateup_bytes,
            "avg_launch_us": dominant["us"],
        },
        "kernels": kernels,
        "other_configs": others,
        "idle_step_graph_us": round(idle_us, 2),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
