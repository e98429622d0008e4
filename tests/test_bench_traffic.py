"""bench.py's HBM-traffic bookkeeping on the CPU: the counter summary's
arithmetic on synthetic counter CSVs, and that bytes measured on other
sources are refused."""
import csv
import json
import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

FIELDS = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def write_csv(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        for i, (name, value) in enumerate(rows):
            w.writerow({"Correlation_Id": i, "Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": counter,
                        "Counter_Value": value})


def synthetic_runs(tmp_path, fetch_scale=0.5):
    """One counter run per counter: setup dispatches of every kernel (which
    must be ignored), the measured launches, then the three copies."""
    kib = bench.TRAFFIC_COPY_BYTES / 1024
    fetch, write = [], []
    for _, prefix, count, _ in bench.TRAFFIC_KERNELS:
        name = f"void dl::(anonymous namespace)::{prefix}(dl::(anonymous namespace)::Args)"
        fetch.append((name, 1e9))  # a setup dispatch: not among the last `count`
        write.append((name, 1e9))
    expect = {}
    for n, (which, prefix, count, plan) in enumerate(bench.TRAFFIC_KERNELS):
        name = f"void dl::(anonymous namespace)::{prefix}(dl::(anonymous namespace)::Args)"
        f_kib, w_kib = 1000.0 * (n + 1), 10.0 * (n + 1)
        for _ in range(count):
            fetch.append((name, f_kib))
            write.append((name, w_kib))
        expect[prefix] = round((f_kib / fetch_scale + w_kib) * 1024)
    for _ in range(3):
        fetch.append(("__amd_rocclr_copyBuffer", kib * fetch_scale))
        write.append(("__amd_rocclr_copyBuffer", kib))
    fp, wp = tmp_path / "f.csv", tmp_path / "w.csv"
    write_csv(fp, "FETCH_SIZE", fetch)
    write_csv(wp, "WRITE_SIZE", write)
    return str(fp), str(wp), expect


def test_summary_scales_by_the_copy_and_takes_the_measured_launches(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "TRAFFIC_PATH", str(tmp_path / "traffic.json"))
    fp, wp, expect = synthetic_runs(tmp_path)
    bench.traffic_summary(fp, wp)
    data = json.load(open(tmp_path / "traffic.json"))
    assert data["copy_calibration"]["fetch_factor"] == pytest.approx(2.0)
    assert data["copy_calibration"]["write_factor"] == pytest.approx(1.0)
    for prefix, want in expect.items():
        assert data["kernels"][prefix]["hbm_bytes_per_launch"] == want, prefix
        assert bench.load_traffic(prefix)[0] == want


def test_missing_dispatches_are_an_error(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "TRAFFIC_PATH", str(tmp_path / "traffic.json"))
    fp, wp, _ = synthetic_runs(tmp_path)
    rows = [r for r in csv.DictReader(open(fp)) if "k_attn_pv" not in r["Kernel_Name"]]
    write_csv(fp, "FETCH_SIZE", [(r["Kernel_Name"], float(r["Counter_Value"])) for r in rows])
    with pytest.raises(SystemExit):
        bench.traffic_summary(fp, wp)


def test_counters_of_other_sources_are_refused(tmp_path, monkeypatch):
    path = tmp_path / "traffic.json"
    monkeypatch.setattr(bench, "TRAFFIC_PATH", str(path))
    entry = {"hbm_bytes_per_launch": 123}
    path.write_text(json.dumps({"sources_sha256": "0" * 64, "kernels": {"k_gateup<1>": entry}}))
    value, reason = bench.load_traffic("k_gateup<1>")
    assert value is None and reason.startswith("stale")
    path.write_text(json.dumps({"sources_sha256": bench.sources_digest(), "kernels": {"k_gateup<1>": entry}}))
    assert bench.load_traffic("k_gateup<1>")[0] == 123
    assert bench.load_traffic("k_lm_head<1>")[0] is None


def test_committed_counters_name_every_measured_kernel():
    data = json.load(open(os.path.join(bench.ROOT, "profiles", "traffic.json")))
    assert set(data["kernels"]) == {prefix for _, prefix, _, _ in bench.TRAFFIC_KERNELS}
    for entry in data["kernels"].values():
        assert 0.99 < entry["traffic_over_algorithmic"] < 1.5
