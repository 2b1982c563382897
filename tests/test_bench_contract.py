"""bench.py's output contract: one JSON line with the driver's keys, the roofline and CPU-baseline objects; more than
one GPU refused with a message (CPU), and a tiny configuration measured end to end (GPU)."""

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout.strip() == ""


@pytest.mark.gpu
def test_tiny_bench_line():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--train-tokens", "3000000", "--query-tokens",
                        "200001", "--steps", "1", "--warmup", "1", "--no-secondary", "--cpu-tokens", "1000000",
                        "--cpu-queries", "20000", "--parity-windows", "50"], capture_output=True, text=True,
                       timeout=600, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    j = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in j, key
    assert j["n_gpus"] == 1 and j["steps"] == 1 and j["value"] > 0 and j["higher_is_better"] is True
    assert "workload" in j["config"] and j["vs_baseline"] is None
    rf = j["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-9 and rf["achieved"] > 0
    cpu = j["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["cores"] >= 1 and cpu["value"] > 0 and cpu["sample"]
    # the GPU's outputs against the oracle's: the baseline's prefix sample and windows over the whole corpus
    par = j["parity"]
    assert par["mismatching_positions"] == 0
    assert par["prefix"]["positions"] == 20000 and par["windows"]["positions"] >= 50 * 64
    assert j["roofline_family"]["frac"] > 0 and j["count_path_roofline"]["frac"] > 0
    # the scans' probe bound against the measured random-load rate of a same-size table: probes per second here (the
    # committed line counters describe the default workload only, and are not used for this one)
    pr = j["probe_roofline"]
    assert pr["peak"] > 0 and pr["achieved"] > 0 and abs(pr["frac"] - pr["achieved"] / pr["peak"]) < 1e-9
    assert pr["achieved_is"] == "probes" and rf["traffic"] is None
    for v in j["levels"].values():
        assert 0 <= v["hits"] <= v["probed"] <= j["config"]["corpus_tokens"]
