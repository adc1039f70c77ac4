"""bench.py's one-line JSON contract: the fields, types and sub-objects the
benchmark line carries (metric and unit, throughput value, timing, dtype,
workload config, roofline of the dominant kernel, CPU baseline), and its
refusal of multi-GPU runs."""

import json
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def test_multi_gpu_runs_are_refused():
    """--gpus above 1 exits with status 2 and says why, before any device work."""
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stdout + r.stderr
    assert r.stdout.strip() == "" or not r.stdout.strip().startswith("{")


@pytest.mark.gpu
def test_bench_line_contract():
    """A short run prints exactly one JSON line with the contract's fields: the
    headline metric as whole-job throughput, the dominant kernel's roofline
    (achieved, peak, fraction, traffic slot) and the CPU baseline (value,
    unit, cores, kind, sample)."""
    r = subprocess.run([sys.executable, "bench.py", "--steps", "3", "--warmup", "1", "--no-copy", "--no-traffic",
                        "--no-extra", "--cold-iters", "2", "--cpu-budget", "0.5"],
                       capture_output=True, text=True, timeout=600, cwd=ROOT)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, lines
    d = json.loads(lines[0])
    for key, typ in (("metric", str), ("value", float), ("unit", str), ("n_gpus", int), ("steps", int),
                     ("warmup", int), ("ms_per_step", float), ("higher_is_better", bool), ("scaling", str),
                     ("dtype", str), ("data", str), ("config", dict), ("roofline", dict), ("cpu_baseline", dict)):
        assert key in d, key
        assert isinstance(d[key], typ), (key, type(d[key]))
    assert "vs_baseline" in d
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["unit"] == "GB/s" and d["higher_is_better"] is True and d["dtype"] == "fp16"
    assert d["config"]["workload"].startswith("C2")
    # value is the algorithmic bytes of one step over the measured step time
    step_s = d["ms_per_step"] * 1e-3
    assert abs(d["config"]["algorithmic_bytes"] / step_s / 1e9 - d["value"]) / d["value"] < 0.01
    rf = d["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in rf, key
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000
    assert 0 < rf["frac"] < 1 and abs(rf["achieved"] / rf["peak"] - rf["frac"]) < 1e-3
    cb = d["cpu_baseline"]
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in cb, key
    assert cb["kind"] in ("reference", "port") and cb["cores"] >= 1 and cb["value"] > 0
