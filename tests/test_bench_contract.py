"""bench.py's contract: one GPU only (--gpus N > 1 exits with a message,
before anything touches a GPU), the driver's flags, and (on a GPU) the one
JSON line with the fields, roofline and CPU baseline the driver reads."""

from __future__ import annotations

import json
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    for n in ("2", "8"):
        r = _run("--gpus", n)
        assert r.returncode == 2
        assert "one GPU" in r.stderr
        assert r.stdout == ""


def test_world_size_above_one_exits_the_same_way():
    import os
    env = dict(os.environ, WORLD_SIZE="2", RANK="0", LOCAL_RANK="0")
    r = subprocess.run([sys.executable, str(ROOT / "bench.py")], capture_output=True, text=True, timeout=120,
                       cwd=ROOT, env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def _no_children(monkeypatch):
    """Makes any attempt to start a child process fail the test."""
    import os

    def refuse(*a, **k):
        raise AssertionError(f"child process started: {a[:1]}")
    monkeypatch.setattr(subprocess, "Popen", refuse)
    for name in ("system", "execv", "execve", "execvp", "execvpe", "posix_spawn", "posix_spawnp", "fork"):
        if hasattr(os, name):
            monkeypatch.setattr(os, name, refuse)


def test_profiler_preload_is_detected():
    import bench
    assert bench.profiler_preloaded({"LD_PRELOAD": "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so"})
    assert bench.profiler_preloaded({"ROCPROF_KERNEL_TRACE": "1"})
    assert bench.profiler_preloaded({"ROCPROFILER_LIBRARY_CTOR": "1"})
    assert not bench.profiler_preloaded({"LD_PRELOAD": "", "PATH": "/usr/bin"})
    assert not bench.profiler_preloaded({})


def test_no_child_process_under_a_profiler(monkeypatch):
    """Under a profiler's preload every child would start GPU-initialized (and
    rocprofv3 is a `#!/usr/bin/env python3` script, i.e. an exec): the traffic
    passes are skipped and nothing is started."""
    import argparse

    import bench
    _no_children(monkeypatch)
    monkeypatch.setenv("LD_PRELOAD", "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so")
    args = argparse.Namespace(config="c2", page_size=16, ctas=0)
    assert bench.measure_traffic(args) is None


def test_device_report_starts_no_child_process(monkeypatch):
    """The device facts come from the HIP runtime in-process (no amd-smi, which
    is itself a `#!/usr/bin/env python3` script); without a device it says so."""
    import bench
    _no_children(monkeypatch)
    monkeypatch.setenv("ROCPROF_KERNEL_TRACE", "1")
    d = bench.device_report(0)
    assert isinstance(d, dict) and "source" in d
    assert "amd-smi" not in json.dumps(d)


def test_help_lists_the_driver_flags():
    r = _run("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--config"):
        assert flag in r.stdout


@pytest.mark.gpu
def test_bench_line_contract():
    """A short run prints exactly one JSON line with the contract's fields: the
    headline metric as whole-job throughput, the dominant kernel's roofline
    (achieved, peak, fraction, traffic slot) and the CPU baseline (value,
    unit, cores, kind, sample)."""
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--steps", "3", "--warmup", "1", "--no-copy",
                        "--no-traffic", "--no-extra", "--cold-iters", "2", "--cpu-budget", "0.5"],
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
    assert d["config"]["merge"] == "in the split kernel, inside one block"   # one launch per step
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
