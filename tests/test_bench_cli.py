"""The native bench CLI (paged-attention_amd/bench/bench_decode.cpp): the
reference's bench/bench_decode.cu modes, flags and CSV columns."""

import csv
import io
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
BIN = ROOT / "paged-attention_amd" / "bench" / "_build" / "bench_decode"
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
HEADER = "gpu,dtype,batch,seq_len,hq,hkv,dim,page,ctas,segments,time_us,gbps,pct_peak"   # bench_decode.cu:194-196


def _bin() -> pathlib.Path:
    if not BIN.exists():
        import importlib.util
        spec = importlib.util.spec_from_file_location("pa_build", ROOT / "paged-attention_amd" / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build_bench()
    return BIN


def _run(*args, timeout=300):
    proc = subprocess.run([str(_bin()), *args], capture_output=True, text=True, timeout=timeout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return proc.stdout


def test_help_needs_no_device():
    out = _run("--help")
    assert out.startswith("usage: bench_decode sweep|ctas|pagesize|capacity|copy|single")


@pytest.mark.gpu
def test_single_row_columns():
    out = _run("single", "--batch", "2", "--len", "300", "--iters", "3")
    lines = out.strip().splitlines()
    assert lines[0] == HEADER
    row = next(csv.DictReader(io.StringIO(out)))
    assert row["dtype"] == "fp16" and int(row["batch"]) == 2 and int(row["seq_len"]) == 300
    assert float(row["time_us"]) > 0 and int(row["ctas"]) > 0 and int(row["segments"]) >= 16
    out = _run("single", "--batch", "1", "--len", "1000", "--dtype", "fp8", "--page", "8", "--iters", "3")
    row = next(csv.DictReader(io.StringIO(out)))
    assert row["dtype"] == "fp8_e4m3" and row["page"] == "8"


@pytest.mark.gpu
def test_capacity_rows_match_reference():
    """The capacity mode reproduces results/h100_capacity.csv (1 GiB budget)."""
    out = _run("capacity")
    got = list(csv.DictReader(io.StringIO(out)))
    want = list(csv.DictReader(open(GOLDEN / "capacity_rows.csv")))
    key = lambda r: (r["dtype"], r["layout"], r["actual_len"])   # noqa: E731
    assert {key(r): (r["sequences"], r["bytes_per_seq"]) for r in got} == \
        {key(r): (r["sequences"], r["bytes_per_seq"]) for r in want}


def test_python_twin_help_needs_no_device():
    """`python -m pa_amd.bench_decode --help` prints the usage without touching a
    GPU (as the native CLI does); an unknown mode exits 2."""
    import sys
    cwd = ROOT / "paged-attention_amd"
    r = subprocess.run([sys.executable, "-m", "pa_amd.bench_decode", "--help"], capture_output=True, text=True,
                       timeout=120, cwd=cwd)
    assert r.returncode == 0
    for mode in ("sweep", "ctas", "pagesize", "capacity", "copy", "single", "append", "order"):
        assert mode in r.stdout
    r = subprocess.run([sys.executable, "-m", "pa_amd.bench_decode", "nosuchmode"], capture_output=True, text=True,
                       timeout=120, cwd=cwd)
    assert r.returncode == 2


def test_bad_command_lines_exit_2_without_a_device():
    """Unknown options, malformed or missing values, stray arguments, an
    unknown dtype or mode: the usage goes to stderr and the CLI exits with 2
    before it touches a device."""
    for args in (["single", "--bogus"], ["single", "--batch", "x"], ["ctas", "--batch"], ["single", "extra"],
                 ["single", "--dtype", "fp9"], ["nosuchmode"], ["single", "--contiguous-pages=1"]):
        proc = subprocess.run([str(_bin()), *args], capture_output=True, text=True, timeout=60)
        assert proc.returncode == 2, (args, proc.stdout, proc.stderr)
        assert "usage: bench_decode" in proc.stderr
    out = _run("--help", "--batch=3")
    assert out.startswith("usage: bench_decode")


def test_page_orders_are_permutations():
    """The page placements of the `order` mode: each is a permutation of the
    batch's pages; memory order is the identity, interleaved hands page i of
    row b the rank i * batch + b, and the grouped shuffles keep every page in
    its group (within) or every group whole (groups)."""
    import sys
    import numpy as np
    sys.path.insert(0, str(ROOT / "paged-attention_amd"))
    from pa_amd.bench_decode import page_orders
    batch, npg, page_bytes = 8, 512, 32 << 10
    n = batch * npg
    orders = page_orders(batch, npg, page_bytes)
    assert set(orders) == {"memory_order", "interleaved", "shuffled", "shuffled_within_256KiB",
                           "256KiB_groups_shuffled", "shuffled_within_2MiB", "2MiB_groups_shuffled"}
    for name, perm in orders.items():
        assert np.array_equal(np.sort(perm), np.arange(n)), name
    assert np.array_equal(orders["memory_order"], np.arange(n))
    inter = orders["interleaved"].reshape(batch, npg)
    assert inter[3, 5] == 5 * batch + 3
    for span, g in (("256KiB", 8), ("2MiB", 64)):
        w = orders[f"shuffled_within_{span}"].reshape(-1, g)
        assert np.array_equal(w // g, np.repeat(np.arange(n // g)[:, None], g, axis=1))
        q = orders[f"{span}_groups_shuffled"].reshape(-1, g)
        assert np.array_equal(q - q[:, :1], np.repeat(np.arange(g)[None, :], n // g, axis=0))
        assert np.array_equal(np.sort(q[:, 0] // g), np.arange(n // g))


@pytest.mark.gpu
def test_page_order_rows():
    """`order` times one decode shape under every placement of its pages."""
    import sys
    cwd = ROOT / "paged-attention_amd"
    r = subprocess.run([sys.executable, "-m", "pa_amd.bench_decode", "order", "--batch", "4", "--len", "2048",
                        "--iters", "3", "--warm"], capture_output=True, text=True, timeout=300, cwd=cwd)
    assert r.returncode == 0, r.stdout + r.stderr
    rows = list(csv.DictReader(io.StringIO(r.stdout)))
    assert {row["order"] for row in rows} >= {"memory_order", "interleaved", "shuffled"}
    assert all(float(row["time_us"]) > 0 and row["page"] == "16" for row in rows)
