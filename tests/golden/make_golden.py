"""Writes the golden fixtures under tests/golden/ (run in the build container).

    python tests/golden/make_golden.py [--reference /root/reference]

Fixtures (data only; nothing here is reference source):
  planner_rows.csv  (source, dtype, batch, seq_len, hkv, tile, requested, ctas, segments):
                    the plan shape columns of the reference's own results
                    (results/h100_sweep.csv, h100_pagesize.csv, h100_ctas.csv).
                    `requested` is the grid the bench asked for: the H100
                    default_ctas (132 SMs x 2 for fp16, x 3 for fp8, decode.cu:55-63)
                    for sweep/pagesize rows, and bench_decode.cu:276's list
                    {sms/2, sms, 2sms, 3sms, wave=3sms} for the ctas rows.
  capacity_rows.csv results/h100_capacity.csv verbatim (1 GiB budget, P=16,
                    Hkv=8, D=128, max_len 8192).
  e4m3_decode.npy   float32 value of each of the 256 E4M3 codes, decoded by
                    torch.float8_e4m3fn (an implementation independent of ours).
  e4m3_encode.npz   x (float32) and torch's E4M3 code for x, |x| < 464 only,
                    where torch and saturating (satfinite) conversion agree.
  accuracy_rows.csv (dtype, batch, seq_len, max_abs_diff_vs_ref, fp8_err_vs_fp16,
                    fp8_rel_err_vs_fp16): the accuracy columns of
                    results/h100_flashinfer.csv (the reference kernel against its
                    fp32 torch reference and FP8 against fp16 on the same seed).
"""

from __future__ import annotations

import argparse
import csv
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
SMS_H100 = 132


def planner_rows(ref: pathlib.Path) -> list[dict]:
    rows = []
    for name in ("h100_sweep.csv", "h100_pagesize.csv"):
        with open(ref / "results" / name) as f:
            for r in csv.DictReader(f):
                dtype = r["dtype"]
                rows.append(dict(source=name, dtype=dtype, batch=int(r["batch"]), seq_len=int(r["seq_len"]),
                                 hkv=int(r["hkv"]), tile=64,
                                 requested=SMS_H100 * (2 if dtype == "fp16" else 3),
                                 ctas=int(r["ctas"]), segments=int(r["segments"])))
    # h100_ctas.csv has no header; rows come in groups of 5 per (dtype, shape):
    # requested = sms/2, sms, 2*sms, 3*sms, wave (= 3*sms on H100).
    order = [SMS_H100 // 2, SMS_H100, 2 * SMS_H100, 3 * SMS_H100, 3 * SMS_H100]
    with open(ref / "results" / "h100_ctas.csv") as f:
        raw = [line.strip().split(",") for line in f if line.strip()]
    for i, r in enumerate(raw):
        rows.append(dict(source="h100_ctas.csv", dtype=r[1], batch=int(r[2]), seq_len=int(r[3]),
                         hkv=int(r[5]), tile=64, requested=order[i % 5], ctas=int(r[8]),
                         segments=int(r[9])))
    return rows


def accuracy_rows(ref: pathlib.Path) -> list[dict]:
    keep = ("dtype", "batch", "seq_len", "max_abs_diff_vs_ref", "fp8_err_vs_fp16", "fp8_rel_err_vs_fp16")
    with open(ref / "results" / "h100_flashinfer.csv") as f:
        return [{k: r[k] for k in keep} for r in csv.DictReader(f)]


def write_accuracy_rows(ref: pathlib.Path) -> None:
    rows = accuracy_rows(ref)
    with open(HERE / "accuracy_rows.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        w.writeheader()
        w.writerows(rows)
    print(f"accuracy_rows.csv: {len(rows)} rows")


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    ref = pathlib.Path(args.reference)

    rows = planner_rows(ref)
    with open(HERE / "planner_rows.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0].keys()))
        w.writeheader()
        w.writerows(rows)
    print(f"planner_rows.csv: {len(rows)} rows")

    (HERE / "capacity_rows.csv").write_text((ref / "results" / "h100_capacity.csv").read_text())
    print("capacity_rows.csv written")
    write_accuracy_rows(ref)

    import torch

    codes = torch.arange(256, dtype=torch.uint8)
    values = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    np.save(HERE / "e4m3_decode.npy", values)

    rng = np.random.default_rng(20261201)
    finite = values[np.isfinite(values)]
    grid = np.unique(np.abs(finite))
    mids = (grid[1:] + grid[:-1]) / 2                     # exact ties
    near = np.concatenate([mids * (1 + 2.0 ** -20), mids * (1 - 2.0 ** -20)])
    samples = np.concatenate([
        grid, mids, near,
        rng.normal(0, 1, 4000), rng.normal(0, 50, 4000), rng.uniform(-463.9, 463.9, 4000),
        rng.uniform(-2 ** -6, 2 ** -6, 2000), 2.0 ** rng.uniform(-14, 8.85, 2000),
    ]).astype(np.float32)
    samples = np.concatenate([samples, -samples])
    samples = samples[np.abs(samples) < 464]
    enc = torch.from_numpy(samples).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.savez_compressed(HERE / "e4m3_encode.npz", x=samples, code=enc)
    print(f"e4m3 fixtures: 256 codes, {len(samples)} encode vectors")


if __name__ == "__main__":
    main()
