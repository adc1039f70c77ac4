"""Decode-step benchmark of the MI355X paged flash-decoding path (one JSON line).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]
                    [--page-size P] [--ctas N] [--no-cpu] [--no-cold] [--no-copy]

One step is one decode of one Llama-3-8B attention layer (Hq=32, Hkv=8,
head_dim=128) over a paged KV cache: the split-KV decode kernel (which merges
split rows itself when they span at most 8 blocks) plus the LSE merge kernel
where a row spans more, with the plan built once outside the timed region (the
reference's bench/bench_decode.cu:198-209). Inputs are synthetic and already
resident in HBM: q/K/V ~ N(0,1) rounded to fp16, appended through the product's
own append(-quantize) kernel into pages scattered by a seeded shuffle of the
free list (bench_decode.cu:149-176); FP8 uses per-tensor amax/448 scales.

Fields of the JSON line:
  value        algorithmic HBM GB/s of the whole step over the K timed steps,
               run back to back (bytes = 2*sum(L)*Hkv*D*e + 2*B*Hq*D*2 +
               sum(ceil(L/P))*4, bench_decode.cu:186-191)
  roofline     the split kernel's algorithmic GB/s against 8 TB/s. Its
               average duration comes from two HIP events bracketing the timed
               steps on the kernels' stream when a step is the split kernel
               alone (C2, C3), else from HIP events around each of K further
               split launches (both figures are reported)
  cold         the reference's method: a 1 GiB flush before each run, HIP
               events around decode + merge, median of --cold-iters
  copy_ceiling best plain streaming read of 4 GiB (bench_decode.cu:224-240,
               unrolled / non-temporal variants of it, and the chunked read
               with one contiguous span per wave), and the chunked read of
               the workload's own byte count; measured before the timed steps
               (its ~25 ms of HBM load settle the GPU's clocks, which five
               warm-up steps alone do not: C2 162-163 us against 157-159 us
               per step)
  workloads    the same figures (step, split kernel, cold) for C1, C3 (the
               FP8 target), C2 at 16-token pages and at one page per
               sequence, C2 at 16-token pages in memory order (free list
               not shuffled), the ragged C4, C5 fp16 and FP8,
               timed in the same run (each over max(K, 100) steps after
               max(W, 20) warm-ups); paging_overhead = C2 at 16-token pages
               against one page per sequence (memory_order_*: the same with
               the pages in memory order); targets = the goals the
               north star states, checked on these figures
  cpu_baseline the reference's cpu_attention (compiled from its source into
               oracle/_ref when that exists, else the oracle's restatement)
               over every (row, query head) pair of the same workload, K/V
               gathered and dequantized to fp32 beforehand (untimed), on
               OMP_NUM_THREADS threads (the CPU share of one GPU on the GPU
               boxes) or every host core; cpu_baseline.c1 times C1 (the
               reference's CPU-runnable configuration) every run
  roofline.traffic  HBM bytes per split-kernel launch from two rocprofv3
               counter passes run as child processes before this process
               touches the GPU (FETCH_SIZE, then WRITE_SIZE, in KiB per
               dispatch), each scaled by what the same counter reads for a
               read kernel and a write kernel of known size in the same run

Multi-GPU runs are not part of this build: --gpus > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import statistics
import subprocess
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (ROOT, ROOT / "paged-attention_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import numpy as np  # noqa: E402

HQ, HKV, D = 32, 8, 128
PEAK_GBPS = 8000.0   # MI355X HBM3E published peak
METRIC = "HBM GB/s & % of peak; µs/decode step (Llama-3-8B layer, fp16/FP8 KV)"

CONFIGS = {
    # name: (description, batch, "ragged" or None, seq_len, fp8)
    "c1": ("C1: 4 x 1024, fp16 KV, 16-token scattered pages", 4, None, 1024, False),
    "c2": ("C2: 32 x 8192, fp16 KV, 16-token scattered pages", 32, None, 8192, False),
    "c3": ("C3: 64 x 8192, FP8 E4M3 KV (amax/448), 16-token scattered pages", 64, None, 8192, True),
    "c4": ("C4: 128 ragged sequences L~U[128,16384] (seed 4), fp16 KV, 16-token scattered pages",
           128, "ragged", 0, False),
    "c5": ("C5: 1 x 131072, fp16 KV, 16-token scattered pages", 1, None, 131072, False),
    "c5fp8": ("C5: 1 x 131072, FP8 E4M3 KV (amax/448), 16-token scattered pages", 1, None, 131072, True),
}


def seq_lens_of(name: str) -> list[int]:
    _, batch, kind, length, _ = CONFIGS[name]
    if kind == "ragged":
        rng = np.random.default_rng(4)
        return [int(x) for x in rng.integers(128, 16385, size=batch)]
    return [length] * batch


def _d2h(ptr: int, nbytes: int) -> np.ndarray:
    """Device bytes at ptr -> new host array (synchronous hipMemcpy)."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    out = np.empty(nbytes, dtype=np.uint8)
    if hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) != 0:   # hipMemcpyDeviceToHost
        raise RuntimeError("hipMemcpy D2H failed")
    return out


def host_fp32_items(s):
    """Every (row, kv head) item gathered through the block table and
    dequantized to fp32 [L][D] (tests/test_paged_decode.cu:28-31 `stored`),
    plus q as fp32: the CPU baseline's untimed preparation."""
    import oracle
    p = s.params
    eb = 1 if s.fp8 else 2
    shape = (s.num_pages, HKV, s.page, D)
    kraw = _d2h(p.k_cache, s.num_pages * HKV * s.page * D * eb)
    vraw = _d2h(p.v_cache, s.num_pages * HKV * s.page * D * eb)
    if s.fp8:
        lut = oracle.e4m3_to_f32(np.arange(256, dtype=np.uint8))
        kp, vp = kraw.reshape(shape), vraw.reshape(shape)
        conv_k = lambda x: lut[x] * np.float32(s.k_scale)   # noqa: E731
        conv_v = lambda x: lut[x] * np.float32(s.v_scale)   # noqa: E731
    else:
        kp, vp = kraw.view(np.float16).reshape(shape), vraw.view(np.float16).reshape(shape)
        conv_k = conv_v = lambda x: x.astype(np.float32)   # noqa: E731
    K, V = [], []
    for b, L in enumerate(s.lens):
        row = s.cache.block_table(b)
        for h in range(HKV):
            K.append(np.ascontiguousarray(conv_k(kp[row, h].reshape(-1, D)[:L])))
            V.append(np.ascontiguousarray(conv_v(vp[row, h].reshape(-1, D)[:L])))
    return s.q.float().cpu().numpy(), K, V


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads(requested: int) -> tuple[int, str]:
    """Threads for the CPU baseline and why: an explicit --cpu-threads, else
    OMP_NUM_THREADS (16 on the GPU boxes, the CPU share one GPU is given there,
    whatever nproc shows), else every core nproc reports."""
    nproc = os.cpu_count() or 1
    if requested > 0:
        return requested, "--cpu-threads"
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        return min(int(omp), nproc), "OMP_NUM_THREADS (the host's CPU share for this GPU)"
    return nproc, "nproc (all host cores)"


def cpu_time(s, budget_s: float, threads: int, max_runs: int = 3) -> tuple[float, int, bool]:
    """Median seconds of the CPU attention over every (row, query head) pair
    of the Setup's workload (K/V gathered and dequantized beforehand, untimed),
    the number of runs, and whether the reference's compiled cpu_attention ran."""
    import oracle
    q, K, V = host_fp32_items(s)
    use_ref = oracle.ref_lib() is not None
    times = []
    t0 = time.perf_counter()
    while True:
        _, secs = oracle.attention_pairs(q, K, V, s.lens, HKV, threads=threads, use_reference=use_ref)
        times.append(secs)
        spent = time.perf_counter() - t0
        if len(times) >= max_runs or spent + secs > budget_s:
            break
    return statistics.median(times), len(times), use_ref


def cpu_baseline(s, name: str, budget_s: float, threads: int, why: str, c1=None, c1_gpu_us=None) -> dict:
    med, runs, use_ref = cpu_time(s, budget_s, threads)
    out = {
        "value": round(s.bytes() / med / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(med * 1e6, 1),
        "cores": threads,
        "cores_source": why,
        "nproc": os.cpu_count(),
        "cpu_model": cpu_model(),
        "kind": "reference" if use_ref else "port",
        "sample": (f"all {s.batch * HQ} (row, query head) pairs of {name} ({s.batch} x {max(s.lens)} tokens), "
                   f"{runs} run(s), median; K/V gathered and dequantized to fp32 beforehand (untimed)"),
    }
    if c1 is not None:
        # The reference's CPU-runnable configuration, timed every run beside
        # the GPU's step on the same inputs.
        med1, runs1, _ = cpu_time(c1, budget_s, threads, max_runs=20)
        out["c1"] = {"workload": CONFIGS["c1"][0], "us_per_step": round(med1 * 1e6, 1), "runs": runs1,
                     "gpu_us_per_step": c1_gpu_us,
                     "gpu_speedup": round(med1 * 1e6 / c1_gpu_us, 1) if c1_gpu_us else None}
    return out


def warm_clocks(bd, reads: int = 160):
    """The copy ceiling's reads also bring the GPU's clocks to their loaded
    state before the timed steps; without them (--no-copy) the same sustained
    load comes from `reads` streaming reads of one 1 GiB buffer (about 25 ms).
    Returns the buffer's Flusher, kept (and reused for the cold runs): a
    timing right after a large free runs slow."""
    import torch
    fl = bd.Flusher()
    stream = torch.cuda.current_stream()
    for _ in range(reads):
        fl.flush(stream)
    torch.cuda.synchronize()
    return fl


def time_steps(s, steps: int, warmup: int):
    """W untimed steps, then K timed steps back to back (wall clock between
    synchronizations: the `value`; two HIP events on the kernels' stream also
    bracket the timed region), then K more split launches with HIP events
    around each one on the same stream (the kernel's average launch duration
    for the roofline; events between steps would stretch the timed steps)."""
    import torch
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    for _ in range(warmup):
        s.split(sh)
        s.merge(sh)
    _barrier()
    torch.cuda.synchronize()
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    r0.record(stream)
    for _ in range(steps):
        s.split(sh)
        s.merge(sh)
    r1.record(stream)
    torch.cuda.synchronize()
    _barrier()
    wall = time.perf_counter() - t0
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        a.record(stream)
        s.split(sh)
        b.record(stream)
        s.merge(sh)
    torch.cuda.synchronize()
    return wall, [a.elapsed_time(b) for a, b in ev], r0.elapsed_time(r1)


CALIB_BYTES = 1 << 30   # size of the counter-calibration read and write kernels


def pmc_child(args) -> None:
    """Runs under rocprofv3 --pmc: a read and a write of CALIB_BYTES each (the
    counters' calibration), then a few decode steps of the workload."""
    import torch
    from pa_amd import bench_decode as bd
    import pa_amd
    torch.cuda.set_device(0)
    pa_amd._lib.load()
    desc, _, _, _, fp8 = CONFIGS[args.config]
    s = bd.Setup(seq_lens_of(args.config), HQ, HKV, D, args.page_size, fp8, shuffle=True, ctas=args.ctas)
    buf = torch.empty(CALIB_BYTES, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    pa_amd.fill_bytes(buf, CALIB_BYTES, 1)
    pa_amd.stream_read(buf, CALIB_BYTES, 2048, sink, threads=256, unroll=8, nontemporal=True)
    sh = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        s.split(sh)
        s.merge(sh)
    torch.cuda.synchronize()
    s.close()


def measure_traffic(args) -> dict | None:
    """Two rocprofv3 counter passes over pmc_child; returns the split kernel's
    HBM bytes per launch (read, written, total) and the calibration factors,
    or None if the profiler is unavailable or a pass fails."""
    import csv
    import shutil
    import tempfile
    if profiler_preloaded():
        print("# traffic passes skipped: this process runs under a profiler", file=sys.stderr, flush=True)
        return None
    prof = shutil.which("rocprofv3")
    if not prof:
        return None
    out = {}
    with tempfile.TemporaryDirectory(prefix="pa_pmc_") as tmp:
        for counter, calib in (("FETCH_SIZE", "stream_read_kernel"), ("WRITE_SIZE", "fill_bytes_kernel")):
            d = pathlib.Path(tmp) / counter
            cmd = [prof, "--pmc", counter, "-d", str(d), "-o", "run", "--output-format", "csv", "--",
                   sys.executable, str(ROOT / "bench.py"), "--pmc-child", "--config", args.config,
                   "--page-size", str(args.page_size), "--ctas", str(args.ctas)]
            print(f"# traffic pass: {counter}", file=sys.stderr, flush=True)
            try:
                subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=180, check=False)
            except subprocess.TimeoutExpired:
                return None
            files = list(d.rglob("*counter_collection.csv"))
            if not files:
                return None
            split, cal = [], []
            with open(files[0]) as f:
                for r in csv.DictReader(f):
                    if r.get("Counter_Name") != counter:
                        continue
                    if "decode_split_kernel" in r["Kernel_Name"]:
                        split.append(float(r["Counter_Value"]))
                    elif calib in r["Kernel_Name"]:
                        cal.append(float(r["Counter_Value"]))
            if not split or not cal or cal[0] <= 0:
                return None
            factor = CALIB_BYTES / (statistics.mean(cal) * 1024.0)   # true bytes per counted byte
            out[counter] = {"kib_per_dispatch": statistics.mean(split), "factor": factor,
                            "bytes": statistics.mean(split) * 1024.0 * factor}
    return out


def profiler_preloaded(env=None) -> bool:
    """True when this process runs under a profiler's preloaded library
    (rocprofv3 sets LD_PRELOAD and ROCPROF_* variables). A child process would
    inherit the preload, which initializes the GPU before the child's own
    program starts; `rocprofv3` is itself a `#!/usr/bin/env python3` script, so
    starting one from here would make a GPU-initialized process exec. bench.py
    therefore starts no child process at all in that case."""
    env = os.environ if env is None else env
    if "rocprof" in env.get("LD_PRELOAD", "").lower():
        return True
    return any(k.startswith(("ROCPROF_", "ROCPROFILER_")) for k in env)


# hipDeviceAttribute_t values (hip/hip_runtime_api.h): global memory bus width
# in bits and peak memory clock in kHz.
_HIP_ATTR_MEMORY_BUS_WIDTH = 59
_HIP_ATTR_MEMORY_CLOCK_RATE = 60


def device_report(dev: int = 0) -> dict:
    """The device's own figures from the HIP runtime in this process (no child
    process): name, ISA, compute units and HBM size from hipGetDeviceProperties,
    and the DRAM peak the device reports, memory clock x bus width x 2 (double
    data rate), derived as bench_decode.cu:87-100 derives it. The line carries
    that reported peak beside the published 8 TB/s it is priced against."""
    try:
        import torch
        if not torch.cuda.is_available():
            return {"source": "no HIP device"}
        props = torch.cuda.get_device_properties(dev)
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        hip.hipDeviceGetAttribute.restype = ctypes.c_int

        def attr(a: int) -> int:
            v = ctypes.c_int(0)
            return v.value if hip.hipDeviceGetAttribute(ctypes.byref(v), a, dev) == 0 else 0

        clock_khz, bus_bits = attr(_HIP_ATTR_MEMORY_CLOCK_RATE), attr(_HIP_ATTR_MEMORY_BUS_WIDTH)
        arch = props.gcnArchName.split(":")[0]
        # The runtime's name is generic on these boxes (the marketing name needs
        # libdrm's id table): the ISA name and PCI device id stand in for it.
        name = props.name if props.name and props.name != "AMD Radeon Graphics" else f"AMD {arch}"
        return {"name": name, "arch": arch, "pci_device_id": f"0x{props.pci_device_id:04x}",
                "cus": props.multi_processor_count, "hbm_bytes": int(props.total_memory),
                "memory_clock_khz": clock_khz, "memory_bus_bits": bus_bits,
                # bench_decode.cu:87-100's formula. HBM3E moves 8 Gb/s per pin
                # (8192 bits x 8 Gb/s / 8 = 8.2 TB/s, the published 8 TB/s), while
                # the runtime reports a 2 GHz memory clock, so on MI355X the
                # formula gives half of that.
                "formula_peak_gbps": round(2.0 * clock_khz * 1e3 * bus_bits / 8 / 1e9, 1),
                "formula_note": "2 x memory clock x bus width (bench_decode.cu:87-100); the runtime's memory "
                                "clock understates HBM3E's 8 Gb/s per pin, so peak_gbps stays the published "
                                f"{PEAK_GBPS:.0f} GB/s",
                "source": "HIP runtime (hipGetDeviceProperties, hipDeviceGetAttribute)"}
    except (OSError, RuntimeError, AttributeError, ValueError) as e:
        return {"source": f"HIP device query failed ({type(e).__name__})"}


# Workloads timed beside the headline one (their figures go under
# "workloads"): the CPU-runnable C1, the FP8 target C3, both ends of C2's
# page-size comparison (paging overhead = C2 at 16-token pages against one
# page per sequence, both timed the same way), C2's 16-token pages in memory
# order (the pool's free list not shuffled: what the placement, not the paging,
# costs), the ragged C4 and C5 in both dtypes.
# (key, config, page size, shuffled free list)
EXTRA = [("c1", "c1", 16, True), ("c3", "c3", 16, True), ("c2_p16", "c2", 16, True), ("c2_p8192", "c2", 8192, True),
         ("c2_p16_memory_order", "c2", 16, False), ("c4", "c4", 16, True), ("c5", "c5", 16, True),
         ("c5fp8", "c5fp8", 16, True)]


MERGE_NAMES = {0: "merge kernel", 1: "in the split kernel, inside one block",
               2: "in the split kernel, across blocks"}


def merge_of(s) -> str:
    """How the plan's split rows are merged (pa_decode_params.block_merge)."""
    if s.params.needs_merge == 0 and s.params.block_merge == 0:
        return "none (no split rows)"
    return MERGE_NAMES.get(int(s.params.block_merge), "?")


def workload_figures(s, desc: str, steps: int, warmup: int, cold_iters: int, flusher) -> dict:
    """One workload's step (K back-to-back steps), split-kernel and cold figures."""
    wall, split_ms, region_ms = time_steps(s, steps, warmup)
    nbytes = s.bytes()
    step_us = wall * 1e6 / steps
    split_us = (region_ms / steps if s.params.needs_merge == 0 else statistics.mean(split_ms)) * 1e3
    out = {"workload": desc, "page_size": s.page, "units": s.plan.num_ctas, "segments": int(len(s.plan.segments)),
           "merge": merge_of(s), "algorithmic_bytes": nbytes,
           "us_per_step": round(step_us, 2), "pct_of_peak": round(100 * nbytes / (step_us * 1e-6) / 1e9 / PEAK_GBPS, 2),
           "split_us": round(split_us, 2),
           "split_pct_of_peak": round(100 * nbytes / (split_us * 1e-6) / 1e9 / PEAK_GBPS, 2)}
    if flusher is not None:
        from pa_amd import bench_decode as bd
        med = statistics.median(bd.time_cold(flusher, cold_iters, s.run))
        out["cold_us"] = round(med * 1e3, 2)
        out["cold_pct_of_peak"] = round(100 * nbytes / (med * 1e-3) / 1e9 / PEAK_GBPS, 2)
    return out


def _barrier() -> None:
    import torch.distributed as dist
    if dist.is_available() and dist.is_initialized():
        dist.barrier()


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--page-size", type=int, default=16)
    ap.add_argument("--ctas", type=int, default=0, help="work units of the plan (0 = one full wave)")
    ap.add_argument("--cold-iters", type=int, default=50)
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU-baseline work")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0 = OMP_NUM_THREADS if set (the box's CPU share), else every host core")
    ap.add_argument("--no-extra", action="store_true", help="time only the headline workload")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-cold", action="store_true")
    ap.add_argument("--no-copy", action="store_true",
                    help="skip the copy ceiling (its reads are replaced by a 25 ms clock warm-up)")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()

    if args.pmc_child:
        pmc_child(args)
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs (--gpus > 1) are not part of it",
              file=sys.stderr)
        sys.exit(2)

    # The counter passes (child processes) run before this process initializes
    # the GPU, and not at all under a profiler.
    traffic = None if args.no_traffic else measure_traffic(args)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: needs a GPU (cuda:0)", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    device = device_report(0)
    from pa_amd import bench_decode as bd
    import pa_amd
    pa_amd._lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count

    desc, _, _, _, fp8 = CONFIGS[args.config]
    print(f"# bench: {desc}, page_size {args.page_size}", file=sys.stderr, flush=True)
    s = bd.Setup(seq_lens_of(args.config), HQ, HKV, D, args.page_size, fp8, shuffle=True, ctas=args.ctas)
    print(f"# setup done: {s.batch} seqs, {s.num_pages} pages, plan {s.plan.num_ctas} units / "
          f"{len(s.plan.segments)} segments", file=sys.stderr, flush=True)

    nbytes = s.bytes()
    # The copy ceiling runs first: ~40 reads of 4 GiB (about 25 ms of sustained
    # HBM load) bring the GPU's clocks to their loaded state, which the W
    # warm-up steps alone (0.8 ms at W = 5) do not.
    copy_ceiling = None
    warm = None
    if not args.no_copy:
        rows = bd.copy_rows(cus)
        best = max(rows, key=lambda r: r["gbps"])
        ref_rows = [r for r in rows if r["kernel"].endswith("x512_u1")]
        copy_ceiling = {
            "gbps": round(best["gbps"], 1), "frac": round(best["gbps"] / PEAK_GBPS, 4), "kernel": best["kernel"],
            "reference_read_gbps": round(max(r["gbps"] for r in ref_rows), 1), "bytes": best["bytes"]}
        same = bd.chunked_read_same_bytes(cus, nbytes)
        if same:
            copy_ceiling["same_size"] = {
                "bytes": same["bytes"], "gbps": round(same["gbps"], 1), "frac": round(same["gbps"] / PEAK_GBPS, 4),
                "kernel": same["kernel"], "time_us": round(same["time_us"], 2)}
    else:
        warm = warm_clocks(bd)

    wall, split_ms, region_ms = time_steps(s, args.steps, args.warmup)
    ms_per_step = wall * 1e3 / args.steps
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    # The split kernel's average duration: from the two events around the timed
    # steps when a step is that kernel alone (no merge launch), else from the
    # events around each of the K further split launches.
    region_avg = region_ms / args.steps
    only_split = s.params.needs_merge == 0
    split_avg = region_avg if only_split else statistics.mean(split_ms)
    achieved = nbytes / (split_avg * 1e-3) / 1e9
    print(f"# timed {args.steps} steps: {ms_per_step * 1e3:.1f} us/step, split kernel {split_avg * 1e3:.1f} us avg",
          file=sys.stderr, flush=True)

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "pct_of_peak": round(100 * value / PEAK_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: q/K/V ~ N(0,1) fp16, appended into seeded scattered pages" +
                (", FP8 E4M3 at amax/448" if fp8 else ""),
        "config": {
            "workload": desc,
            "batch": s.batch,
            "seq_len": max(s.lens),
            "total_tokens": sum(s.lens),
            "num_q_heads": HQ,
            "num_kv_heads": HKV,
            "head_dim": D,
            "page_size": args.page_size,
            "kv_dtype": "fp8_e4m3" if fp8 else "fp16",
            "units": s.plan.num_ctas,
            "segments": int(len(s.plan.segments)),
            "merge": merge_of(s),
            "algorithmic_bytes": nbytes,
        },
        "roofline": {
            "kernel": "decode_split_kernel",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBPS, 4),
            "traffic": None,
            "avg_us": round(split_avg * 1e3, 2),
            "avg_source": "timed-region events" if only_split else "per-launch events",
            # HIP events bracketing the K timed steps on the kernels' stream:
            # split + merge (if any) per step, launch gaps included.
            "timed_region_avg_us": round(region_avg * 1e3, 2),
            "per_launch_avg_us": round(statistics.mean(split_ms) * 1e3, 2),
        },
    }
    if traffic:
        rd, wr = traffic["FETCH_SIZE"], traffic["WRITE_SIZE"]
        result["roofline"]["traffic"] = int(rd["bytes"] + wr["bytes"])
        result["roofline"]["traffic_detail"] = {
            "read_bytes": int(rd["bytes"]), "write_bytes": int(wr["bytes"]),
            "fetch_kib_per_dispatch": round(rd["kib_per_dispatch"], 1),
            "write_kib_per_dispatch": round(wr["kib_per_dispatch"], 1),
            "fetch_factor": round(rd["factor"], 4), "write_factor": round(wr["factor"], 4),
            "vs_algorithmic": round((rd["bytes"] + wr["bytes"]) / nbytes, 4)}

    if copy_ceiling is not None:
        result["copy_ceiling"] = copy_ceiling
    fl = None if args.no_cold else (warm or bd.Flusher())
    if fl is not None:
        cold = bd.time_cold(fl, args.cold_iters, s.run)
        med = statistics.median(cold)
        result["cold"] = {"us_median": round(med * 1e3, 2), "gbps": round(nbytes / (med * 1e-3) / 1e9, 1),
                          "frac": round(nbytes / (med * 1e-3) / 1e9 / PEAK_GBPS, 4),
                          "iters": args.cold_iters, "flush_bytes": fl.buf.numel()}

    # Every setup stays allocated until the end: a timing taken right after a
    # large free runs a few percent slow while the memory is released.
    kept = {}
    if not args.no_extra:
        result["workloads"] = {}
        headline = (args.config, args.page_size)
        for key, cfg, page, shuffled in EXTRA:
            if (cfg, page) == headline and shuffled and key != "c2_p16":
                continue
            head = f"{CONFIGS[cfg][0].split(',')[0]}, {CONFIGS[cfg][0].split(', ')[1]}"
            d = (CONFIGS[cfg][0] if page == 16 and shuffled else
                 f"{head}, 16-token pages in memory order (free list not shuffled)" if page == 16 else
                 f"{head}, {page}-token pages (one page per sequence)")
            print(f"# workload {key}: {d}", file=sys.stderr, flush=True)
            kept[key] = bd.Setup(seq_lens_of(cfg), HQ, HKV, D, page, CONFIGS[cfg][4], shuffle=shuffled, ctas=args.ctas)
            # Each is timed over at least 100 steps after 20 warm-ups (K and W
            # count the headline's steps; a short window reads a few percent
            # slow while a new workload's first launches settle).
            result["workloads"][key] = workload_figures(kept[key], d, max(args.steps, 100), max(args.warmup, 20),
                                                        min(args.cold_iters, 20), fl)
        w = result["workloads"]
        if "c2_p16" in w and "c2_p8192" in w:
            a, c = w["c2_p16"], w["c2_p8192"]
            result["paging_overhead"] = {
                "page_size": 16, "against_page_size": 8192,
                "step_pct": round(100 * (a["us_per_step"] / c["us_per_step"] - 1), 2),
                "split_pct": round(100 * (a["split_us"] / c["split_us"] - 1), 2),
                "cold_pct": (round(100 * (a["cold_us"] / c["cold_us"] - 1), 2)
                             if "cold_us" in a and "cold_us" in c else None)}
            if "c2_p16_memory_order" in w:
                m = w["c2_p16_memory_order"]
                # The same 16-token paging with the pages in memory order: the
                # gap to the shuffled pool is what the random placement costs.
                result["paging_overhead"]["memory_order_step_pct"] = round(
                    100 * (m["us_per_step"] / c["us_per_step"] - 1), 2)
                result["paging_overhead"]["memory_order_cold_pct"] = (
                    round(100 * (m["cold_us"] / c["cold_us"] - 1), 2) if "cold_us" in m and "cold_us" in c else None)
        if args.config == "c2" and args.page_size == 16:
            result["targets"] = {
                "c2_fp16_step_ge_80pct": result["pct_of_peak"] >= 80.0,
                "c3_fp8_step_ge_75pct": w["c3"]["pct_of_peak"] >= 75.0 if "c3" in w else None,
                "paging_overhead_step_lt_2pct": (result["paging_overhead"]["step_pct"] < 2.0
                                                 if "paging_overhead" in result else None)}
    if not args.no_cpu:
        threads, why = cpu_threads(args.cpu_threads)
        c1 = kept.get("c1")
        c1_gpu = result["workloads"]["c1"]["us_per_step"] if c1 is not None else None
        result["cpu_baseline"] = cpu_baseline(s, args.config, args.cpu_budget, threads, why, c1, c1_gpu)

    result["device"] = device
    for k in kept.values():
        k.close()
    s.close()
    del fl
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
