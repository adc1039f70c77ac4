"""Decode-step benchmark of the MI355X paged flash-decoding path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]
                    [--page-size P] [--no-cpu] [--no-cold] [--no-copy]

One step is one decode of one Llama-3-8B attention layer (Hq=32, Hkv=8,
head_dim=128) over a paged KV cache: the split-KV decode kernel plus the LSE
merge kernel, with the plan built once outside the timed region
(bench/bench_decode.cu:198-209 of the reference). Inputs are synthetic and
already resident in HBM: q/K/V ~ N(0,1) rounded to fp16, appended through the
product's own append(-quantize) kernel into pages scattered by a seeded
shuffle of the free list (bench_decode.cu:149-176), FP8 with per-tensor
amax/448 scales.

Printed JSON line (rank 0, one line):
  value        algorithmic HBM GB/s of the whole step over the K timed steps
               (bytes = 2*sum(L)*Hkv*D*e + 2*B*Hq*D*2 + sum(ceil(L/P))*4,
               bench_decode.cu:186-191), steps back to back
  roofline     the split kernel's algorithmic GB/s from HIP events around each
               of its launches in the timed loop, against 8 TB/s
  cold         the reference's method: >= 1 GiB cache flush before each run,
               HIP events around decode+merge, median of --cold-iters
  copy_ceiling plain 16 B/lane streaming read of 4 GiB (bench_decode.cu:224-240)
  cpu_baseline the reference's cpu_attention (compiled from its source into
               oracle/_ref when available, else the oracle's restatement) over
               every (row, query head) pair of the same workload, dequantized to
               fp32 beforehand (untimed), on the host's cores

Multi-GPU runs are not part of this build: --gpus > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import statistics
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
    # name: (description, batch, lens (None = uniform), seq_len, fp8)
    "c1": ("C1: 4 x 1024, fp16 KV, 16-token scattered pages", 4, None, 1024, False),
    "c2": ("C2: 32 x 8192, fp16 KV, 16-token scattered pages", 32, None, 8192, False),
    "c3": ("C3: 64 x 8192, FP8 E4M3 KV (amax/448), 16-token scattered pages", 64, None, 8192, True),
    "c4": ("C4: 128 ragged sequences L~U[128,16384] (seed 4), fp16 KV, 16-token scattered pages",
           128, "ragged", 0, False),
    "c5": ("C5: 1 x 131072, fp16 KV, 16-token scattered pages", 1, None, 131072, False),
    "c5fp8": ("C5: 1 x 131072, FP8 E4M3 KV, 16-token scattered pages", 1, None, 131072, True),
}


def seq_lens_of(name: str) -> list[int]:
    _, batch, kind, L, _ = CONFIGS[name]
    if kind == "ragged":
        rng = np.random.default_rng(4)
        return [int(x) for x in rng.integers(128, 16385, size=batch)]
    return [L] * batch


def algorithmic_bytes(lens, page_size: int, fp8: bool) -> int:
    """bench_decode.cu:186-191: K and V once, q in and out once, the table."""
    e = 1 if fp8 else 2
    return (2 * sum(lens) * HKV * D * e + 2 * len(lens) * HQ * D * 2
            + sum(math.ceil(L / page_size) for L in lens) * 4)


class Workload:
    """A filled PagedKVCache plus a bound plan for one configuration."""

    def __init__(self, name: str, page_size: int, seed: int = 42):
        import torch
        import pa_amd

        self.name = name
        desc, batch, _, _, fp8 = CONFIGS[name]
        self.desc = desc
        self.fp8 = fp8
        self.lens = seq_lens_of(name)
        self.page_size = page_size
        self.batch = len(self.lens)
        self.dtype = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
        pages = [math.ceil(L / page_size) for L in self.lens]
        self.num_pages = sum(pages)
        g = torch.Generator(device="cuda").manual_seed(seed)
        # K/V of every sequence, N(0,1) fp16; FP8 scales are amax/448 over all of K (V).
        srcs = [(torch.randn(L, HKV, D, device="cuda", dtype=torch.float16, generator=g),
                 torch.randn(L, HKV, D, device="cuda", dtype=torch.float16, generator=g)) for L in self.lens]
        if fp8:
            self.k_scale = max(float(k.abs().max()) for k, _ in srcs) / 448.0
            self.v_scale = max(float(v.abs().max()) for _, v in srcs) / 448.0
        else:
            self.k_scale = self.v_scale = 1.0
        self.cache = pa_amd.PagedKVCache(self.num_pages, page_size, HKV, D, self.batch, max(pages), self.dtype,
                                         self.k_scale, self.v_scale)
        self.cache.shuffle_free_pages(seed)
        stream = torch.cuda.current_stream()
        for b, (k, v) in enumerate(srcs):
            assert self.cache.admit() == b
            assert self.cache.append(b, k, v, self.lens[b], stream)
        del srcs
        self.q = torch.randn(self.batch, HQ, D, device="cuda", dtype=torch.float16, generator=g)
        self.out = torch.empty_like(self.q)
        self.plan = pa_amd.make_plan(self.dtype, self.lens, HQ, HKV, D, 0)
        self.dplan = pa_amd.DevicePlan()
        self.dplan.upload(self.plan, HQ // HKV, D, stream)
        p = self.cache.params()
        p.q = self.q.data_ptr()
        p.out = self.out.data_ptr()
        p.slot_ids = None              # slots 0..B-1 are rows 0..B-1
        p.batch = self.batch
        p.num_q_heads = HQ
        self.dplan.bind(p)
        self.params = p
        self.bytes = algorithmic_bytes(self.lens, page_size, fp8)
        torch.cuda.synchronize()

    def split(self, stream_handle: int) -> None:
        from pa_amd import _lib
        _lib.check(self._lib.pa_decode_split(self.dtype, self._pref, stream_handle))

    def merge(self, stream_handle: int) -> None:
        from pa_amd import _lib
        _lib.check(self._lib.pa_decode_merge(self.dtype, self._pref, stream_handle))

    def bind_fast(self) -> None:
        import ctypes

        from pa_amd import _lib
        self._lib = _lib.load()
        self._pref = ctypes.byref(self.params)

    def host_fp32_items(self):
        """Gathers and dequantizes every (row, kv head) item to fp32 [L][D]
        (the CPU baseline's untimed preparation), plus q as fp32."""
        import oracle
        p = self.params
        eb = 1 if self.fp8 else 2
        nbytes = self.num_pages * HKV * self.page_size * D * eb
        shape = (self.num_pages, HKV, self.page_size, D)
        kraw = _d2h(p.k_cache, nbytes)
        vraw = _d2h(p.v_cache, nbytes)
        if self.fp8:
            lut = oracle.e4m3_to_f32(np.arange(256, dtype=np.uint8))
            kp, vp = kraw.reshape(shape), vraw.reshape(shape)
            conv_k = lambda x: lut[x] * np.float32(self.k_scale)   # noqa: E731
            conv_v = lambda x: lut[x] * np.float32(self.v_scale)   # noqa: E731
        else:
            kp, vp = kraw.view(np.float16).reshape(shape), vraw.view(np.float16).reshape(shape)
            conv_k = conv_v = lambda x: x.astype(np.float32)   # noqa: E731
        K, V = [], []
        for b, L in enumerate(self.lens):
            row = self.cache.block_table(b)
            for h in range(HKV):
                K.append(np.ascontiguousarray(conv_k(kp[row, h].reshape(-1, D)[:L])))
                V.append(np.ascontiguousarray(conv_v(vp[row, h].reshape(-1, D)[:L])))
        q = self.q.float().cpu().numpy()
        return q, K, V

    def close(self) -> None:
        self.cache.close()


def _d2h(ptr: int, nbytes: int) -> np.ndarray:
    """Device bytes at ptr -> new host array (synchronous hipMemcpy)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    out = np.empty(nbytes, dtype=np.uint8)
    if hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) != 0:   # hipMemcpyDeviceToHost
        raise RuntimeError("hipMemcpy D2H failed")
    return out


def time_steps(w: Workload, steps: int, warmup: int):
    """W untimed steps, then K timed steps with HIP events around each split
    launch (on the stream the kernels run on)."""
    import torch
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    for _ in range(warmup):
        w.split(sh)
        w.merge(sh)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    _barrier()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in ev:
        a.record(stream)
        w.split(sh)
        b.record(stream)
        w.merge(sh)
    torch.cuda.synchronize()
    _barrier()
    wall = time.perf_counter() - t0
    split_ms = [a.elapsed_time(b) for a, b in ev]
    return wall, split_ms


def time_cold(w: Workload, iters: int, flush_buf, sink) -> list[float]:
    """bench_decode.cu:120-139 with a flush larger than L2 + the 256 MiB
    Infinity Cache: flush, event, decode + merge, event; per-run ms."""
    import torch
    import pa_amd
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    out = []
    for i in range(iters + 5):
        pa_amd.stream_read(flush_buf, flush_buf.numel(), 2048, sink, stream)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        w.split(sh)
        w.merge(sh)
        b.record(stream)
        b.synchronize()
        if i >= 5:
            out.append(a.elapsed_time(b))
    return out


def copy_ceiling(buf, sink, cus: int) -> dict:
    """bench_decode.cu:224-240: 16 B/lane streaming read at several grids."""
    import torch
    import pa_amd
    stream = torch.cuda.current_stream()
    best = None
    rows = []
    for mult in (4, 8, 16, 32):
        blocks = cus * mult
        ms = []
        for i in range(8):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            pa_amd.stream_read(buf, buf.numel(), blocks, sink, stream)
            b.record(stream)
            b.synchronize()
            if i >= 2:
                ms.append(a.elapsed_time(b))
        med = statistics.median(ms)
        gbps = buf.numel() / (med * 1e-3) / 1e9
        rows.append({"blocks": blocks, "gbps": round(gbps, 1)})
        if best is None or gbps > best:
            best = gbps
    return {"gbps": round(best, 1), "frac": round(best / PEAK_GBPS, 4), "bytes": buf.numel(), "grids": rows}


def cpu_baseline(w: Workload, budget_s: float, threads: int) -> dict:
    import oracle
    q, K, V = w.host_fp32_items()
    use_ref = oracle.ref_lib() is not None
    times = []
    t_start = time.perf_counter()
    while True:
        _, secs = oracle.attention_pairs(q, K, V, w.lens, HKV, threads=threads, use_reference=use_ref)
        times.append(secs)
        if len(times) >= 3 or time.perf_counter() - t_start > budget_s:
            break
        if len(times) >= 1 and (time.perf_counter() - t_start) + secs > budget_s:
            break
    med = statistics.median(times)
    return {
        "value": round(w.bytes / med / 1e9, 3),
        "unit": "GB/s",
        "us_per_step": round(med * 1e6, 1),
        "cores": threads,
        "kind": "reference" if use_ref else "port",
        "sample": (f"all {w.batch * HQ} (row, query head) pairs of {w.name} "
                   f"({w.batch} x {max(w.lens)} tokens), {len(times)} run(s), median; "
                   f"K/V gathered and dequantized to fp32 beforehand (untimed)"),
    }


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
    ap.add_argument("--cold-iters", type=int, default=50)
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU-baseline work")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = min(16, host cores)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-cold", action="store_true")
    ap.add_argument("--no-copy", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs (--gpus > 1) are not part of it",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import pa_amd
    if not torch.cuda.is_available():
        print("bench.py: needs a GPU (cuda:0)", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    pa_amd._lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count

    print(f"# bench: config {args.config}, page_size {args.page_size}", file=sys.stderr, flush=True)
    w = Workload(args.config, args.page_size)
    w.bind_fast()
    print(f"# setup done: {w.batch} seqs, {w.num_pages} pages, plan {w.plan.num_ctas} units / "
          f"{len(w.plan.segments)} segments", file=sys.stderr, flush=True)

    wall, split_ms = time_steps(w, args.steps, args.warmup)
    ms_per_step = wall * 1e3 / args.steps
    value = w.bytes / (ms_per_step * 1e-3) / 1e9
    split_avg = statistics.mean(split_ms)
    achieved = w.bytes / (split_avg * 1e-3) / 1e9
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
                (", FP8 E4M3 at amax/448" if w.fp8 else ""),
        "config": {
            "workload": w.desc,
            "batch": w.batch,
            "seq_len": max(w.lens),
            "total_tokens": sum(w.lens),
            "num_q_heads": HQ,
            "num_kv_heads": HKV,
            "head_dim": D,
            "page_size": args.page_size,
            "kv_dtype": "fp8_e4m3" if w.fp8 else "fp16",
            "units": w.plan.num_ctas,
            "segments": int(len(w.plan.segments)),
            "algorithmic_bytes": w.bytes,
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
        },
    }

    if not args.no_cold or not args.no_copy:
        flush = torch.empty(4 << 30, dtype=torch.uint8, device="cuda")
        flush.fill_(1)
        sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        if not args.no_copy:
            result["copy_ceiling"] = copy_ceiling(flush, sink, cus)
        if not args.no_cold:
            cold = time_cold(w, args.cold_iters, flush[: 1 << 30], sink)
            med = statistics.median(cold)
            result["cold"] = {"us_median": round(med * 1e3, 2), "gbps": round(w.bytes / (med * 1e-3) / 1e9, 1),
                              "frac": round(w.bytes / (med * 1e-3) / 1e9 / PEAK_GBPS, 4),
                              "iters": args.cold_iters, "flush_bytes": 1 << 30}
        del flush

    if not args.no_cpu:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_budget, threads)

    w.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
