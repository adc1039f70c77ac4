"""Benchmarks of the paged split-KV decode path; CSV on stdout, the same modes,
flags and columns as the reference's bench/bench_decode.cu:1-16:

    python -m pa_amd.bench_decode sweep     [--dtype fp16|fp8]   batch x seq_len sweep
    python -m pa_amd.bench_decode ctas      --batch B --len L     persistent-grid sweep
    python -m pa_amd.bench_decode pagesize  --batch B --len L     page-size sweep
    python -m pa_amd.bench_decode capacity  [--budget-gib G]     sequences per KV budget
    python -m pa_amd.bench_decode copy                           attainable read bandwidth
    python -m pa_amd.bench_decode single    --batch B --len L    one configuration
    python -m pa_amd.bench_decode append    --batch B --len L    per-slot vs batched append
    python -m pa_amd.bench_decode order     --batch B --len L    decode time per page placement

Common flags: --hq 32 --hkv 8 --dim 128 --page 16 --iters 50 --dtype fp16|fp8
              --ctas N (0 = default grid) --contiguous-pages (no free-list shuffle)
              --peak-gbps X (default 8000, MI355X HBM3E)
              --warm (no cache flush between iterations: what a working set that
                      fits the 256 MiB Infinity Cache costs when it is resident)

Timing (bench_decode.cu:120-139): the step is planned once; every iteration
first streams a 1 GiB buffer (larger than L2 plus the 256 MiB Infinity Cache,
where the reference's 2 x L2 would not be) so the KV cache is read from HBM,
then times only the decode kernels with HIP events; the median is reported.
Bandwidth counts the bytes the kernel must move (bench_decode.cu:186-191).

Data: q/K/V ~ N(0,1) rounded to fp16, distinct per sequence, appended through
PagedKVCache.append (FP8: per-tensor amax/448 scales, quantized by the append
kernel). The reference bench fills uniform [-2, 2] and appends one K/V to every
sequence; the values do not change the timing.
"""

from __future__ import annotations

import math
import statistics
import sys

from . import core
from ._lib import InvalidArgument

PEAK_GBPS = 8000.0
FLUSH_BYTES = 1 << 30


def algorithmic_bytes(lens, hq: int, hkv: int, dim: int, page: int, fp8: bool) -> int:
    """bench_decode.cu:186-191: K and V once, q in and out once, the block table."""
    e = 1 if fp8 else 2
    return (2 * sum(lens) * hkv * dim * e + 2 * len(lens) * hq * dim * 2
            + sum(math.ceil(L / page) for L in lens) * 4)


class Setup:
    """A populated PagedKVCache plus q/out and a bound plan for one decode shape
    (bench_decode.cu:142-192)."""

    def __init__(self, lens, hq: int = 32, hkv: int = 8, dim: int = 128, page: int = 16,
                 fp8: bool = False, shuffle: bool = True, ctas: int = 0, seed: int = 42,
                 k_scale: float | None = None, v_scale: float | None = None):
        import torch

        self.lens = [int(x) for x in lens]
        self.batch = len(self.lens)
        self.hq, self.hkv, self.dim, self.page, self.fp8 = hq, hkv, dim, page, fp8
        self.dtype = core.FP8_E4M3 if fp8 else core.FP16
        pages = [math.ceil(L / page) for L in self.lens]
        self.num_pages = sum(pages)
        g = torch.Generator(device="cuda").manual_seed(seed)
        stream = torch.cuda.current_stream()
        srcs = [(torch.randn(L, hkv, dim, device="cuda", dtype=torch.float16, generator=g),
                 torch.randn(L, hkv, dim, device="cuda", dtype=torch.float16, generator=g)) for L in self.lens]
        if fp8:
            self.k_scale = k_scale or max(float(k.abs().max()) for k, _ in srcs) / 448.0
            self.v_scale = v_scale or max(float(v.abs().max()) for _, v in srcs) / 448.0
        else:
            self.k_scale = self.v_scale = 1.0
        self.cache = core.PagedKVCache(self.num_pages, page, hkv, dim, self.batch, max(pages), self.dtype,
                                       self.k_scale, self.v_scale)
        if shuffle:
            self.cache.shuffle_free_pages(seed)
        for b, (k, v) in enumerate(srcs):
            slot = self.cache.admit()
            assert slot == b
            if not self.cache.append(slot, k, v, self.lens[b], stream):
                raise RuntimeError("setup: out of pages")
        del srcs
        self.q = torch.randn(self.batch, hq, dim, device="cuda", dtype=torch.float16, generator=g)
        self.out = torch.empty_like(self.q)
        self.dplan = core.DevicePlan()
        self.replan(ctas)
        torch.cuda.synchronize()

    def replan(self, ctas: int) -> None:
        """PagedKVCache::plan with slots 0..B-1 (bench_decode.cu:198-201)."""
        import ctypes
        import torch
        self.plan = core.make_plan(self.dtype, self.lens, self.hq, self.hkv, self.dim, ctas)
        self.dplan.upload(self.plan, self.hq // self.hkv, self.dim, torch.cuda.current_stream())
        p = self.cache.params()
        p.q = self.q.data_ptr()
        p.out = self.out.data_ptr()
        p.slot_ids = None   # slot b holds row b
        p.batch = self.batch
        p.num_q_heads = self.hq
        self.dplan.bind(p)
        self.params = p
        self._lib = core.load()
        self._pref = ctypes.byref(self.params)

    def bytes(self) -> int:
        return algorithmic_bytes(self.lens, self.hq, self.hkv, self.dim, self.page, self.fp8)

    # The two launches of one decode step on a raw hipStream_t handle.
    def split(self, sh: int) -> None:
        core.check(self._lib.pa_decode_split(self.dtype, self._pref, sh))

    def merge(self, sh: int) -> None:
        core.check(self._lib.pa_decode_merge(self.dtype, self._pref, sh))

    def run(self, sh: int) -> None:
        core.check(self._lib.pa_decode(self.dtype, self._pref, sh))

    def close(self) -> None:
        self.cache.close()


class Flusher:
    """Streams FLUSH_BYTES so the next kernel reads from HBM (bench_decode.cu:105-117)."""

    def __init__(self, nbytes: int = FLUSH_BYTES):
        import torch
        self.buf = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
        self.sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def flush(self, stream) -> None:
        core.stream_read(self.buf, self.buf.numel(), 2048, self.sink, stream)


def time_cold(flusher: Flusher | None, iters: int, fn) -> list[float]:
    """bench_decode.cu:120-139: 5 flushed warm-ups, then per iteration flush,
    event, fn, event. Returns the per-iteration milliseconds. flusher=None
    times warm (no flush)."""
    import torch
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    for _ in range(5):
        if flusher:
            flusher.flush(stream)
        fn(sh)
    ms = []
    for _ in range(iters):
        if flusher:
            flusher.flush(stream)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn(sh)
        b.record(stream)
        b.synchronize()
        ms.append(a.elapsed_time(b))
    return ms


def copy_rows(cus: int, iters: int = 10, nbytes: int = 4 << 30) -> list[dict]:
    """bench_decode.cu:224-240 plus unrolled and non-temporal variants of the
    same 16 B/lane read: one row per (grid, block, unroll, nt); then the
    chunked read (one contiguous span per wave), the best read shape."""
    import torch
    buf = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    rows = []
    variants = [(m, 512, 1, False) for m in (4, 8, 16, 32)]
    variants += [(m, 256, u, nt) for m in (4, 8, 16) for u in (4, 8) for nt in (False, True)]
    for mult, threads, unroll, nt in variants:
        blocks = cus * mult
        ms = []
        for i in range(iters + 2):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            core.stream_read(buf, nbytes, blocks, sink, stream, threads=threads, unroll=unroll, nontemporal=nt)
            b.record(stream)
            b.synchronize()
            if i >= 2:
                ms.append(a.elapsed_time(b))
        med = statistics.median(ms)
        rows.append({"kernel": f"read_{blocks}x{threads}_u{unroll}{'_nt' if nt else ''}", "bytes": nbytes,
                     "time_us": med * 1e3, "gbps": nbytes / (med * 1e-3) / 1e9})
    for mult, unroll in ((1, 16), (2, 16), (4, 8)):
        blocks = cus * mult
        ms = []
        try:
            for i in range(iters + 2):
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                core.stream_read_chunked(buf, nbytes, blocks, sink, stream, threads=512, unroll=unroll)
                b.record(stream)
                b.synchronize()
                if i >= 2:
                    ms.append(a.elapsed_time(b))
        except InvalidArgument:   # spans do not divide evenly on this CU count
            continue
        med = statistics.median(ms)
        rows.append({"kernel": f"read_chunked_{blocks}x512_u{unroll}_nt", "bytes": nbytes,
                     "time_us": med * 1e3, "gbps": nbytes / (med * 1e-3) / 1e9})
    del buf
    return rows


def gpu_name() -> str:
    """The device name for CSV rows: the runtime's, or the ISA name when the
    runtime only has a generic one (its marketing names need libdrm's id table)."""
    import torch
    props = torch.cuda.get_device_properties(0)
    name = props.name
    if not name or name == "AMD Radeon Graphics":
        name = "AMD " + props.gcnArchName.split(":")[0]
    return name.replace(",", " ")


def chunked_read_same_bytes(cus: int, nbytes: int, iters: int = 10) -> dict | None:
    """The best chunked streaming read (one contiguous span per wave) of about
    `nbytes` (rounded down to what the span shapes divide): the read ceiling at
    a workload's own size, where launch ramp and tail weigh as they do for it."""
    import torch
    best = None
    for mult, unroll in ((1, 16), (2, 16), (4, 8)):
        blocks = cus * mult
        gran = blocks * 8 * unroll * 1024          # waves x unroll x 1 KiB
        n = nbytes // gran * gran
        if n == 0:
            continue
        buf = torch.ones(n, dtype=torch.uint8, device="cuda")
        sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        stream = torch.cuda.current_stream()
        ms = []
        try:
            for i in range(iters + 2):
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record(stream)
                core.stream_read_chunked(buf, n, blocks, sink, stream, threads=512, unroll=unroll)
                b.record(stream)
                b.synchronize()
                if i >= 2:
                    ms.append(a.elapsed_time(b))
        except InvalidArgument:
            continue
        finally:
            del buf
        med = statistics.median(ms)
        row = {"kernel": f"read_chunked_{blocks}x512_u{unroll}_nt", "bytes": n, "time_us": med * 1e3,
               "gbps": n / (med * 1e-3) / 1e9}
        if best is None or row["gbps"] > best["gbps"]:
            best = row
    return best


# ---- CLI (bench_decode.cu:213-326) ------------------------------------------

HEADER = "gpu,dtype,batch,seq_len,hq,hkv,dim,page,ctas,segments,time_us,gbps,pct_peak"

SWEEP_SHAPES = [(1, 4096), (1, 16384), (1, 65536), (1, 131072), (8, 4096), (8, 16384), (8, 32768),
                (32, 1024), (32, 4096), (32, 8192), (64, 1024), (64, 4096), (128, 1024), (128, 2048)]


def append_rows(batch: int, hkv: int, dim: int, page: int, fp8: bool, steps: int, prefill: int) -> list[dict]:
    """Cost of growing the cache (paged_kv_cache.cu:95-136). A decode step
    appends one token to each of `batch` sequences: `batch` append calls (each
    synchronizes its stream, as the reference's) against one append_batch call
    (one pinned copy + one kernel, no synchronization); wall time per step over
    `steps` steps. Then a prefill of `prefill` tokens per sequence through one
    append_batch call, timed with events (host staging and its copy included;
    median of 5); bytes = fp16 K and V read + K and V written at the cache's
    width."""
    import time

    import torch
    dt = core.FP8_E4M3 if fp8 else core.FP16
    eb = 1 if fp8 else 2
    per_seq = 2 * steps + 6 * prefill
    max_pages = math.ceil(per_seq / page)
    cache = core.PagedKVCache(batch * max_pages, page, hkv, dim, batch, max_pages, dt, 4.0 / 448, 4.0 / 448)
    slots = [cache.admit() for _ in range(batch)]
    ones = [1] * batch
    k1 = torch.randn(batch, hkv, dim, device="cuda", dtype=torch.float16)
    v1 = torch.randn_like(k1)
    sh = torch.cuda.current_stream()
    rows = []
    row_bytes = hkv * dim * 2

    def per_slot():
        for b in slots:
            cache.append(b, k1.data_ptr() + b * row_bytes, v1.data_ptr() + b * row_bytes, 1, sh)

    def batched():
        cache.append_batch(slots, ones, k1, v1, sh)

    for name, fn in (("per_slot", per_slot), ("batched", batched)):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps - 1):
            fn()
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) / (steps - 1) * 1e6
        nbytes = batch * row_bytes * 2 + batch * hkv * dim * eb * 2
        rows.append(dict(mode=name, tokens=1, calls=batch if name == "per_slot" else 1, us=us,
                         gbps=nbytes / (us * 1e-6) / 1e9))
    kp = torch.randn(batch * prefill, hkv, dim, device="cuda", dtype=torch.float16)
    vp = torch.randn_like(kp)
    counts = [prefill] * batch
    ms = []
    for _ in range(5):   # the first call of each of the two staging buffers allocates it
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        assert cache.append_batch(slots, counts, kp, vp, sh)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    us = statistics.median(ms) * 1e3
    nbytes = batch * prefill * (row_bytes * 2 + hkv * dim * eb * 2)
    rows.append(dict(mode="prefill_batched", tokens=prefill, calls=1, us=us, gbps=nbytes / (us * 1e-6) / 1e9))
    # Read+write ceiling for comparison: a device-to-device copy of the fp16
    # K and V (the runtime's copy kernel), same read bytes, fp16 write bytes.
    dst = torch.empty_like(kp)
    ms = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(kp)
        dst.copy_(vp)
        e1.record()
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
    us = statistics.median(ms) * 1e3
    nbytes = 4 * kp.numel() * kp.element_size()
    rows.append(dict(mode="d2d_copy_ceiling", tokens=prefill, calls=2, us=us, gbps=nbytes / (us * 1e-6) / 1e9))
    cache.close()
    return rows


def _options(argv: list[str]):
    """The command line as typed options (argparse: unknown options, bad values
    and unknown modes exit with status 2; --help prints the usage). No device
    is touched before it succeeds."""
    import argparse
    ap = argparse.ArgumentParser(prog="python -m pa_amd.bench_decode", description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("mode", nargs="?", default="sweep", choices=MODES)
    for name, default in (("batch", None), ("len", None), ("hq", 32), ("hkv", 8), ("dim", 128), ("page", 16),
                          ("iters", 50), ("ctas", 0), ("steps", 200), ("max-len", 8192)):
        ap.add_argument(f"--{name}", type=int, default=default)
    ap.add_argument("--dtype", choices=("fp16", "fp8"), default=None)
    ap.add_argument("--budget-gib", type=float, default=1.0)
    ap.add_argument("--peak-gbps", type=float, default=PEAK_GBPS)
    ap.add_argument("--contiguous-pages", action="store_true", help="no free-list shuffle")
    ap.add_argument("--warm", action="store_true", help="no cache flush between iterations")
    return ap.parse_args(argv)


def run_one(gpu: str, peak: float, fl: Flusher | None, s: Setup, ctas: int, iters: int) -> dict:
    s.replan(ctas)
    ms = statistics.median(time_cold(fl, iters, s.run))
    gbps = s.bytes() / (ms * 1e-3) / 1e9
    row = dict(gpu=gpu, dtype=core.kv_dtype_name(s.dtype), batch=s.batch, seq_len=max(s.lens), hq=s.hq,
               hkv=s.hkv, dim=s.dim, page=s.page, ctas=s.plan.num_ctas, segments=len(s.plan.segments),
               time_us=ms * 1e3, gbps=gbps, pct_peak=100.0 * gbps / peak)
    print(f"{gpu},{row['dtype']},{s.batch},{row['seq_len']},{s.hq},{s.hkv},{s.dim},{s.page},{row['ctas']},"
          f"{row['segments']},{row['time_us']:.2f},{gbps:.1f},{row['pct_peak']:.1f}", flush=True)
    return row


def page_orders(batch: int, npg: int, page_bytes: int, seed: int = 7) -> dict:
    """Placements of the batch's pages, each a permutation of the page ranks
    0 .. batch * npg - 1 (rank r = row r // npg, page r % npg of an in-order
    pool): entry (b, i) of the block table takes the perm[b * npg + i]-th page
    of the pool in memory order."""
    import numpy as np
    n = batch * npg
    rng = np.random.default_rng(seed)
    order = {"memory_order": np.arange(n),
             # page i of row b handed out as all rows grow together
             "interleaved": (np.arange(npg)[None, :] * batch + np.arange(batch)[:, None]).reshape(-1),
             "shuffled": rng.permutation(n)}
    for span in (256 << 10, 2 << 20):
        g = max(1, span // page_bytes)
        if n % g:
            continue
        q = np.arange(n).reshape(-1, g)
        name = f"{span >> 10}KiB" if span < (1 << 20) else f"{span >> 20}MiB"
        order[f"shuffled_within_{name}"] = np.concatenate([rng.permutation(r) for r in q])
        order[f"{name}_groups_shuffled"] = q[rng.permutation(len(q))].reshape(-1)
    return order


def page_order_rows(gpu: str, peak: float, fl, batch: int, length: int, hq: int, hkv: int, dim: int, page: int,
                    fp8: bool, iters: int) -> list[dict]:
    """Decode time at one page size under different placements of the same
    pages. The pool is filled in memory order (no free-list shuffle); each row
    points the step at a block table that permutes its pages (page_orders), so
    the kernels read the same number of bytes from other addresses. The values
    then belong to other rows' tokens: the rows time placement only."""
    import numpy as np
    import torch
    s = Setup([length] * batch, hq, hkv, dim, page, fp8, shuffle=False)
    npg = math.ceil(length / page)
    own = np.stack([s.cache.block_table(b)[:npg] for b in range(batch)])
    pages = np.sort(own.reshape(-1))   # the pool's pages in memory order
    stride = s.params.block_table_stride
    eb = 1 if fp8 else 2
    page_bytes = hkv * page * dim * eb
    rows = []
    for name, perm in page_orders(batch, npg, page_bytes).items():
        t = np.zeros((batch, stride), np.int32)
        t[:, :npg] = pages[perm].reshape(batch, npg)
        table = torch.from_numpy(t).cuda()
        s.replan(0)
        s.params.block_table = table.data_ptr()
        ms = statistics.median(time_cold(fl, iters, s.run))
        gbps = s.bytes() / (ms * 1e-3) / 1e9
        row = dict(order=name, time_us=ms * 1e3, gbps=gbps, pct_peak=100.0 * gbps / peak)
        print(f"{gpu},{core.kv_dtype_name(s.dtype)},{batch},{length},{page},{name},{row['time_us']:.2f},"
              f"{gbps:.1f},{row['pct_peak']:.1f}", flush=True)
        rows.append(row)
        del table
    s.close()
    return rows


MODES = ("sweep", "ctas", "pagesize", "capacity", "copy", "single", "append", "order")


def main(argv: list[str] | None = None) -> int:
    o = _options(sys.argv[1:] if argv is None else argv)
    mode = o.mode
    import torch
    core.load()
    props = torch.cuda.get_device_properties(0)
    gpu = gpu_name()
    cus = props.multi_processor_count
    peak = o.peak_gbps
    print(f"# {gpu}, {cus} CUs, HBM peak {peak:.0f} GB/s", file=sys.stderr, flush=True)
    hq, hkv, dim = o.hq, o.hkv, o.dim
    page, iters, ctas = o.page, o.iters, o.ctas
    shuffle = not o.contiguous_pages

    if mode == "copy":
        print("gpu,kernel,bytes,time_us,gbps,pct_peak")
        for r in copy_rows(cus):
            print(f"{gpu},{r['kernel']},{r['bytes']},{r['time_us']:.2f},{r['gbps']:.1f},"
                  f"{100 * r['gbps'] / peak:.1f}", flush=True)
        return 0

    fp8 = o.dtype == "fp8"
    if mode == "append":
        print("gpu,dtype,mode,batch,tokens_per_seq,calls_per_step,us_per_step,gbps,pct_peak")
        b = o.batch if o.batch is not None else 64
        for r in append_rows(b, hkv, dim, page, fp8, o.steps, o.len if o.len is not None else 1024):
            print(f"{gpu},{'fp8_e4m3' if fp8 else 'fp16'},{r['mode']},{b},{r['tokens']},{r['calls']},"
                  f"{r['us']:.2f},{r['gbps']:.1f},{100 * r['gbps'] / peak:.1f}", flush=True)
        return 0

    fl = None if o.warm else Flusher()
    # Multi-row modes keep every row's cache until the mode ends: a row timed
    # within some milliseconds of freeing an earlier row's cache ran about 5%
    # slower (32 x 8192 fp16: 170.8 against 161.7 us) while the freed memory
    # was being released.
    kept: list[Setup] = []
    if mode == "sweep":
        print(HEADER)
        dts = [fp8] if o.dtype else [False, True]
        for dt in dts:
            for b, L in SWEEP_SHAPES:
                kept.append(Setup([L] * b, hq, hkv, dim, page, dt, shuffle))
                run_one(gpu, peak, fl, kept[-1], ctas, iters)
        for s in kept:
            s.close()
        return 0

    batch = o.batch if o.batch is not None else 32
    length = o.len if o.len is not None else 4096
    if mode == "single":
        print(HEADER)
        s = Setup([length] * batch, hq, hkv, dim, page, fp8, shuffle)
        run_one(gpu, peak, fl, s, ctas, iters)
        return 0
    if mode == "order":
        print("gpu,dtype,batch,seq_len,page,order,time_us,gbps,pct_peak")
        page_order_rows(gpu, peak, fl, batch, length, hq, hkv, dim, page, fp8, iters)
        return 0
    if mode == "ctas":
        print(HEADER)
        s = Setup([length] * batch, hq, hkv, dim, page, fp8, shuffle)
        wave = core.wave_ctas(s.dtype, dim, hq // hkv)
        print(f"# one wave = {wave} work units", file=sys.stderr, flush=True)
        grid = [cus // 2, cus, 2 * cus, 3 * cus, 4 * cus, 6 * cus, 8 * cus, 12 * cus, 16 * cus, wave]
        for n in sorted(set(grid)):
            run_one(gpu, peak, fl, s, n, iters)
        return 0
    if mode == "pagesize":
        print(HEADER)
        for ps in (1, 4, 8, 16, 32, 64, 128, 256, 1024, length):
            if ps > length:
                continue
            kept.append(Setup([length] * batch, hq, hkv, dim, ps, fp8, shuffle))
            run_one(gpu, peak, fl, kept[-1], ctas, iters)
        for s in kept:
            s.close()
        return 0
    if mode == "capacity":
        # bench_decode.cu:285-321: sequences that fit one layer's KV budget.
        budget = int(o.budget_gib * (1 << 30))
        max_len = o.max_len
        print("dtype,layout,max_len,actual_len,sequences,bytes_per_seq")
        for actual in (256, 512, 1024, 2048, 4096, 8192):
            per_contig = 2 * max_len * hkv * dim * 2
            print(f"fp16,contiguous,{max_len},{actual},{budget // per_contig},{per_contig}")
            for dt in (core.FP16, core.FP8_E4M3):
                cfg = core.CacheConfig(0, page, hkv, dim, 0, (max_len + page - 1) // page, dt,
                                       2.0 / 448.0, 2.0 / 448.0)
                n_pages = core.PagedKVCache.pages_for_budget(cfg, budget)
                cache = core.PagedKVCache(n_pages, page, hkv, dim, n_pages, (max_len + page - 1) // page, dt,
                                          2.0 / 448.0, 2.0 / 448.0)
                src = (torch.rand(actual, hkv, dim, device="cuda") * 4 - 2).to(torch.float16)
                n = 0
                while True:
                    slot = cache.admit()
                    if slot < 0 or not cache.append(slot, src, src, actual):
                        break
                    n += 1
                print(f"{core.kv_dtype_name(dt)},paged,{max_len},{actual},{n},"
                      f"{cache.total_bytes() // n if n else 0}", flush=True)
                cache.close()
        return 0
    raise AssertionError(f"mode {mode} has no handler")


if __name__ == "__main__":
    sys.exit(main())
