"""Where a decode step's time goes inside the split kernel: per-block
s_memrealtime stamps of its phases, from a diagnostic build of the library.

    python3 build.py -D PA_STAMPS=1 --lib lib/variants/libpa_decode_stamps.so
    PA_DECODE_LIB=lib/variants/libpa_decode_stamps.so \\
        python3 -m pa_amd.phase_stamps [--shape B L fp16|fp8]... [--heads HQ HKV] [--merge-kernel]

For each shape (default: 4 x 1024, 2 x 16384 and 1 x 131072, fp16 and FP8 for
the last) a populated cache (bench_decode.Setup: 16-token shuffled pages, the
default grid) runs 50 warm decode steps, then 200 timed back to back (HIP
events: the period of one step), and the stamps of the last step are read
back. Times are microseconds after the first block started (100 MHz clock).
One JSON line per shape:

  period_us          one step back to back (kernel plus the gap to the next);
                     with --cold, cold_step_us: the median step after a 1 GiB flush
  wave_end           p0 / p50 / p100 of the waves' ends of their split loop
  block_mean_end     p0 / p50 / p100 over blocks of their waves' mean end
  xcd_mean_end       that mean per XCD (blocks b, b + 8, ... run on XCD b % 8)
  xcd_clock_mhz      the shader clock per XCD over wave 0's split loop (s_memtime
                     ticks per microsecond)
  merge_in_block     per block, from its last wave's end to its merged items
                     (the LDS merge, and for items that span blocks the
                     partial row stored), then its parts: barrier (to the
                     merge's start), lds (the slots' partials read),
                     count (the first item's segment count loaded), average
                     (the weighted average computed, its stores issued)
  store_wait         those partial rows complete at the coherence point
  arrive             the arrival counter's round trip
  combine            the last block's combine of an item's block partials:
                     loads returned / running maximum / lane tree / output
  last_end           the last stamp of the step

The phases after `wave_end` exist when the plan merges across blocks inside
the split kernel (block_merge 2); --merge-kernel forces the merge kernel on
the same plan instead (block_merge 0), whose launch the period then includes.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import sys

from . import core
from .bench_decode import Flusher, Setup

TICK_US = 0.01   # s_memrealtime runs at 100 MHz
SLOTS = 24       # stamps per block: 0 start, 1-8 wave ends, 9-15 and 16-19 the merge phases,
                 # 20-21 the shader clock (s_memtime) at the start and at wave 0's end


def stamps_of(s: Setup, steps: int = 200, flusher: Flusher | None = None) -> dict:
    import numpy as np
    import torch
    lib = core.load()
    if not hasattr(lib, "pa_debug_stamps"):
        raise SystemExit("the loaded library has no stamps: build it with -D PA_STAMPS=1 and set PA_DECODE_LIB")
    lib.pa_debug_stamps.argtypes = [ctypes.c_void_p, ctypes.c_ulong]
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    for _ in range(50):
        s.run(sh)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if flusher is None:
        a.record(stream)
        for _ in range(steps):
            s.run(sh)
        b.record(stream)
        b.synchronize()
        period_ms = a.elapsed_time(b) / steps
    else:
        # The reference's cold method: a 1 GiB read before every step, events
        # around the step alone; the median step.
        ms = []
        for _ in range(steps // 4):
            flusher.flush(stream)
            a.record(stream)
            s.run(sh)
            b.record(stream)
            b.synchronize()
            ms.append(a.elapsed_time(b))
        period_ms = sorted(ms)[len(ms) // 2]
    nb = (s.plan.num_ctas + 7) // 8
    buf = np.zeros(nb * SLOTS, np.uint64)
    if lib.pa_debug_stamps(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("pa_debug_stamps failed")
    st = buf.reshape(nb, SLOTS).astype(np.int64)
    clk = st[:, 20:22].copy()      # another counter: not comparable with the 100 MHz stamps
    st[:, 20:22] = 0
    # A stamp older than its block's start belongs to an earlier step (a phase
    # this step's block did not reach): dropped.
    st = np.where(st >= st[:, :1], st, 0)
    t0 = st[:, 0].min()

    def us(x):
        return (x - t0) * TICK_US

    def p50_max(x):
        return [round(float(np.median(x)), 2), round(float(np.max(x)), 2)] if len(x) else None

    wend = st[:, 1:9]
    blk_end = wend.max(1)
    cu_mean = us(wend).mean(1)   # one block per CU: its waves' mean end
    r = {"batch": s.batch, "len": s.lens[0], "hq": s.hq, "hkv": s.hkv,
         "dtype": "fp8_e4m3" if s.fp8 else "fp16", "page": s.page,
         "block_merge": int(s.params.block_merge), "blocks": nb,
         "period_us" if flusher is None else "cold_step_us": round(period_ms * 1e3, 2),
         "wave_end": [round(float(np.percentile(us(wend), q)), 2) for q in (0, 50, 100)],
         "block_mean_end": [round(float(np.percentile(cu_mean, q)), 2) for q in (0, 50, 100)],
         "xcd_mean_end": [round(float(cu_mean[x::8].mean()), 2) for x in range(8)] if nb % 8 == 0 else None}
    # Shader clock of each block's CU over wave 0's split loop (MHz).
    span = (st[:, 1] - st[:, 0]) * TICK_US
    ok = (span > 0) & (clk[:, 1] > clk[:, 0])
    mhz = np.where(ok, (clk[:, 1] - clk[:, 0]) / np.where(span > 0, span, 1), np.nan)
    if nb % 8 == 0 and ok.any():
        r["xcd_clock_mhz"] = [round(float(np.nanmean(mhz[x::8])), 0) for x in range(8)]
    last_end = us(blk_end).max()
    if s.params.block_merge != 0:
        cnt = np.maximum(st[:, 18], st[:, 19])   # blocks holding a split segment
        ent = (st[:, 16] > 0) & (cnt > 0)
        r["merge_barrier"] = p50_max((st[ent, 16] - blk_end[ent]) * TICK_US)
        r["merge_lds"] = p50_max((st[ent, 17] - st[ent, 16]) * TICK_US)
        r["merge_count"] = p50_max((cnt[ent] - st[ent, 17]) * TICK_US)
    if s.params.block_merge == 2:
        arr = st[:, 9] > 0
        r["merge_average"] = p50_max((st[arr, 9] - cnt[arr]) * TICK_US)
        last = st[:, 15] > st[:, 11]
        r["merge_in_block"] = p50_max((st[arr, 9] - blk_end[arr]) * TICK_US)
        r["store_wait"] = p50_max((st[arr, 10] - st[arr, 9]) * TICK_US)
        r["arrive"] = p50_max((st[arr, 11] - st[arr, 10]) * TICK_US)
        r["combine"] = [round(float(np.median((st[last, k + 1] - st[last, k]) * TICK_US)), 2)
                        for k in (11, 12, 13, 14)] if last.any() else None
        r["combining_blocks"] = int(last.sum())
        if last.any():
            last_end = max(last_end, us(st[last, 15]).max())
    r["last_end"] = round(float(last_end), 2)
    return r


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", nargs=3, action="append", metavar=("BATCH", "LEN", "DTYPE"))
    ap.add_argument("--heads", nargs=2, type=int, default=(32, 8), metavar=("HQ", "HKV"),
                    help="query and kv heads (default 32 8; e.g. 4 1 for one GPU's share of 8-way head sharding)")
    ap.add_argument("--merge-kernel", action="store_true", help="force the merge kernel (block_merge 0)")
    ap.add_argument("--page", type=int, default=16, help="tokens per page")
    ap.add_argument("--contiguous-pages", action="store_true", help="no free-list shuffle (pages in memory order)")
    ap.add_argument("--cold", action="store_true", help="a 1 GiB flush before every step (the stamps are the last step's)")
    o = ap.parse_args(sys.argv[1:] if argv is None else argv)
    shapes = o.shape or [("4", "1024", "fp16"), ("2", "16384", "fp16"), ("1", "131072", "fp16"),
                         ("1", "131072", "fp8")]
    import torch
    torch.cuda.init()
    core.load()
    flusher = Flusher() if o.cold else None
    for b, length, dt in shapes:
        s = Setup([int(length)] * int(b), hq=o.heads[0], hkv=o.heads[1], page=o.page, fp8=dt == "fp8",
                  shuffle=not o.contiguous_pages)
        if o.merge_kernel and s.params.block_merge != 0:
            s.params.block_merge, s.params.needs_merge = 0, 1
        print(json.dumps(stamps_of(s, flusher=flusher)), flush=True)
        s.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
