"""Our paged decode against a ROCm comparator on identical inputs, through the
torch `Decoder` binding (the counterpart of scripts/compare_flashinfer.py).

    python -m pa_amd.compare [--iters 50] [--quick] [--repeats 1]

FlashInfer has no ROCm build, so the comparator is what a torch-ROCm user
without a paged kernel runs: gather the pages of every sequence through the
block table into contiguous [B, Hq, L, D] fp16 K/V (dequantizing FP8), then
torch's scaled_dot_product_attention with its flash or memory-efficient
backend (the faster one is kept, as compare_flashinfer.py keeps the faster
FlashInfer variant). The gather is inside the comparator's timed region: it is
the price of not reading pages in place.

Inputs follow compare_flashinfer.py:80-97: N(0,1) fp16 pools drawn from a
seeded CUDA generator, a random page permutation as the block table, and for
FP8 the pools divided by the per-tensor amax/448 scales and cast to
float8_e4m3fn (so the FP8 cache is a quantized copy of the fp16 one of the
same seed). Timing is bench_decode.py's cold method (1 GiB flush, events,
median).

CSV columns are compare_flashinfer.py's, with the comparator in FlashInfer's
two columns: gpu,dtype,batch,seq_len,ours_us,comparator_us,comparator_variant,
ours_gbps,ours_pct_peak,ratio (comparator time / ours),max_abs_diff (ours vs
comparator),max_abs_diff_vs_ref (vs the fp32 torch reference),
fp8_err_vs_fp16,fp8_rel_err_vs_fp16 (FP8 output vs the fp16-cache output:
max abs, relative L2).
"""

from __future__ import annotations

import argparse
import math
import statistics
import sys

import torch

from . import bench_decode, core
from .decoder import Decoder

HQ, HKV, DIM, PAGE = 32, 8, 128, 16
SHAPES = [(1, 16384), (1, 65536), (1, 131072), (8, 4096), (8, 16384), (8, 32768),
          (32, 1024), (32, 4096), (32, 8192), (64, 4096), (128, 1024), (128, 2048)]
QUICK = [(32, 8192), (8, 32768)]
REF_LIMIT = 32 * 4096   # compare_flashinfer.py:163: the fp32 reference runs up to this many tokens
HEADER = ("gpu,dtype,batch,seq_len,ours_us,comparator_us,comparator_variant,ours_gbps,ours_pct_peak,ratio,"
          "max_abs_diff,max_abs_diff_vs_ref,fp8_err_vs_fp16,fp8_rel_err_vs_fp16")


def make_inputs(batch: int, seq_len: int, fp8: bool, seed: int = 0):
    """compare_flashinfer.py:80-97: q, k, v, k_scale, v_scale, block_table,
    seq_lens (CPU int32). Pools are [pages, Hkv, P, D]."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    pages_per_seq = math.ceil(seq_len / PAGE)
    num_pages = batch * pages_per_seq
    k = torch.randn(num_pages, HKV, PAGE, DIM, device="cuda", dtype=torch.float16, generator=g)
    v = torch.randn(num_pages, HKV, PAGE, DIM, device="cuda", dtype=torch.float16, generator=g)
    k_scale = v_scale = 1.0
    if fp8:
        k_scale = k.abs().max().item() / 448.0
        v_scale = v.abs().max().item() / 448.0
        k = (k / k_scale).to(torch.float8_e4m3fn)
        v = (v / v_scale).to(torch.float8_e4m3fn)
    # The same values in pools laid out as the library's own caches lay theirs
    # out (one allocation, V a small gap after K; see core.alloc_kv_pools).
    kp, vp = core.alloc_kv_pools(num_pages, HKV, PAGE, DIM, fp8)
    if fp8:
        kp, vp = kp.view(torch.float8_e4m3fn), vp.view(torch.float8_e4m3fn)
    kp.copy_(k)
    vp.copy_(v)
    k, v = kp, vp
    perm = torch.randperm(num_pages, device="cuda", generator=g).to(torch.int32)
    block_table = perm.view(batch, pages_per_seq).contiguous()
    q = torch.randn(batch, HQ, DIM, device="cuda", dtype=torch.float16, generator=g)
    seq_lens = torch.full((batch,), seq_len, dtype=torch.int32)
    return q, k, v, k_scale, v_scale, block_table, seq_lens


def gather(cache: torch.Tensor, block_table: torch.Tensor, seq_len: int, scale: float) -> torch.Tensor:
    """[pages, Hkv, P, D] pool -> contiguous fp16 [B, Hkv, seq_len, D] per block-table row."""
    b, n = block_table.shape
    x = cache[block_table.reshape(-1).long()]                       # [B*n, Hkv, P, D]
    if x.dtype != torch.float16:
        x = x.to(torch.float16) * scale if scale != 1.0 else x.to(torch.float16)
    x = x.view(b, n, HKV, PAGE, DIM).permute(0, 2, 1, 3, 4).reshape(b, HKV, n * PAGE, DIM)
    return x[:, :, :seq_len]


def comparator(q, k, v, k_scale, v_scale, block_table, seq_len, backend):
    """Gather + expand to Hq heads + SDPA(backend) in fp16; returns [B, Hq, D]."""
    from torch.nn.attention import sdpa_kernel
    g = HQ // HKV

    def run():
        kb = gather(k, block_table, seq_len, k_scale).repeat_interleave(g, dim=1)
        vb = gather(v, block_table, seq_len, v_scale).repeat_interleave(g, dim=1)
        with sdpa_kernel(backend):
            o = torch.nn.functional.scaled_dot_product_attention(q.unsqueeze(2), kb, vb)
        return o.squeeze(2)
    return run


def reference(q, k, v, k_scale, v_scale, block_table, seq_len):
    """compare_flashinfer.py:113-126: fp32 attention over the dequantized
    pages, one sequence at a time (matmuls on contiguous fp32 operands)."""
    g = HQ // HKV
    outs = []
    for b in range(block_table.shape[0]):
        pages = block_table[b].long()
        kb = (k[pages].float() * k_scale).permute(1, 0, 2, 3).reshape(HKV, -1, DIM)[:, :seq_len]
        vb = (v[pages].float() * v_scale).permute(1, 0, 2, 3).reshape(HKV, -1, DIM)[:, :seq_len]
        qb = q[b].float().view(HKV, g, DIM)
        s = torch.matmul(qb, kb.transpose(1, 2).contiguous()) / math.sqrt(DIM)
        outs.append(torch.matmul(s.softmax(-1), vb.contiguous()).reshape(HQ, DIM))
    return torch.stack(outs)


def _time(fn, flusher, iters: int, repeats: int) -> float:
    return statistics.median(statistics.median(bench_decode.time_cold(flusher, iters, lambda _sh: fn()))
                             for _ in range(repeats))


def rows(shapes=SHAPES, iters: int = 50, repeats: int = 1, dtypes=(False, True), peak: float = 8000.0,
         log=sys.stderr):
    """Yields one dict per (dtype, shape), in compare_flashinfer.py's order (all
    fp16 shapes, then all FP8 shapes, so every FP8 row has its fp16 twin)."""
    from torch.nn.attention import SDPBackend
    gpu = bench_decode.gpu_name()
    flusher = bench_decode.Flusher()
    fp16_out = {}
    for fp8 in dtypes:
        for batch, seq_len in shapes:
            q, k, v, ks, vs, bt, lens = make_inputs(batch, seq_len, fp8)
            dec = Decoder(HQ, HKV, DIM, PAGE, fp8)
            dec.plan(lens, 0)
            lens_dev = lens.cuda()
            ours = lambda: dec.run(q, k, v, bt, lens_dev, ks, vs)   # noqa: E731
            ours_ms = _time(ours, flusher, iters, repeats)
            out = ours()
            best = None
            for name, backend in (("gather+sdpa_flash", SDPBackend.FLASH_ATTENTION),
                                  ("gather+sdpa_efficient", SDPBackend.EFFICIENT_ATTENTION)):
                try:
                    fn = comparator(q, k, v, ks, vs, bt, seq_len, backend)
                    c_out = fn()
                    c_ms = _time(fn, flusher, iters, repeats)
                except Exception as e:   # a backend can be unavailable for a shape or build
                    print(f"# comparator {name} failed: {e}", file=log, flush=True)
                    continue
                if best is None or c_ms < best[0]:
                    best = (c_ms, name, c_out)
            c_ms, variant, c_out = best if best else (float("nan"), "none", None)
            diff = (out.float() - c_out.float()).abs().max().item() if c_out is not None else float("nan")
            ref_diff = float("nan")
            if batch * seq_len <= REF_LIMIT:
                ref_diff = (out.float() - reference(q, k, v, ks, vs, bt, seq_len)).abs().max().item()
            fp8_err = fp8_rel = float("nan")
            if fp8 and (batch, seq_len) in fp16_out:
                base = fp16_out[(batch, seq_len)].cuda()
                fp8_err = (out.float() - base).abs().max().item()
                fp8_rel = ((out.float() - base).norm() / base.norm()).item()
            elif not fp8:
                fp16_out[(batch, seq_len)] = out.float().cpu()
            nbytes = bench_decode.algorithmic_bytes([seq_len] * batch, HQ, HKV, DIM, PAGE, fp8)
            gbps = nbytes / (ours_ms * 1e-3) / 1e9
            yield (dict(gpu=gpu, dtype="fp8_e4m3" if fp8 else "fp16", batch=batch, seq_len=seq_len,
                                 ours_us=ours_ms * 1e3, comparator_us=c_ms * 1e3, comparator_variant=variant,
                                 ours_gbps=gbps, ours_pct_peak=100 * gbps / peak, ratio=c_ms / ours_ms,
                                 max_abs_diff=diff, max_abs_diff_vs_ref=ref_diff, fp8_err_vs_fp16=fp8_err,
                                 fp8_rel_err_vs_fp16=fp8_rel))
            del q, k, v, bt, dec, out, c_out


def format_row(r: dict) -> str:
    return (f"{r['gpu']},{r['dtype']},{r['batch']},{r['seq_len']},{r['ours_us']:.2f},{r['comparator_us']:.2f},"
            f"{r['comparator_variant']},{r['ours_gbps']:.1f},{r['ours_pct_peak']:.1f},{r['ratio']:.3f},"
            f"{r['max_abs_diff']:.2e},{r['max_abs_diff_vs_ref']:.2e},{r['fp8_err_vs_fp16']:.2e},"
            f"{r['fp8_rel_err_vs_fp16']:.2e}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--repeats", type=int, default=1)
    ap.add_argument("--peak-gbps", type=float, default=bench_decode.PEAK_GBPS)
    args = ap.parse_args(argv)
    core.load()
    print(f"# {bench_decode.gpu_name()}, torch {torch.__version__}, peak {args.peak_gbps} GB/s",
          file=sys.stderr, flush=True)
    print(HEADER, flush=True)
    shapes = QUICK if args.quick else SHAPES
    for r in rows(shapes, args.iters, args.repeats, peak=args.peak_gbps):
        print(format_row(r), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
