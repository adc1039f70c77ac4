"""GPU tests of the cache side of the path, through the C ABI: the FP8
append-quantizer and page scatter (bit-exact against the oracle), the
block-table resolution probe, batched appends (paged_kv_cache.cu:95-136 grown
to a decode step's batch), PagedKVCache::plan over a subset of slots, and
planning the next step while the previous one is still queued.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
import pa_amd
from helpers import D, TOL, d2h, normal_f16, run_cache_case, to_device

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu_device")]

DTYPES = [False, True]   # fp8?
IDS = ["fp16", "fp8"]


@pytest.mark.parametrize("scale", [1.0, 4.0 / 448.0, 2.0 / 448.0, 4.87 / 448.0, 0.5, 3.0, 1e-3])
def test_append_fp8_bytes_exhaustive(scale):
    """Every fp16 input (all 65536 bit patterns, NaN and infinity included)
    through the append kernel, bit-exact against the oracle's E4M3 encoder."""
    import torch
    hkv, P = 1, 16
    n = 65536 // D                                  # 512 tokens x 128 dims
    k = np.arange(65536, dtype=np.uint16).reshape(n, hkv * D)
    v = k[::-1].copy()
    pages = n // P
    table = np.random.default_rng(1).permutation(pages).astype(np.int32)
    kc = torch.zeros(pages * hkv * P * D, dtype=torch.uint8, device="cuda")
    vc = torch.zeros_like(kc)
    inv = float(np.float32(1.0) / np.float32(scale))
    pa_amd.append_quantize(pa_amd.FP8_E4M3, to_device(k), to_device(v), kc, vc, to_device(table), 0, n, hkv, D,
                           P, inv, inv)
    torch.cuda.synchronize()
    ck = np.zeros(pages * P * D, dtype=np.uint8)
    cv = np.zeros_like(ck)
    oracle.append(1, k, v, ck, cv, table, 0, hkv, D, P, inv, inv)
    assert np.array_equal(kc.cpu().numpy(), ck)
    assert np.array_equal(vc.cpu().numpy(), cv)

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
@pytest.mark.parametrize("page_size,start", [(1, 0), (3, 5), (16, 0), (16, 9), (64, 100)])
def test_append_and_gather_bit_exact(fp8, page_size, start):
    """Append at an offset into scattered pages, then read it back through the
    decode kernel's own address function (gather probe); both bit-exact."""
    import torch
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    hkv, n = 4, 333
    rng = np.random.default_rng(page_size * 100 + start)
    k = normal_f16(rng, (n, hkv * D))
    v = normal_f16(rng, (n, hkv * D))
    pages = math.ceil((start + n) / page_size)
    pool_pages = pages + 7
    table = rng.permutation(pool_pages)[:pages].astype(np.int32)
    eb = 1 if fp8 else 2
    nbytes = pool_pages * hkv * page_size * D * eb
    kc = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    vc = torch.zeros_like(kc)
    inv = float(np.float32(448.0 / 4.0))
    pa_amd.append_quantize(dt, to_device(k), to_device(v), kc, vc, to_device(table), start, n, hkv, D, page_size,
                           inv, inv)
    ck = np.zeros(nbytes, dtype=np.uint8)
    cv = np.zeros_like(ck)
    view = (lambda a: a) if fp8 else (lambda a: a.view(np.uint16))
    oracle.append(dt, k, v, view(ck), view(cv), table, start, hkv, D, page_size, inv, inv)
    torch.cuda.synchronize()
    assert np.array_equal(kc.cpu().numpy(), ck)
    assert np.array_equal(vc.cpu().numpy(), cv)
    length = start + n
    dtable = to_device(table)
    for h in range(hkv):
        got = torch.zeros(length * D * eb, dtype=torch.uint8, device="cuda")
        pa_amd.gather_kv(dt, kc, dtable, hkv, D, page_size, h, length, got)
        torch.cuda.synchronize()
        exp = oracle.gather_raw(dt, view(ck), table, hkv, D, page_size, h, length)
        assert np.array_equal(got.cpu().numpy(), exp.view(np.uint8).reshape(-1))

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
@pytest.mark.parametrize("page_size,chunk", [(16, 1), (16, 7), (5, 3), (64, 0)])
def test_append_batch_decode_steps(fp8, page_size, chunk):
    """Sequences grown by batched appends (chunk=1: one token per sequence per
    call, as a decode step; many calls back to back, no synchronization between
    them): stored bytes bit-exact and decode within TOL of the oracle."""
    err, _, _ = run_cache_case(fp8, 32, 8, page_size, [1, 17, 100, 333, 16], chunk=chunk, shuffle_seed=11,
                               batched=True)
    assert err <= TOL

def _device_state(cache, slots, max_pages):
    p = cache.params()
    table = d2h(p.block_table, 4 * len(slots) * max_pages, np.int32).reshape(len(slots), max_pages)
    lens = d2h(p.seq_lens, 4 * len(slots), np.int32)
    return table, lens

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_append_batch_matches_sequential_appends(fp8):
    """Two caches, same shuffled free list: one grown by append (one call per
    slot and chunk), the other by append_batch with the same entries (a slot
    repeated within a batch, zero counts). Pools, device block tables and
    device lengths are bit-identical; an all-or-nothing refusal changes none."""
    import torch
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    hkv, P, slots_n, max_pages = 4, 8, 4, 12
    rng = np.random.default_rng(5)
    caches = [pa_amd.PagedKVCache(30, P, hkv, D, slots_n, max_pages, dt, 4.0 / 448, 3.0 / 448) for _ in range(2)]
    for c in caches:
        c.shuffle_free_pages(3)
        for _ in range(slots_n):
            c.admit()
    rounds = [([0, 1, 2, 3], [1, 9, 0, 17]), ([2, 0, 2], [5, 8, 3]), ([3, 1, 0, 2], [1, 1, 1, 1]),
              ([1], [30])]
    for slots, counts in rounds:
        total = sum(counts)
        k = to_device(normal_f16(rng, (total, hkv, D)))
        v = to_device(normal_f16(rng, (total, hkv, D)))
        off = 0
        for s_, n in zip(slots, counts):
            assert caches[0].append(s_, k.data_ptr() + off * hkv * D * 2, v.data_ptr() + off * hkv * D * 2, n)
            off += n
        assert caches[1].append_batch(slots, counts, k, v)
    # 18 pages are free; growing slots 0 and 2 to 90 and 89 tokens needs 10 + 10.
    free = caches[1].pool.free_pages()
    assert free == 18
    big = to_device(normal_f16(rng, (160, hkv, D)))
    assert not caches[1].append_batch([0, 2], [80, 80], big, big)
    assert caches[1].pool.free_pages() == free
    torch.cuda.synchronize()
    eb = 1 if fp8 else 2
    nbytes = 30 * hkv * P * D * eb
    pa, pb = caches[0].params(), caches[1].params()
    view = (lambda a: a) if fp8 else (lambda a: a.view(np.uint16))
    pools = [[view(d2h(getattr(p_, f), nbytes)) for f in ("k_cache", "v_cache")] for p_ in (pa, pb)]
    for s_ in range(slots_n):   # pools are not cleared at creation: compare the stored tokens
        t = caches[0].block_table(s_)
        assert list(t) == list(caches[1].block_table(s_))
        for h in range(hkv):
            for f in range(2):
                a = oracle.gather_raw(dt, pools[0][f], t, hkv, D, P, h, caches[0].seq_len(s_))
                b = oracle.gather_raw(dt, pools[1][f], t, hkv, D, P, h, caches[1].seq_len(s_))
                assert np.array_equal(a, b), f"slot {s_} head {h} {'kv'[f]}"
    ta, la = _device_state(caches[0], range(slots_n), max_pages)
    tb, lb = _device_state(caches[1], range(slots_n), max_pages)
    assert np.array_equal(ta, tb) and np.array_equal(la, lb)
    assert list(lb) == [caches[1].seq_len(s_) for s_ in range(slots_n)] == [10, 40, 9, 18]
    for s_ in range(slots_n):
        t = caches[1].block_table(s_)
        assert list(tb[s_, :len(t)]) == list(t)
    for c in caches:
        c.close()

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_append_batch_uniform_prefill_matches_sequential_appends(fp8):
    """Batches whose entries all hold the same number of tokens (a uniform
    prefill: the batched kernel finds every token's entry with its first guess,
    entry t * entries / tokens) and one whose counts differ by one token (the
    guess misses, the binary search finds the entry): pools, block tables and
    lengths are bit-identical to per-slot appends of the same tokens."""
    import torch
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    hkv, P, slots_n, max_pages = 4, 16, 5, 40
    rng = np.random.default_rng(11)
    caches = [pa_amd.PagedKVCache(160, P, hkv, D, slots_n, max_pages, dt, 4.0 / 448, 3.0 / 448) for _ in range(2)]
    for c in caches:
        c.shuffle_free_pages(9)
        for _ in range(slots_n):
            c.admit()
    rounds = [([0, 1, 2, 3, 4], [37] * 5), ([4, 2, 0], [16] * 3), ([1, 3, 0, 2, 4], [33, 32, 33, 32, 33])]
    for slots, counts in rounds:
        total = sum(counts)
        k = to_device(normal_f16(rng, (total, hkv, D)))
        v = to_device(normal_f16(rng, (total, hkv, D)))
        off = 0
        for s_, n in zip(slots, counts):
            assert caches[0].append(s_, k.data_ptr() + off * hkv * D * 2, v.data_ptr() + off * hkv * D * 2, n)
            off += n
        assert caches[1].append_batch(slots, counts, k, v)
    torch.cuda.synchronize()
    eb = 1 if fp8 else 2
    nbytes = 160 * hkv * P * D * eb
    view = (lambda a: a) if fp8 else (lambda a: a.view(np.uint16))
    pools = [[view(d2h(getattr(c.params(), f), nbytes)) for f in ("k_cache", "v_cache")] for c in caches]
    for s_ in range(slots_n):
        t = caches[0].block_table(s_)
        assert list(t) == list(caches[1].block_table(s_))
        for h in range(hkv):
            for f in range(2):
                a = oracle.gather_raw(dt, pools[0][f], t, hkv, D, P, h, caches[0].seq_len(s_))
                b = oracle.gather_raw(dt, pools[1][f], t, hkv, D, P, h, caches[1].seq_len(s_))
                assert np.array_equal(a, b), f"slot {s_} head {h} {'kv'[f]}"
    ta, la = _device_state(caches[0], range(slots_n), max_pages)
    tb, lb = _device_state(caches[1], range(slots_n), max_pages)
    assert np.array_equal(ta, tb) and np.array_equal(la, lb)
    assert list(lb) == [37 + 16 + 33, 37 + 33, 37 + 16 + 32, 37 + 32, 37 + 16 + 33]
    for c in caches:
        c.close()

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_cache_plan_subset_of_slots_in_any_order(fp8):
    """PagedKVCache::plan(slots) (paged_kv_cache.cu:173-191): batch row i reads
    cache slot slots[i]. A released and re-admitted slot, a subset of the
    slots in a permuted order, and rows of different lengths; against the
    oracle with the same slot mapping."""
    import torch
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    hq, hkv, P = 32, 8, 16
    scale = 4.0 / 448 if fp8 else 1.0
    rng = np.random.default_rng(21)
    lens = [100, 1, 700, 33, 2000, 16]
    pages = sum(-(-L // P) for L in lens) + 8
    cache = pa_amd.PagedKVCache(pages, P, hkv, D, 6, 2000 // P + 1, dt, scale, scale)
    cache.shuffle_free_pages(4)
    for L in lens:
        s_ = cache.admit()
        k = to_device(normal_f16(rng, (L, hkv, D)))
        assert cache.append(s_, k, to_device(normal_f16(rng, (L, hkv, D))), L)
    cache.release(1)
    assert cache.admit() == 1
    lens[1] = 50
    assert cache.append(1, to_device(normal_f16(rng, (50, hkv, D))), to_device(normal_f16(rng, (50, hkv, D))), 50)
    slots = [4, 1, 0, 5, 2]
    q = normal_f16(rng, (len(slots), hq, D))
    out = torch.empty((len(slots), hq, D), dtype=torch.float16, device="cuda")
    cache.plan(slots, hq)
    cache.run(to_device(q), out)
    torch.cuda.synchronize()
    p = cache.params()
    eb = 1 if fp8 else 2
    nbytes = pages * hkv * P * D * eb
    view = (lambda a: a) if fp8 else (lambda a: a.view(np.uint16))
    kc, vc = view(d2h(p.k_cache, nbytes)), view(d2h(p.v_cache, nbytes))
    table = np.zeros((6, 2000 // P + 1), np.int32)
    for s_ in range(6):
        t = cache.block_table(s_)
        table[s_, :len(t)] = t
    ref = oracle.paged_decode(dt, q, kc, vc, table, np.asarray([lens[s_] for s_ in slots], np.int32), hq, hkv, D, P,
                              scale, scale, slot_ids=np.asarray(slots, np.int32))
    got = out.float().cpu().numpy()
    assert float(np.max(np.abs(got - ref))) < TOL
    cache.close()


def _busy_stream(ms_of_reads: int = 20):
    """Queues ~ms_of_reads x 0.16 ms of plain 1 GiB reads on the current stream
    and returns an event recorded after them (the reads keep the stream busy)."""
    import torch
    buf = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    for _ in range(ms_of_reads):
        pa_amd.stream_read_chunked(buf, buf.numel(), 256, sink)
    ev = torch.cuda.Event()
    ev.record()
    return ev, buf


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_plan_next_step_while_previous_is_queued(fp8):
    """PagedKVCache::plan (decode.cu:131-146 DevicePlan::upload under it) queues
    its copies from pinned staging and does not synchronize the stream: with
    ~3 ms of reads queued, plan() returns while they still run; a sequence of
    steps (different slot subsets and orders, a re-plan of an earlier one)
    planned and run back to back without any synchronization equals,
    bitwise, the same steps each planned, run and synchronized alone."""
    import torch
    hq, hkv = 32, 8
    lens = [3000, 17, 1, 4100, 700, 16384]
    pages = [math.ceil(L / 16) for L in lens]
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    cache = pa_amd.PagedKVCache(sum(pages) + 8, 16, hkv, D, len(lens), max(pages), dt, 0.02, 0.02)
    cache.shuffle_free_pages(5)
    g = torch.Generator(device="cuda").manual_seed(2)
    for L in lens:
        s_ = cache.admit()
        k = torch.randn(L, hkv, D, device="cuda", dtype=torch.float16, generator=g)
        assert cache.append(s_, k, torch.randn_like(k), L)
    steps = [[0, 1, 2, 3, 4, 5], [5, 3, 1], [2], [4, 0], [0, 1, 2, 3, 4, 5], [1, 5]]
    qs = [torch.randn(len(s_), hq, D, device="cuda", dtype=torch.float16, generator=g) for s_ in steps]
    ref = []
    for slots, q in zip(steps, qs):
        out = torch.empty_like(q)
        cache.plan(slots, hq)
        cache.run(q, out)
        torch.cuda.synchronize()
        ref.append(out)
    ev, buf = _busy_stream()
    outs = []
    for i, (slots, q) in enumerate(zip(steps, qs)):
        cache.plan(slots, hq)
        if i == 0:
            assert not ev.query(), "plan() waited for work queued before it"
        outs.append(torch.empty_like(q))
        cache.run(q, outs[-1])
    assert not ev.query(), "the queued steps synchronized the stream"
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(outs, ref)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"step {i} differs"
    cache.close()


def test_decoder_plan_while_previous_run_is_queued():
    """The torch Decoder: run() with plan A, then plan(B) and run() without a
    synchronization in between (and with the stream busy): each output equals
    the eager one; plan(B) returns before the queued work is done."""
    import torch
    from helpers import paged_inputs
    lens_a, lens_b = [1024] * 4, [300, 5000, 77, 1]
    qa, ka, va, ta, _, _ = paged_inputs(4, lens_a, 32, 8, 16, False, seed=3)
    qb, kb, vb, tb, _, _ = paged_inputs(4, lens_b, 32, 8, 16, False, seed=4)
    la, lb = torch.tensor(lens_a, dtype=torch.int32), torch.tensor(lens_b, dtype=torch.int32)
    la_dev, lb_dev = la.cuda(), lb.cuda()        # (a blocking copy would synchronize the stream)
    dec = pa_amd.Decoder(32, 8, D, 16, False)
    dec.plan(la)
    ref_a = dec.run(qa, ka, va, ta, la_dev, 1.0, 1.0)
    dec.plan(lb)
    ref_b = dec.run(qb, kb, vb, tb, lb_dev, 1.0, 1.0)
    torch.cuda.synchronize()
    ev, buf = _busy_stream()
    dec.plan(la)
    out_a = dec.run(qa, ka, va, ta, la_dev, 1.0, 1.0)
    dec.plan(lb)
    assert not ev.query(), "Decoder.plan waited for queued work"
    out_b = dec.run(qb, kb, vb, tb, lb_dev, 1.0, 1.0)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), ref_a.view(torch.int16))
    assert torch.equal(out_b.view(torch.int16), ref_b.view(torch.int16))


def test_f32_f16_conversions():
    """pa_f32_to_f16 rounds to nearest even (the oracle's encoder, every fp16
    value, the midpoints between neighbours and one ulp either side, specials);
    pa_f16_to_f32 is exact for all 65536 codes."""
    import torch
    from pa_amd._lib import load
    lib = load()
    codes = np.arange(65536, dtype=np.uint16)
    h = to_device(codes)
    f = torch.empty(65536, dtype=torch.float32, device="cuda")
    assert lib.pa_f16_to_f32(h.data_ptr(), f.data_ptr(), 65536, None) == 0
    torch.cuda.synchronize()
    want = oracle.f16_bits_to_f32(codes)
    got = f.cpu().numpy()
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    v = oracle.f16_bits_to_f32(np.arange(0x7c00, dtype=np.uint16))
    mid = ((v[:-1].astype(np.float64) + v[1:]) / 2).astype(np.float32)
    x = np.concatenate([v, mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)),
                        [65504.0, 65519.0, 65520.0, 1e9, np.inf, 5.9e-8, 3e-8, 2.9e-8, 0.0]]).astype(np.float32)
    x = np.concatenate([x, -x])
    xd = torch.from_numpy(x).cuda()
    o = torch.empty(x.size, dtype=torch.int16, device="cuda")
    assert lib.pa_f32_to_f16(xd.data_ptr(), o.data_ptr(), x.size, None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(o.cpu().numpy().view(np.uint16), oracle.f32_to_f16_bits(x))


def test_cache_plan_and_run_of_no_slots():
    """PagedKVCache::plan of an empty slot list and PagedKVCache::decode of
    batch 0 (paged_kv_cache.cu:157-210 with no rows): a plan of zero work
    units and segments, and run / decode return without a launch or an error,
    also right after a non-empty decode on the same cache."""
    import torch
    hq, hkv = 32, 8
    cache = pa_amd.PagedKVCache(8, 16, hkv, D, 2, 4, pa_amd.FP16)
    q0 = torch.empty(0, hq, D, dtype=torch.float16, device="cuda")
    out0 = torch.empty_like(q0)
    cache.plan([], hq)
    assert cache.last_plan().num_ctas == 0 and len(cache.last_plan().segments) == 0
    cache.run(q0, out0)
    s_ = cache.admit()
    k = torch.randn(20, hkv, D, dtype=torch.float16, device="cuda")
    assert cache.append(s_, k, k, 20)
    q = torch.randn(1, hq, D, dtype=torch.float16, device="cuda")
    out = torch.empty_like(q)
    cache.decode(q, out, 1, hq)
    cache.decode(q0, out0, 0, hq)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    cache.close()
