"""GPU parity tests of the paged decode path, through the C ABI.

Cases mirror tests/test_paged_decode.cu:158-221 of the reference (same shapes,
lengths, page sizes, grids and chunked appends). The bar is tighter than the
reference's 4e-3: max-abs <= 2e-3 against the fp32 CPU oracle (fp16 KV) or the
oracle over the same dequantized FP8 values; stored cache bytes (block-table
scatter and FP8 quantization) must be bit-exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
import pa_amd
from helpers import D, TOL, d2h, normal_f16, run_cache_case, to_device

pytestmark = pytest.mark.gpu

DTYPES = [False, True]   # fp8?
IDS = ["fp16", "fp8"]


@pytest.fixture(scope="module", autouse=True)
def _device():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a device"
    pa_amd._lib.load()
    yield


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_single_token_sequence(fp8):
    err, _, _ = run_cache_case(fp8, 32, 8, 16, [1])
    assert err < TOL, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (16, 4), (32, 8), (8, 1)])
def test_gqa_groups(fp8, hq, hkv):
    err, _, _ = run_cache_case(fp8, hq, hkv, 16, [777])
    assert err < TOL, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_mixed_length_batch(fp8):
    err, _, _ = run_cache_case(fp8, 32, 8, 16, [1, 15, 16, 17, 129, 1000, 4099])
    assert err < TOL, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
@pytest.mark.parametrize("page_size", [1, 3, 8, 16, 32, 128])
def test_page_sizes(fp8, page_size):
    err, _, _ = run_cache_case(fp8, 16, 4, page_size, [300, 2500])
    assert err < TOL, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
@pytest.mark.parametrize("ctas", [1, 2, 7, 64, 1000])
def test_forced_cta_counts(fp8, ctas):
    err, _, plan = run_cache_case(fp8, 32, 8, 16, [5000, 90, 1, 700], num_ctas=ctas)
    assert plan.num_ctas <= ctas
    assert err < TOL, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_scattered_pages(fp8):
    err, _, _ = run_cache_case(fp8, 32, 8, 16, [400, 333, 612], chunk=5, shuffle_seed=7)
    assert err < TOL, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_long_sequence(fp8):
    err, _, _ = run_cache_case(fp8, 32, 8, 16, [32768], threads=16)
    assert err < TOL, err


def test_fp8_quantization_error_is_small():
    # tests/test_paged_decode.cu:200-204: against the unquantized fp16 values.
    err, _, _ = run_cache_case(True, 32, 8, 16, [2048], quantized_reference=False)
    assert err < 5e-2, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_output_invariant_under_page_placement(fp8):
    """The plan and the arithmetic do not depend on where pages live: outputs
    must be bitwise identical across page permutations and page sizes."""
    lens = [700, 1, 2049, 64]
    outs = []
    for page_size, shuffle in [(16, None), (16, 3), (4, 11), (1, 5), (2048 + 64, None)]:
        _, out, _ = run_cache_case(fp8, 32, 8, page_size, lens, shuffle_seed=shuffle)
        outs.append(out)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


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


@pytest.mark.parametrize("lens", [[1024] * 4, [20000], [300, 4100, 17]], ids=["c1", "long", "ragged"])
def test_graph_capture_replays_match_eager(lens):
    """A decode step (PagedKVCache::run: split + merge launches) captured into
    a HIP graph: every replay, with q rewritten and an eager decode of other
    inputs between replays, equals the eager decode of the same q bitwise. The
    launches record no memset nodes and keep no state between calls."""
    import torch
    hq, hkv = 32, 8
    pages = [-(-L // 16) for L in lens]
    cache = pa_amd.PagedKVCache(sum(pages) + 4, 16, hkv, D, len(lens), max(pages), pa_amd.FP16)
    g = torch.Generator(device="cuda").manual_seed(3)
    for L in lens:
        s_ = cache.admit()
        k = torch.randn(L, hkv, D, device="cuda", dtype=torch.float16, generator=g)
        assert cache.append(s_, k, torch.randn_like(k), L)
    cache.plan(list(range(len(lens))), hq)
    q = torch.randn(len(lens), hq, D, device="cuda", dtype=torch.float16, generator=g)
    out = torch.empty_like(q)
    other_q = torch.randn(q.shape, device="cuda", dtype=q.dtype, generator=g)
    other_out = torch.empty_like(q)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        cache.run(q, out, st)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            cache.run(q, out, torch.cuda.current_stream())
        torch.cuda.synchronize()
        for rep in range(4):
            q.normal_(generator=g)
            cache.run(q, out, st)                  # eager reference for this q
            torch.cuda.synchronize()
            ref = out.clone()
            out.zero_()
            graph.replay()
            cache.run(other_q, other_out, st)      # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {rep} differs"
    assert cache.last_plan().num_ctas > 0
    cache.close()


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


def _paged_inputs(batch, seq_lens, hq, hkv, page_size, fp8, seed):
    """compare_flashinfer.py:80-97 style inputs: N(0,1) pools filled on the
    device, a random page permutation as block table, per-tensor amax/448
    scales with append-time quantization for FP8."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    pages_per = [math.ceil(L / page_size) for L in seq_lens]
    num_pages = sum(pages_per)
    max_pages = max(pages_per)
    perm = torch.randperm(num_pages, device="cuda", generator=g).to(torch.int32)
    table = torch.zeros(batch, max_pages, dtype=torch.int32, device="cuda")
    off = 0
    for b, n in enumerate(pages_per):
        table[b, :n] = perm[off:off + n]
        off += n
    q = torch.randn(batch, hq, D, device="cuda", dtype=torch.float16, generator=g)
    if not fp8:
        k = torch.randn(num_pages, hkv, page_size, D, device="cuda", dtype=torch.float16, generator=g)
        v = torch.randn(num_pages, hkv, page_size, D, device="cuda", dtype=torch.float16, generator=g)
        return q, k, v, table, 1.0, 1.0
    kc = torch.zeros(num_pages, hkv, page_size, D, device="cuda", dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    srcs = []
    for b, L in enumerate(seq_lens):
        srcs.append((torch.randn(L, hkv, D, device="cuda", dtype=torch.float16, generator=g),
                     torch.randn(L, hkv, D, device="cuda", dtype=torch.float16, generator=g)))
    k_scale = max(float(s[0].abs().max()) for s in srcs) / 448.0
    v_scale = max(float(s[1].abs().max()) for s in srcs) / 448.0
    ik = float(np.float32(1.0) / np.float32(k_scale))
    iv = float(np.float32(1.0) / np.float32(v_scale))
    for b, (ks, vs) in enumerate(srcs):
        pa_amd.append_quantize(pa_amd.FP8_E4M3, ks, vs, kc, vc, table[b], 0, seq_lens[b], hkv, D, page_size, ik, iv)
    return q, kc, vc, table, k_scale, v_scale


def _decoder_case(batch, seq_lens, fp8, page_size=16, hq=32, hkv=8, seed=0, threads=16, rows=None):
    """Decodes the whole batch on the GPU; checks every row against the oracle,
    or only `rows` (a sample, for batches whose full oracle would take minutes)."""
    import torch
    q, k, v, table, ks, vs = _paged_inputs(batch, seq_lens, hq, hkv, page_size, fp8, seed)
    dec = pa_amd.Decoder(hq, hkv, D, page_size, fp8)
    lens = torch.tensor(seq_lens, dtype=torch.int32)
    dec.plan(lens, 0)
    out = dec.run(q, k, v, table, lens.cuda(), ks, vs)
    torch.cuda.synchronize()
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    kb = k.view(torch.uint8).cpu().numpy() if fp8 else k.view(torch.int16).cpu().numpy().view(np.uint16)
    vb = v.view(torch.uint8).cpu().numpy() if fp8 else v.view(torch.int16).cpu().numpy().view(np.uint16)
    sel = np.arange(batch) if rows is None else np.asarray(rows)
    qb = q.view(torch.int16).cpu().numpy().view(np.uint16)[sel]
    ref = oracle.paged_decode(dt, qb, kb, vb, table.cpu().numpy()[sel], np.asarray(seq_lens, np.int32)[sel], hq,
                              hkv, D, page_size, ks, vs, threads=threads)
    got = out.float().cpu().numpy()[sel]
    return float(np.max(np.abs(got - ref))), dec


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_decoder_binding_config1(fp8):
    """BASELINE config 1 shape (4 x 1024, P=16, scattered) via the torch_decode
    `Decoder` signature."""
    err, dec = _decoder_case(4, [1024] * 4, fp8)
    assert dec.num_ctas > 0 and dec.num_segments >= 32
    assert err < TOL, err


def test_decoder_full_size_config2():
    """BASELINE config 2 at full size: 32 x 8192 fp16, 16-token scattered pages."""
    err, _ = _decoder_case(32, [8192] * 32, False, threads=16)
    assert err < TOL, err


def test_decoder_long_context_config5_fp8():
    """BASELINE config 5 (1 x 131072), FP8 KV: hundreds of splits per row."""
    err, dec = _decoder_case(1, [131072], True, threads=8)
    assert dec.num_segments > 8 * 64
    assert err < TOL, err


def test_decoder_full_size_config3():
    """BASELINE config 3 at full size: 64 x 8192, FP8 E4M3 (amax/448 scales,
    quantized by the append kernel), 16-token scattered pages."""
    err, _ = _decoder_case(64, [8192] * 64, True, threads=16)
    assert err < TOL, err


def test_decoder_full_size_config4_sampled_rows():
    """BASELINE config 4 at full size (128 ragged rows, L ~ U[128, 16384],
    seed 4) decoded in one batch; 12 rows spread over the batch (first, last,
    longest, shortest, 8 seeded) checked against the oracle."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(128, 16385, size=128)]
    pick = {0, 127, int(np.argmax(lens)), int(np.argmin(lens))}
    pick |= set(int(x) for x in np.random.default_rng(9).choice(128, 8, replace=False))
    err, dec = _decoder_case(128, lens, False, threads=16, rows=sorted(pick))
    assert dec.num_segments >= 128 * 8
    assert err < TOL, err


def test_decoder_long_context_config5_fp16():
    """BASELINE config 5 (1 x 131072), fp16 KV."""
    err, dec = _decoder_case(1, [131072], False, threads=8)
    assert dec.num_segments > 8 * 64
    assert err < TOL, err


def test_full_size_output_invariant_under_page_placement():
    """At config 2's full size the output is bitwise the same for two
    different page permutations (the plan and tile order do not depend on
    placement), a size-independent check of block-table resolution."""
    import torch
    outs = []
    for seed in (0, 1):
        g = torch.Generator(device="cuda").manual_seed(123)
        n = 32 * 512
        k = torch.randn(n, 8, 16, D, device="cuda", dtype=torch.float16, generator=g)
        v = torch.randn(n, 8, 16, D, device="cuda", dtype=torch.float16, generator=g)
        q = torch.randn(32, 32, D, device="cuda", dtype=torch.float16, generator=g)
        logical = torch.arange(n, device="cuda", dtype=torch.int32).view(32, 512)
        perm = torch.randperm(n, device="cuda", generator=torch.Generator(device="cuda").manual_seed(seed))
        perm = perm.to(torch.int32)
        kp, vp = torch.empty_like(k), torch.empty_like(v)
        kp[perm.long()] = k                      # logical page i lives at physical page perm[i]
        vp[perm.long()] = v
        table = perm[logical.reshape(-1).long()].view(32, 512).contiguous()
        dec = pa_amd.Decoder(32, 8, D, 16, False)
        lens = torch.full((32,), 8192, dtype=torch.int32)
        dec.plan(lens, 0)
        outs.append(dec.run(q, kp, vp, table, lens.cuda(), 1.0, 1.0).view(torch.int16).cpu().numpy())
        del k, v, kp, vp
    assert np.array_equal(outs[0], outs[1])


def test_decoder_ragged_config4_subset():
    """BASELINE config 4's ragged lengths (U[128, 16384] from a seed), first 16 rows."""
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(128, 16385, size=16)]
    err, _ = _decoder_case(len(lens), lens, False, threads=16)
    assert err < TOL, err


@pytest.mark.parametrize("case", range(24))
def test_seeded_random_configurations(case):
    """24 seeded random combinations of dtype, GQA shape, page size, batch,
    lengths (1 .. 3000), grid size and append chunking through the cache,
    each against the oracle (bytes bit-exact, output within TOL)."""
    rng = np.random.default_rng(1000 + case)
    fp8 = bool(rng.integers(0, 2))
    hq, hkv = [(8, 8), (8, 4), (16, 4), (32, 8), (8, 1), (32, 4)][int(rng.integers(0, 6))]
    page = int(rng.choice([1, 2, 3, 5, 8, 16, 32, 64, 128]))
    lens = [int(x) for x in rng.integers(1, 3001, size=int(rng.integers(1, 9)))]
    ctas = int(rng.choice([0, 0, 1, 3, 17, 300]))
    chunk = int(rng.choice([0, 0, 7, 64]))
    err, _, plan = run_cache_case(fp8, hq, hkv, page, lens, num_ctas=ctas, chunk=chunk, seed=case,
                                  shuffle_seed=case, batched=bool(rng.integers(0, 2)))
    assert ctas == 0 or plan.num_ctas <= ctas
    assert err < TOL, (err, fp8, hq, hkv, page, lens, ctas, chunk)


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_many_short_rows(fp8):
    """600 rows of 1..200 tokens: more (row, kv head) items (4800) than work
    units, so units stream several whole items back to back and the pipeline
    crosses many segment boundaries (segment-start q loads, finishes)."""
    rng = np.random.default_rng(17)
    lens = [int(x) for x in rng.integers(1, 201, size=600)]
    err, dec = _decoder_case(len(lens), lens, fp8, threads=16)
    assert dec.num_segments >= 600 * 8
    assert err < TOL, err


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_pages_beyond_4gib_of_pool(fp8):
    """Pools larger than 4 GiB: the same sequence stored in the first pages
    and in pages past the 4 GiB mark of each pool decodes to the same bits
    (64-bit page offsets in every load path: power-of-two and per-lane)."""
    import torch
    hq, hkv = 32, 8
    for P in (16, 5):
        page_bytes = hkv * P * D * (1 if fp8 else 2)
        pages = (4 << 30) // page_bytes + 4096                 # the last pages start past 4 GiB
        dt = torch.uint8 if fp8 else torch.float16
        k = torch.empty((pages, hkv, P, D), dtype=dt, device="cuda")
        v = torch.empty_like(k)
        L = 300
        n = -(-L // P)
        g = torch.Generator(device="cuda").manual_seed(P)
        if fp8:
            k[:n] = torch.randint(0, 0x7f, (n, hkv, P, D), device="cuda", generator=g, dtype=torch.int32).to(torch.uint8)
            v[:n] = torch.randint(0, 0x7f, (n, hkv, P, D), device="cuda", generator=g, dtype=torch.int32).to(torch.uint8)
        else:
            k[:n] = torch.randn((n, hkv, P, D), device="cuda", generator=g, dtype=torch.float16)
            v[:n] = torch.randn((n, hkv, P, D), device="cuda", generator=g, dtype=torch.float16)
        high = torch.arange(pages - n, pages, device="cuda")
        assert int(high[0]) * page_bytes >= (4 << 30)
        q = torch.randn((1, hq, D), device="cuda", generator=g, dtype=torch.float16)
        lens = torch.tensor([L], dtype=torch.int32)
        dec = pa_amd.Decoder(hq, hkv, D, P, fp8)
        dec.plan(lens, 0)

        def run(table):
            return dec.run(q, k, v, table.to(torch.int32).view(1, n).contiguous(), lens.cuda(), 0.01, 0.01)

        outs = [run(torch.arange(n, device="cuda"))]
        k[high] = k[:n].clone()
        v[high] = v[:n].clone()
        k[: pages - n].zero_()        # a wrapped 32-bit offset would now read zeros
        v[: pages - n].zero_()
        outs.append(run(high))
        torch.cuda.synchronize()
        assert torch.isfinite(outs[0].float()).all()
        assert torch.equal(outs[0], outs[1]), f"page size {P}"
        del k, v
        torch.cuda.empty_cache()


def test_decoder_rejects_inconsistent_inputs():
    """Decoder.run raises RuntimeError (the reference's TORCH_CHECK) for inputs
    whose shapes or types do not match the plan, before any launch."""
    import torch
    q, k, v, table, ks, vs = _paged_inputs(2, [40, 17], 32, 8, 16, False, 0)
    dec = pa_amd.Decoder(32, 8, D, 16, False)
    lens = torch.tensor([40, 17], dtype=torch.int32)
    dec.plan(lens, 0)
    good = dict(q=q, k_cache=k, v_cache=v, block_table=table, seq_lens_dev=lens.cuda(), k_scale=1.0, v_scale=1.0)
    dec.run(**good)
    bad = [dict(q=q.float()), dict(q=q[:1].contiguous()), dict(q=q.view(2, 8, 4 * D)),
           dict(k_cache=k.view(-1, 8, 8, D)), dict(v_cache=v.view(torch.uint8)), dict(block_table=table[:, :2].contiguous()),
           dict(block_table=table.long()), dict(seq_lens_dev=lens), dict(k_cache=k.cpu())]
    for change in bad:
        with pytest.raises(RuntimeError):
            dec.run(**{**good, **change})
    torch.cuda.synchronize()


@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_block_merge_and_merge_kernel_agree(fp8):
    """A plan whose split rows each lie in one block of 8 work units (8 units
    per row) is merged inside the split kernel; forcing the merge kernel on the
    same plan must give the same answer, both against the oracle."""
    import torch
    lens = [2048] * 8
    q, k, v, table, ks, vs = _paged_inputs(len(lens), lens, 32, 8, 16, fp8, seed=5)
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    tile = pa_amd.tile_tokens(dt, D, 4)
    units = len(lens) * 8 * 8                      # 8 units per (row, kv head)
    plan = pa_amd.make_plan(dt, lens, 32, 8, D, units)
    assert plan.num_ctas == units and len(plan.segments) == units and 2048 // tile % 8 == 0
    dplan = pa_amd.DevicePlan()
    dplan.upload(plan, 4, D)
    outs = []
    for force_kernel in (False, True):
        p = pa_amd.DecodeParams()
        p.q, p.k_cache, p.v_cache, p.block_table = q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr()
        out = torch.empty_like(q)
        p.out = out.data_ptr()
        p.block_table_stride = table.size(1)
        p.batch, p.num_q_heads, p.num_kv_heads, p.head_dim, p.page_size = len(lens), 32, 8, D, 16
        p.sm_scale, p.k_scale, p.v_scale = pa_amd.sm_scale(D), ks, vs
        dplan.bind(p)
        assert p.block_merge == 1 and p.needs_merge == 0
        if force_kernel:
            p.block_merge, p.needs_merge = 0, 1
        pa_amd.paged_decode(dt, p)
        torch.cuda.synchronize()
        outs.append(out.float().cpu().numpy())
    kb = k.view(torch.uint8).cpu().numpy() if fp8 else k.view(torch.int16).cpu().numpy().view(np.uint16)
    vb = v.view(torch.uint8).cpu().numpy() if fp8 else v.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = oracle.paged_decode(dt, q.view(torch.int16).cpu().numpy().view(np.uint16), kb, vb, table.cpu().numpy(),
                              np.asarray(lens, np.int32), 32, 8, D, 16, ks, vs, threads=16)
    for o in outs:
        assert float(np.max(np.abs(o - ref))) < TOL
    assert float(np.max(np.abs(outs[0] - outs[1]))) < 1e-3
