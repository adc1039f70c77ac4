"""GPU parity tests of the split-KV decode kernels, through the C ABI.

Cases mirror tests/test_paged_decode.cu:158-221 of the reference (same shapes,
lengths, page sizes, grids and chunked appends), plus seeded random
configurations, many short rows, pools past 4 GiB, the in-block merge against
the merge kernel and HIP-graph capture. The bar is tighter than the
reference's 4e-3: max-abs <= 2e-3 against the fp32 CPU oracle (fp16 KV) or the
oracle over the same dequantized FP8 values; stored cache bytes (block-table
scatter and FP8 quantization) must be bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
import pa_amd
from helpers import D, TOL, decoder_case, paged_inputs, run_cache_case

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu_device")]

DTYPES = [False, True]   # fp8?
IDS = ["fp16", "fp8"]


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
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (8, 1)])
@pytest.mark.parametrize("page_size", [1, 3, 4])
def test_small_pages_every_group(fp8, hq, hkv, page_size):
    """The per-lane staged page path (page sizes 1, 2, FP8 4 and non-powers
    of two) for GQA groups 1, 2 and 8, with a ragged batch whose rows end
    inside a step."""
    err, _, _ = run_cache_case(fp8, hq, hkv, page_size, [5, 333, 1027])
    assert err < TOL, err

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_mixed_length_batch(fp8):
    err, _, _ = run_cache_case(fp8, 32, 8, 16, [1, 15, 16, 17, 129, 1000, 4099])
    assert err < TOL, err

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
@pytest.mark.parametrize("page_size", [1, 2, 3, 4, 6, 8, 16, 32, 128, 256, 8192])
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
    for page_size, shuffle in [(16, None), (16, 3), (8, 2), (4, 11), (1, 5), (2048 + 64, None), (8192, 9)]:
        _, out, _ = run_cache_case(fp8, 32, 8, page_size, lens, shuffle_seed=shuffle)
        outs.append(out)
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))

@pytest.mark.parametrize("case", range(24))
def test_seeded_random_configurations(case):
    """24 seeded random combinations of dtype, GQA shape (groups 1 to 8), page
    size (1 to 1024, powers of two and not), batch, lengths (1 .. 6000), grid
    size (one unit to more than one resident wave) and append chunking (per
    slot or batched) through the cache, each against the oracle (bytes
    bit-exact, output within TOL)."""
    rng = np.random.default_rng(1000 + case)
    fp8 = bool(rng.integers(0, 2))
    shapes = [(8, 8), (8, 4), (16, 4), (32, 8), (8, 1), (32, 4), (64, 8), (16, 2), (2, 1)]
    hq, hkv = shapes[int(rng.integers(0, len(shapes)))]
    page = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 12, 16, 32, 64, 128, 256, 1024]))
    lens = [int(x) for x in rng.integers(1, 6001, size=int(rng.integers(1, 9)))]
    ctas = int(rng.choice([0, 0, 1, 3, 17, 300, 2048, 3000]))
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
    err, dec = decoder_case(len(lens), lens, fp8, threads=16)
    assert dec.num_segments >= 600 * 8
    assert err < TOL, err

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_pages_beyond_4gib_of_pool(fp8):
    """Pools larger than 4 GiB: the same sequence stored in the first pages
    and in pages past the 4 GiB mark of each pool decodes to the same bits
    (64-bit page offsets in every load path: power-of-two, staged small
    pages and per-lane)."""
    import torch
    hq, hkv = 32, 8
    for P in (16, 8, 5):
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

@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_block_merge_and_merge_kernel_agree(fp8):
    """A plan whose split rows each lie in one block of 8 work units (8 units
    per row) is merged inside the split kernel; forcing the merge kernel on the
    same plan must give the same answer, both against the oracle."""
    import torch
    lens = [2048] * 8
    q, k, v, table, ks, vs = paged_inputs(len(lens), lens, 32, 8, 16, fp8, seed=5)
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

def test_persistent_grid_is_two_waves_per_simd():
    """The default grid is 8 work units (2 waves per SIMD) per CU for every
    dtype and group, whatever the kernels' register counts would let the
    hardware hold: more concurrent streams per CU read HBM less efficiently."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for dt in (pa_amd.FP16, pa_amd.FP8_E4M3):
        for g in (1, 2, 4, 8):
            assert pa_amd.wave_ctas(dt, D, g) == 8 * cus
    assert pa_amd.make_plan(pa_amd.FP16, [8192] * 32, 32, 8, D, 0).num_ctas == 8 * cus

def test_device_plan_rejects_unaligned_segment_starts():
    """A plan cut at 8-token tiles has segments starting off the kernels'
    16-token groups; DevicePlan::upload refuses it instead of letting a group
    read across a page boundary."""
    plan = pa_amd.make_plan_tiled(8, [100, 37], 8, 64)
    assert any(int(s[2]) % 16 for s in plan.segments)
    dplan = pa_amd.DevicePlan()
    with pytest.raises(pa_amd.InvalidArgument):
        dplan.upload(plan, 4, D)
    ok = pa_amd.make_plan_tiled(16, [100, 37], 8, 64)
    dplan.upload(ok, 4, D)

@pytest.mark.parametrize("group", [1, 2, 4, 8])
@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_block_merge_two_split_segments_per_unit(fp8, group):
    """Items of 8 tiles over units of 3 tiles: each 8-unit block holds three
    whole rows, and units 2 and 5 of a block end one row and start the next,
    so those waves hold two split segments (both LDS slots) and a block merges
    three runs of lengths 3, 4 and 3. Every group size (the LDS slot rows are
    G x head_dim) must match the merge kernel on the same plan and the oracle."""
    import torch
    hkv = 8
    hq = hkv * group
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    tile = pa_amd.tile_tokens(dt, D, group)
    lens = [8 * tile] * 3                          # 24 items x 8 tiles = 192 tiles
    units = 64                                     # 3 tiles per unit, 3 items per block
    q, k, v, table, ks, vs = paged_inputs(len(lens), lens, hq, hkv, 16, fp8, seed=11 + group)
    plan = pa_amd.make_plan(dt, lens, hq, hkv, D, units)
    assert plan.num_ctas == units
    dplan = pa_amd.DevicePlan()
    dplan.upload(plan, group, D)
    outs = []
    for force_kernel in (False, True):
        p = pa_amd.DecodeParams()
        p.q, p.k_cache, p.v_cache, p.block_table = q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr()
        out = torch.empty_like(q)
        p.out = out.data_ptr()
        p.block_table_stride = table.size(1)
        p.batch, p.num_q_heads, p.num_kv_heads, p.head_dim, p.page_size = len(lens), hq, hkv, D, 16
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
                              np.asarray(lens, np.int32), hq, hkv, D, 16, ks, vs, threads=16)
    for o in outs:
        assert float(np.max(np.abs(o - ref))) < TOL
    assert float(np.max(np.abs(outs[0] - outs[1]))) < 1e-3

def _device_ints(ptr, n):
    """n int32 from device memory (synchronous hipMemcpy)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    out = np.zeros(n, np.int32)
    assert hip.hipMemcpy(out.ctypes.data, ptr, 4 * n, 2) == 0   # hipMemcpyDeviceToHost
    return out

@pytest.mark.parametrize("lens,ctas,group", [
    ([1024] * 4, 0, 4),                    # C1's shape on the default grid: 8 blocks per item
    ([16384] * 4, 0, 4),                   # 8 blocks per item, the most the split kernel merges
    ([300, 4100, 17, 9000, 2500, 7000, 12000, 5000, 6000, 9000], 0, 4),   # ragged: items of 1 to 8 blocks
    ([3000, 5000, 64], 150, 1),            # G = 1 (a block merges fewer elements than threads)
    ([2048, 6000], 300, 2),
    ([4096] * 6, 0, 8),                    # G = 8 (two elements per thread)
    ([100] * 40 + [12000], 500, 4),        # many short whole items and one long split one
], ids=["c1", "two_rows", "ragged", "g1", "g2", "g8", "short_and_long"])
@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_chained_merge_matches_merge_kernel(fp8, lens, ctas, group):
    _chained_case(fp8, lens, ctas, group, 16)


@pytest.mark.parametrize("page", [1, 4, 8, 64])
@pytest.mark.parametrize("fp8", DTYPES, ids=IDS)
def test_chained_merge_every_page_path(fp8, page):
    """The merge across blocks on every page path (per-lane lookups at 1
    token per page, staged 1 KiB parts at 4 and 8, page runs at 64): 4 rows
    of 1024 tokens over 8 blocks each."""
    _chained_case(fp8, [1024] * 4, 0, 4, page)


def _chained_case(fp8, lens, ctas, group, page):
    """Plans whose split items span blocks are merged inside the split kernel
    (block_merge 2: block partials, per-item arrival counters, the last block
    combines). Against the merge kernel on the same plan and the oracle; two
    runs are bitwise equal (the combine order does not depend on which block
    finishes last), and the counters are back at zero after each decode."""
    import torch
    hkv = 8
    hq = hkv * group
    dt = pa_amd.FP8_E4M3 if fp8 else pa_amd.FP16
    q, k, v, table, ks, vs = paged_inputs(len(lens), lens, hq, hkv, page, fp8, seed=61 + group + len(lens) + page)
    plan = pa_amd.make_plan(dt, lens, hq, hkv, D, ctas)
    assert plan.merge_mode == 2
    dplan = pa_amd.DevicePlan()
    dplan.upload(plan, group, D)
    outs = []
    for force_kernel in (False, False, True):
        p = pa_amd.DecodeParams()
        p.q, p.k_cache, p.v_cache, p.block_table = q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr()
        out = torch.full_like(q, float("nan"))
        p.out = out.data_ptr()
        p.block_table_stride = table.size(1)
        p.batch, p.num_q_heads, p.num_kv_heads, p.head_dim, p.page_size = len(lens), hq, hkv, D, page
        p.sm_scale, p.k_scale, p.v_scale = pa_amd.sm_scale(D), ks, vs
        dplan.bind(p)
        assert p.block_merge == 2 and p.needs_merge == 0 and p.merge_counters
        if force_kernel:
            p.block_merge, p.needs_merge = 0, 1
        pa_amd.paged_decode(dt, p)
        torch.cuda.synchronize()
        assert not _device_ints(p.merge_counters, len(lens) * hkv).any()
        outs.append(out)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    kb = k.view(torch.uint8).cpu().numpy() if fp8 else k.view(torch.int16).cpu().numpy().view(np.uint16)
    vb = v.view(torch.uint8).cpu().numpy() if fp8 else v.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = oracle.paged_decode(dt, q.view(torch.int16).cpu().numpy().view(np.uint16), kb, vb, table.cpu().numpy(),
                              np.asarray(lens, np.int32), hq, hkv, D, page, ks, vs, threads=16)
    res = [o.float().cpu().numpy() for o in outs]
    for o in res:
        assert np.isfinite(o).all()
        assert float(np.max(np.abs(o - ref))) < TOL
    assert float(np.max(np.abs(res[0] - res[2]))) < 1e-3

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
def test_decoders_on_concurrent_streams_match_alone(fp8):
    """Three Decoders with different plans (32 x 2048: split rows merged in
    the split kernel; 4 x 1024 and a ragged batch: through the merge kernel)
    launched on three streams at once, five steps each with no
    synchronization between them: every output equals the same decoder's
    output when it runs alone, bitwise. Decoders share no device state (each
    has its own device plan and partial workspace)."""
    import torch
    cases = [([2048] * 32, 5), ([1024] * 4, 6), ([3000, 17, 9000], 7)]
    decs, args, alone = [], [], []
    for lens, seed in cases:
        q, k, v, table, ks, vs = paged_inputs(len(lens), lens, 32, 8, 16, fp8, seed)
        dec = pa_amd.Decoder(32, 8, D, 16, fp8)
        lt = torch.tensor(lens, dtype=torch.int32)
        dec.plan(lt, 0)
        a = (q, k, v, table, lt.cuda(), ks, vs)
        alone.append(dec.run(*a))
        decs.append(dec)
        args.append(a)
    torch.cuda.synchronize()
    assert decs[0].num_segments > 32 * 8 and decs[1].num_segments > 4 * 8   # split rows in both
    streams = [torch.cuda.Stream() for _ in cases]
    outs = [[] for _ in cases]
    for _ in range(5):
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                outs[i].append(decs[i].run(*args[i]))
    torch.cuda.synchronize()
    for i, lens_seed in enumerate(cases):
        for n, o in enumerate(outs[i]):
            assert torch.equal(o, alone[i]), f"decoder {i} {lens_seed[0][:3]} step {n} differs"
