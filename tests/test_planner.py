"""The persistent planner (decode.cu:65-108), through the C ABI and the oracle.

Pinned by the reference's own data: the (ctas, segments) columns of the 68
rows of results/h100_{sweep,pagesize,ctas}.csv (tests/golden/planner_rows.csv),
replayed at the reference's tile (64 tokens) and requested grid. Then the
product planner must equal the oracle's independent restatement exactly, and
satisfy the schedule's invariants, on random ragged batches.
"""

import csv
import pathlib

import numpy as np
import pytest

import oracle
import pa_amd

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _rows():
    with open(GOLDEN / "planner_rows.csv") as f:
        return list(csv.DictReader(f))


@pytest.mark.parametrize("row", _rows(), ids=lambda r: f"{r['source']}-{r['dtype']}-{r['batch']}x{r['seq_len']}-{r['requested']}")
def test_reference_plan_shapes(row):
    lens = [int(row["seq_len"])] * int(row["batch"])
    plan = pa_amd.make_plan_tiled(int(row["tile"]), lens, int(row["hkv"]), int(row["requested"]))
    assert plan.num_ctas == int(row["ctas"])
    assert len(plan.segments) == int(row["segments"])
    n, segs, _, _ = oracle.make_plan(int(row["tile"]), lens, int(row["hkv"]), int(row["requested"]))
    assert n == int(row["ctas"]) and len(segs) == int(row["segments"])


def _check_invariants(plan, lens, hkv, tile, requested):
    segs = plan.segments
    total = sum((L + tile - 1) // tile for L in lens) * hkv
    per = -(-total // requested)
    assert plan.num_ctas == -(-total // per)
    cta = plan.cta_seg_begin
    assert cta[0] == 0 and cta[-1] == len(segs) and np.all(np.diff(cta) >= 0)
    # each unit covers at most `per` tiles
    for u in range(plan.num_ctas):
        s = segs[cta[u]:cta[u + 1]]
        tiles = sum(-(-(int(t1) - int(t0)) // tile) for _, _, t0, t1 in s)
        assert 0 < tiles <= per
    # segments partition every item in token order
    item = plan.item_seg_begin
    assert item[0] == 0 and item[-1] == len(segs)
    for b, L in enumerate(lens):
        for h in range(hkv):
            i = b * hkv + h
            s = segs[item[i]:item[i + 1]]
            assert len(s) >= 1
            assert np.all(s[:, 0] == b) and np.all(s[:, 1] == h)
            assert s[0, 2] == 0 and s[-1, 3] == L
            assert np.all(s[1:, 2] == s[:-1, 3])
            assert np.all(s[:, 2] % tile == 0) and np.all(s[:, 3] > s[:, 2])


@pytest.mark.parametrize("seed", range(12))
def test_product_equals_oracle_and_invariants(seed):
    rng = np.random.default_rng(seed)
    batch = int(rng.integers(1, 40))
    lens = [int(x) for x in rng.integers(1, 20000, size=batch)]
    hkv = int(rng.choice([1, 2, 4, 8]))
    tile = int(rng.choice([16, 64]))
    requested = int(rng.integers(1, 2048))
    plan = pa_amd.make_plan_tiled(tile, lens, hkv, requested)
    n, segs, cta, item = oracle.make_plan(tile, lens, hkv, requested)
    assert plan.num_ctas == n
    assert np.array_equal(plan.segments, segs)
    assert np.array_equal(plan.cta_seg_begin, cta)
    assert np.array_equal(plan.item_seg_begin, item)
    _check_invariants(plan, lens, hkv, tile, requested)


def test_make_plan_uses_kernel_tile_and_validates():
    plan = pa_amd.make_plan(pa_amd.FP16, [8192] * 32, 32, 8, 128, 1024)
    assert plan.tile == pa_amd.tile_tokens(pa_amd.FP16, 128, 4) == 16
    _check_invariants(plan, [8192] * 32, 8, plan.tile, 1024)
    assert plan.needs_merge
    with pytest.raises(pa_amd.InvalidArgument, match="at least one token"):
        pa_amd.make_plan(pa_amd.FP16, [5, 0], 32, 8, 128, 64)
    with pytest.raises(pa_amd.InvalidArgument, match="multiple"):
        pa_amd.make_plan(pa_amd.FP16, [5], 30, 8, 128, 64)
    with pytest.raises(pa_amd.InvalidArgument, match="head_dim"):
        pa_amd.make_plan(pa_amd.FP16, [5], 32, 8, 64, 64)
    with pytest.raises(pa_amd.InvalidArgument, match="group"):
        pa_amd.make_plan(pa_amd.FP8_E4M3, [5], 48, 3, 128, 64)


def test_single_segment_rows_need_no_merge():
    plan = pa_amd.make_plan_tiled(64, [100, 64, 1], 2, 6)
    assert len(plan.segments) == 6 and not plan.needs_merge


def test_empty_batch_gives_empty_plan():
    plan = pa_amd.make_plan_tiled(64, [], 8, 100)
    assert plan.num_ctas == 0 and len(plan.segments) == 0


def _create(plan, num_kv_heads=0):
    import ctypes
    lib = pa_amd._lib.load()
    h = ctypes.c_void_p()
    seg = np.ascontiguousarray(plan["segments"], np.int32)
    cta = np.ascontiguousarray(plan["cta"], np.int32)
    itm = np.ascontiguousarray(plan["item"], np.int32)
    st = lib.pa_plan_create(plan["num_ctas"], plan["tile"], seg.ctypes.data, len(seg), cta.ctypes.data,
                            itm.ctypes.data, len(itm) - 1, num_kv_heads, ctypes.byref(h))
    if st == 0:
        lib.pa_plan_destroy(h.value)
    return st


def test_plan_create_accepts_built_plans_and_rejects_broken_ones():
    """pa_plan_create (behind DevicePlan::upload of a caller's DecodePlan)
    accepts every plan make_plan builds and rejects inconsistent ones."""
    rng = np.random.default_rng(3)
    lens = [int(x) for x in rng.integers(1, 3000, size=9)]
    built = pa_amd.make_plan_tiled(16, lens, 4, 37)
    good = dict(num_ctas=built.num_ctas, tile=16, segments=built.segments, cta=built.cta_seg_begin,
                item=built.item_seg_begin)
    assert _create(good) == 0 and _create(good, 4) == 0
    assert _create(good, 3) == 1                                  # items not a multiple of 3
    bad = dict(good, segments=built.segments.copy())
    bad["segments"][0, 3] = bad["segments"][0, 2]                 # empty segment
    assert _create(bad) == 1
    bad = dict(good, segments=built.segments.copy())
    a, b = int(built.item_seg_begin[0]), int(built.item_seg_begin[1])
    bad["segments"][[a, b]] = bad["segments"][[b, a]]             # listed under the wrong item
    assert _create(bad) == 1
    bad = dict(good, cta=built.cta_seg_begin.copy())
    bad["cta"][1], bad["cta"][2] = bad["cta"][2], bad["cta"][1]   # falling prefix
    assert _create(bad) == 1 or np.all(np.diff(bad["cta"]) >= 0)
    bad = dict(good, segments=built.segments.copy())
    i = int(np.argmax(built.segments[:, 3] - built.segments[:, 2]))
    assert built.segments[i, 3] - built.segments[i, 2] > 16
    bad["segments"][i, 2] += 8                                     # starts off a 16-token boundary
    assert _create(bad) == 1
    bad = dict(good, item=built.item_seg_begin.copy())
    bad["item"][-1] += 1                                           # does not end at num_segments
    assert _create(bad) == 1


def _created_mode(plan, num_kv_heads=0):
    """merge mode of a caller-built plan (pa_plan_create), or None if refused."""
    import ctypes
    lib = pa_amd._lib.load()
    h = ctypes.c_void_p()
    seg = np.ascontiguousarray(plan["segments"], np.int32)
    cta = np.ascontiguousarray(plan["cta"], np.int32)
    itm = np.ascontiguousarray(plan["item"], np.int32)
    if lib.pa_plan_create(plan["num_ctas"], plan["tile"], seg.ctypes.data, len(seg), cta.ctypes.data,
                          itm.ctypes.data, len(itm) - 1, num_kv_heads, ctypes.byref(h)) != 0:
        return None
    out = ctypes.c_int(-1)
    assert lib.pa_plan_merge_mode(h.value, ctypes.byref(out)) == 0
    lib.pa_plan_destroy(h.value)
    return out.value


@pytest.mark.parametrize("lens,units,tile,mode", [
    ([1024] * 4, 2048, 16, 2),        # C1 on the full grid: 8 blocks per (row, kv head)
    ([8192] * 32, 2048, 16, 1),       # C2: 8 units per item, one block each
    ([8192] * 64, 2048, 32, 1),       # C3 (FP8 step)
    ([131072], 2048, 16, 0),          # C5: 32 blocks per item, past the split kernel's limit of 8
    ([65536] * 2, 2048, 16, 0),       # 16 blocks per item
    ([32768] * 4, 2048, 16, 2),       # 8 blocks per item
    ([8192] * 32, 256, 16, 0),        # one unit per item: nothing split
    ([700, 33, 2000], 100, 16, 2),
])
def test_merge_mode_of_make_plan_cuts(lens, units, tile, mode):
    """Every make_plan cut keeps an item's segments in consecutive units, each
    the first or last of its unit, so the split kernel merges every split
    item itself: inside one block (1) or across blocks (2)."""
    plan = pa_amd.make_plan_tiled(tile, lens, 8, units)
    assert plan.merge_mode == mode
    n = len(plan.item_seg_begin) - 1
    if mode:
        assert len(plan.segments) > n
        unit_of = np.repeat(np.arange(plan.num_ctas), np.diff(plan.cta_seg_begin))
        for i in range(n):
            a, z = int(plan.item_seg_begin[i]), int(plan.item_seg_begin[i + 1])
            assert list(unit_of[a:z]) == list(range(unit_of[a], unit_of[a] + z - a))
            # The split kernel's addressing of a row's block partials: block j
            # of the row keeps its partial at the row's first segment in j,
            # a + max(0, 8 j - u0), for j from u0 // 8 to (u0 + n - 1) // 8.
            u0 = int(unit_of[a])
            for j in range(u0 // 8, (u0 + z - a - 1) // 8 + 1):
                first = min(sg for sg in range(a, z) if unit_of[sg] // 8 == j)
                assert first == a + max(0, 8 * j - u0)


def _expected_mode(plan):
    """The merge mode restated from the schedule: nothing split -> 0; every
    split item inside one block of 8 units -> 1; every split item over at most
    8 blocks -> 2 (make_plan cuts always keep an item's segments in
    consecutive units); else 0."""
    n = len(plan.item_seg_begin) - 1
    if len(plan.segments) <= n:
        return 0
    unit_of = np.repeat(np.arange(plan.num_ctas), np.diff(plan.cta_seg_begin))
    nbs = [unit_of[z - 1] // 8 - unit_of[a] // 8 + 1
           for a, z in zip(plan.item_seg_begin[:-1], plan.item_seg_begin[1:]) if z - a > 1]
    return 1 if max(nbs) == 1 else 2 if max(nbs) <= 8 else 0


def test_merge_mode_of_ragged_make_plan_cuts():
    rng = np.random.default_rng(4)
    lens = [int(x) for x in rng.integers(128, 16385, size=128)]   # C4
    assert pa_amd.make_plan_tiled(16, lens, 8, 2048).merge_mode == 2
    modes = set()
    for seed in range(40):
        rng = np.random.default_rng(100 + seed)
        lens = [int(x) for x in rng.integers(1, 40000, size=int(rng.integers(1, 40)))]
        plan = pa_amd.make_plan_tiled(16, lens, int(rng.choice([1, 2, 4, 8])), int(rng.integers(1, 3000)))
        assert plan.merge_mode == _expected_mode(plan)
        modes.add(plan.merge_mode)
    assert modes == {0, 1, 2}


def test_merge_mode_of_caller_plans():
    """Caller-built plans the split kernel cannot merge fall back to the merge
    kernel (0): an item whose segments skip a unit across blocks, and a split
    segment in the middle of a unit."""
    # hkv 1: item 0 = 64 tokens in units 0 and 9 (units 1..8 empty), item 1 whole.
    skip = dict(num_ctas=10, tile=16,
                segments=[[0, 0, 0, 32], [0, 0, 32, 64], [1, 0, 0, 32]],
                cta=[0, 1, 1, 1, 1, 1, 1, 1, 1, 1, 3], item=[0, 2, 3])
    assert _created_mode(skip, 1) == 0
    skip_in_block = dict(skip, num_ctas=3, cta=[0, 1, 1, 3])    # the same inside one block
    assert _created_mode(skip_in_block, 1) == 1
    # item 1 split twice inside unit 1: its first part is neither first nor last there.
    middle = dict(num_ctas=3, tile=16,
                  segments=[[0, 0, 0, 32], [0, 0, 32, 48], [1, 0, 0, 16], [1, 0, 16, 32], [1, 0, 32, 48],
                            [2, 0, 0, 16]],
                  cta=[0, 1, 5, 6], item=[0, 2, 5, 6])
    assert _created_mode(middle, 1) == 0
    whole = dict(num_ctas=2, tile=16, segments=[[0, 0, 0, 32], [1, 0, 0, 16]], cta=[0, 1, 2], item=[0, 1, 2])
    assert _created_mode(whole, 1) == 0                          # nothing to merge
