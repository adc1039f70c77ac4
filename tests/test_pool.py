"""Page pool and cache sizing (paged_kv_cache.cu:43-151), host-only, through the C ABI.

Pinned by the reference's known-answer test PagedKVCache.OutOfPagesRejectsAppend
(tests/test_paged_decode.cu:206-221) and by the 18 rows of
results/h100_capacity.csv (tests/golden/capacity_rows.csv), replayed by running
the allocator until it is full, as bench_decode.cu:291-325 does.
"""

import csv
import pathlib

import pytest

import pa_amd

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def test_out_of_pages_rejects_append():
    pool = pa_amd.PagePool(num_pages=2, page_size=16, max_slots=2, max_pages_per_slot=4)
    s = pool.admit()
    assert s == 0
    assert pool.reserve(s, 32)[0]
    assert pool.free_pages() == 0
    ok, _, num_new = pool.reserve(s, 1)
    assert not ok and num_new == 0
    assert pool.seq_len(s) == 32
    pool.release(s)
    assert pool.free_pages() == 2


def _cfg(dtype, page=16, hkv=8, dim=128, max_len=8192):
    return pa_amd.CacheConfig(0, page, hkv, dim, 0, (max_len + page - 1) // page, dtype, 2.0 / 448, 2.0 / 448)


@pytest.mark.parametrize("row", [r for r in csv.DictReader(open(GOLDEN / "capacity_rows.csv"))],
                         ids=lambda r: f"{r['dtype']}-{r['layout']}-{r['actual_len']}")
def test_capacity_rows(row):
    budget = 1 << 30
    max_len, actual = int(row["max_len"]), int(row["actual_len"])
    if row["layout"] == "contiguous":
        per_seq = 2 * max_len * 8 * 128 * 2
        assert budget // per_seq == int(row["sequences"]) and per_seq == int(row["bytes_per_seq"])
        return
    dtype = pa_amd.FP16 if row["dtype"] == "fp16" else pa_amd.FP8_E4M3
    cfg = _cfg(dtype, max_len=max_len)
    num_pages = pa_amd.PagedKVCache.pages_for_budget(cfg, budget)
    pool = pa_amd.PagePool(num_pages, 16, num_pages, cfg.max_pages_per_slot)
    n = 0
    while True:
        slot = pool.admit()
        if slot < 0 or not pool.reserve(slot, actual)[0]:
            break
        n += 1
    total = pa_amd.PagedKVCache.bytes_per_page(cfg) * num_pages
    assert n == int(row["sequences"])
    assert total // n == int(row["bytes_per_seq"])


def test_bytes_per_page():
    assert pa_amd.PagedKVCache.bytes_per_page(_cfg(pa_amd.FP16)) == 65536
    assert pa_amd.PagedKVCache.bytes_per_page(_cfg(pa_amd.FP8_E4M3)) == 32768


def test_free_list_order_and_reuse():
    pool = pa_amd.PagePool(8, 4, 3, 8)
    a = pool.admit()
    assert pool.reserve(a, 9)[0]                       # 3 pages
    assert list(pool.block_table(a)) == [0, 1, 2]      # page 0 is handed out first
    b = pool.admit()
    assert pool.reserve(b, 4)[0]
    assert list(pool.block_table(b)) == [3]
    pool.release(a)                                    # pushed back in table order
    c = pool.admit()
    assert c == a                                      # lowest free slot is reused
    assert pool.reserve(c, 12)[0]
    assert list(pool.block_table(c)) == [2, 1, 0]      # popped from the back
    assert pool.max_seq_len() == 12 and pool.occupied(b) and pool.seq_len(b) == 4


def test_incremental_growth_reports_new_entries():
    pool = pa_amd.PagePool(10, 16, 1, 10)
    s = pool.admit()
    assert pool.reserve(s, 5) == (True, 0, 1)
    assert pool.reserve(s, 11) == (True, 1, 0)          # fills page 0 exactly (16 tokens)
    assert pool.reserve(s, 1) == (True, 1, 1)
    assert pool.reserve(s, 0) == (True, 2, 0)
    assert pool.seq_len(s) == 17


def test_shuffle_is_a_deterministic_permutation():
    def order(seed):
        pool = pa_amd.PagePool(64, 1, 1, 64)
        pool.shuffle_free_pages(seed)
        s = pool.admit()
        pool.reserve(s, 64)
        return list(pool.block_table(s))
    a, b, c = order(42), order(42), order(43)
    assert sorted(a) == list(range(64)) and a == b and a != c and a != list(range(64))


def test_errors():
    with pytest.raises(pa_amd.InvalidArgument):
        pa_amd.PagePool(0, 16, 1, 1)
    pool = pa_amd.PagePool(4, 16, 2, 2)
    with pytest.raises(pa_amd.InvalidArgument, match="not admitted"):
        pool.reserve(1, 5)
    s = pool.admit()
    with pytest.raises(pa_amd.LengthError, match="max_pages_per_slot"):
        pool.reserve(s, 33)
    assert pool.seq_len(s) == 0
    with pytest.raises(pa_amd.InvalidArgument):
        pool.release(1)
    assert pool.admit() == 1 and pool.admit() == -1


def _twin_pools(seed=7):
    a, b = pa_amd.PagePool(40, 4, 6, 12), pa_amd.PagePool(40, 4, 6, 12)
    for p in (a, b):
        p.shuffle_free_pages(seed)
        for _ in range(5):
            p.admit()
    return a, b


def _state(pool, slots=range(5)):
    return pool.free_pages(), [(pool.seq_len(s), list(pool.block_table(s))) for s in slots]


def test_reserve_batch_equals_sequential_reserves():
    """A batch (with a repeated slot and a zero count) hands out the same pages,
    in the same order, as the reserves it stands for, made one by one."""
    a, b = _twin_pools()
    rounds = [([0, 1, 2, 3, 4], [3, 1, 9, 0, 4]), ([2, 0, 2, 4], [2, 5, 7, 1]), ([1, 3], [16, 4])]
    for slots, counts in rounds:
        assert a.reserve_batch(slots, counts)
        for s, n in zip(slots, counts):
            assert b.reserve(s, n)[0]
        assert _state(a) == _state(b)
    assert a.seq_len(2) == 18 and len(a.block_table(2)) == 5


def test_reserve_batch_is_all_or_nothing():
    pool = pa_amd.PagePool(5, 4, 3, 8)
    s0, s1 = pool.admit(), pool.admit()
    assert pool.reserve_batch([s0, s1], [4, 5])            # 1 + 2 pages
    before = _state(pool, (s0, s1))
    assert not pool.reserve_batch([s0, s1], [5, 8])         # needs 2 + 2 more, 2 left
    assert _state(pool, (s0, s1)) == before
    assert pool.reserve_batch([s0, s1], [4, 4])             # 1 + 1: exactly the 2 left
    assert pool.free_pages() == 0


def test_reserve_batch_errors_change_nothing():
    pool = pa_amd.PagePool(20, 4, 3, 3)
    s0, s1 = pool.admit(), pool.admit()
    before = _state(pool, (s0, s1))
    with pytest.raises(pa_amd.LengthError, match="max_pages_per_slot"):
        pool.reserve_batch([s0, s1, s1], [4, 8, 5])           # s1 reaches 13 > 12 tokens on its 2nd entry
    with pytest.raises(pa_amd.InvalidArgument, match="not admitted"):
        pool.reserve_batch([s0, 2], [1, 1])
    with pytest.raises(pa_amd.InvalidArgument, match="negative"):
        pool.reserve_batch([s0, s1], [1, -1])
    assert _state(pool, (s0, s1)) == before
    assert pool.reserve_batch([], [])
