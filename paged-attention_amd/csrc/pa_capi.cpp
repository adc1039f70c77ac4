// C-ABI host layer of libpa_decode.so: the persistent planner, the device plan,
// the host page pool and the paged KV cache, over the gfx950 kernels in
// pa_kernels.hip. Every exported function catches exceptions and returns a
// pa_status (see pa_decode.h for the mapping to the reference's errors).

#include "pa_decode.h"
#include "pa_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <new>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

// Host copy of a schedule (decode.hpp:21-27 DecodePlan).
struct pa_plan {
    int num_ctas = 0;
    int tile     = 0;
    int items    = 0;
    std::vector<int32_t> segments;        // [n][4] = (row, kv head, tok_begin, tok_end)
    std::vector<int32_t> cta_seg_begin;   // [num_ctas + 1]
    std::vector<int32_t> item_seg_begin;  // [items + 1]
};

// Device copy of a plan plus the partial workspace (decode.hpp:44-63).
struct pa_device_plan {
    int32_t* segments       = nullptr;
    int32_t* cta_seg_begin  = nullptr;
    int32_t* item_seg_begin = nullptr;
    float*   partial_out    = nullptr;
    float*   partial_lse    = nullptr;
    size_t   seg_cap = 0, cta_cap = 0, item_cap = 0, part_cap = 0;
    int      num_ctas    = 0;
    int      needs_merge = 0;
    int      max_item_segments = 0;
    bool     block_merge = false;
};

// Host page allocator and per-slot block tables (paged_kv_cache.hpp:89-92).
struct pa_pool {
    int page_size          = 0;
    int max_slots          = 0;
    int max_pages_per_slot = 0;
    std::vector<int32_t>              free_pages;   // back() is handed out next
    std::vector<std::vector<int32_t>> tables;
    std::vector<int32_t>              seq_lens;
    std::vector<char>                 occupied;
};

// One host-to-device staging buffer of the batched append: pinned host ints,
// their device copy, and an event recorded after the kernel that reads them.
struct pa_stage {
    int32_t*   host = nullptr;
    int32_t*   dev  = nullptr;
    size_t     cap  = 0;   // int32 elements
    hipEvent_t done = nullptr;
};

struct pa_cache {
    pa_cache_config cfg{};
    pa_pool         pool;
    void*           d_k          = nullptr;
    void*           d_v          = nullptr;
    int32_t*        d_table      = nullptr;   // [max_slots][max_pages_per_slot]
    int32_t*        d_seq_lens   = nullptr;   // [max_slots]
    int32_t*        d_slot_ids   = nullptr;
    size_t          slot_ids_cap = 0;
    pa_plan         plan;
    pa_device_plan  dplan;
    int             plan_batch = 0;
    int             plan_hq    = 0;
    pa_stage        stage[2];   // used in turn, so one batch may still be in flight while the next is staged
    int             stage_next = 0;
};

namespace {

thread_local std::string g_last_error;

template <class F>
pa_status guarded(F&& f) {
    try {
        f();
        return PA_OK;
    } catch (const std::invalid_argument& e) {
        g_last_error = e.what();
        return PA_ERR_INVALID_ARGUMENT;
    } catch (const std::length_error& e) {
        g_last_error = e.what();
        return PA_ERR_LENGTH;
    } catch (const pa::DeviceError& e) {
        g_last_error = e.what();
        return PA_ERR_DEVICE;
    } catch (const std::bad_alloc&) {
        g_last_error = "host allocation failed";
        return PA_ERR_DEVICE;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return PA_ERR_DEVICE;
    }
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

void check_dtype(int dtype) {
    if (dtype != PA_KV_FP16 && dtype != PA_KV_FP8_E4M3)
        throw std::invalid_argument("unknown kv dtype " + std::to_string(dtype));
}

int group_of(int num_q_heads, int num_kv_heads) {
    if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0)
        throw std::invalid_argument("num_q_heads must be a multiple of num_kv_heads");
    return num_q_heads / num_kv_heads;
}

void check_shape(int dtype, int head_dim, int group) {
    check_dtype(dtype);
    if (head_dim != pa::kHeadDim) throw std::invalid_argument("unsupported head_dim " + std::to_string(head_dim));
    if (group != 1 && group != 2 && group != 4 && group != 8)
        throw std::invalid_argument("unsupported GQA group size " + std::to_string(group));
}

int device_cus() {
    int dev = 0, cus = 0;
    pa::hip_check(hipGetDevice(&dev), "hipGetDevice");
    pa::hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    return cus;
}

int wave_ctas_impl(int dtype, int head_dim, int group) {
    check_shape(dtype, head_dim, group);
    return device_cus() * pa::kernel_units_per_cu(dtype, group);
}

// The persistent cut (decode.cu:65-108): all (row, kv head) items are laid out
// in order as runs of `tile`-token tiles; the total is split into equal
// contiguous ranges of `per` tiles, one per work unit, and every maximal run of
// one item inside a range becomes a segment.
void cut(pa_plan& plan, int tile, const int32_t* lens, int batch, int hkv, int requested) {
    if (tile <= 0) throw std::invalid_argument("make_plan: tile must be positive");
    if (batch < 0 || hkv <= 0) throw std::invalid_argument("make_plan: bad batch or kv head count");
    if (batch > 0 && !lens) throw std::invalid_argument("make_plan: seq_lens is null");
    if (requested <= 0) throw std::invalid_argument("make_plan: num_ctas must be positive");
    plan = pa_plan{};
    plan.tile  = tile;
    plan.items = batch * hkv;

    std::vector<long> tiles_of(static_cast<size_t>(batch));
    long total = 0;
    for (int b = 0; b < batch; ++b) {
        if (lens[b] <= 0) throw std::invalid_argument("make_plan: every sequence needs at least one token");
        tiles_of[b] = (static_cast<long>(lens[b]) + tile - 1) / tile;
        total += tiles_of[b] * hkv;
    }
    plan.item_seg_begin.assign(static_cast<size_t>(plan.items) + 1, 0);
    if (total == 0) {
        plan.cta_seg_begin.push_back(0);
        return;
    }
    const long per = (total + requested - 1) / requested;
    plan.num_ctas = static_cast<int>((total + per - 1) / per);
    plan.cta_seg_begin.reserve(static_cast<size_t>(plan.num_ctas) + 1);

    int  item = 0;
    long done = 0;   // tiles of `item` already assigned
    for (int u = 0; u < plan.num_ctas; ++u) {
        plan.cta_seg_begin.push_back(static_cast<int32_t>(plan.segments.size() / 4));
        long budget = per;
        while (budget > 0 && item < plan.items) {
            const int  b     = item / hkv;
            const long avail = tiles_of[b] - done;
            const long take  = std::min(budget, avail);
            const long t0    = done * tile;
            const long t1    = std::min((done + take) * tile, static_cast<long>(lens[b]));
            plan.segments.insert(plan.segments.end(),
                                 {b, item % hkv, static_cast<int32_t>(t0), static_cast<int32_t>(t1)});
            plan.item_seg_begin[static_cast<size_t>(item) + 1] += 1;
            done += take;
            budget -= take;
            if (done == tiles_of[b]) {
                ++item;
                done = 0;
            }
        }
    }
    plan.cta_seg_begin.push_back(static_cast<int32_t>(plan.segments.size() / 4));
    for (int i = 0; i < plan.items; ++i) plan.item_seg_begin[i + 1] += plan.item_seg_begin[i];
}

void make_plan_impl(pa_plan& plan, int dtype, const int32_t* lens, int batch, int hq, int hkv, int hd,
                    int num_ctas) {
    const int group = group_of(hq, hkv);
    check_shape(dtype, hd, group);
    const int tile = pa::kernel_tile_tokens(dtype, group);
    if (num_ctas <= 0) num_ctas = wave_ctas_impl(dtype, hd, group);
    cut(plan, tile, lens, batch, hkv, num_ctas);
}

template <class T>
void upload_grow(T*& dst, size_t& cap, const T* src, size_t n, hipStream_t s) {
    if (n > cap) {
        pa::hip_check(hipFree(dst), "hipFree");
        dst = nullptr;
        pa::hip_check(hipMalloc(reinterpret_cast<void**>(&dst), sizeof(T) * n), "hipMalloc");
        cap = n;
    }
    if (n) pa::hip_check(hipMemcpyAsync(dst, src, sizeof(T) * n, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
}

void device_plan_upload(pa_device_plan& dp, const pa_plan& plan, int group, int head_dim, hipStream_t s) {
    if (group <= 0 || head_dim <= 0) throw std::invalid_argument("upload: bad group or head_dim");
    const size_t nseg = plan.segments.size() / 4;
    upload_grow(dp.segments, dp.seg_cap, plan.segments.data(), plan.segments.size(), s);
    upload_grow(dp.cta_seg_begin, dp.cta_cap, plan.cta_seg_begin.data(), plan.cta_seg_begin.size(), s);
    upload_grow(dp.item_seg_begin, dp.item_cap, plan.item_seg_begin.data(), plan.item_seg_begin.size(), s);
    const size_t rows = nseg * static_cast<size_t>(group);
    const size_t need = rows * (static_cast<size_t>(head_dim) + 1);
    if (need > dp.part_cap) {
        pa::hip_check(hipFree(dp.partial_out), "hipFree");
        dp.partial_out = nullptr;
        pa::hip_check(hipMalloc(reinterpret_cast<void**>(&dp.partial_out), sizeof(float) * need), "hipMalloc");
        dp.part_cap = need;
    }
    dp.partial_lse = dp.partial_out ? dp.partial_out + rows * head_dim : nullptr;
    dp.num_ctas = plan.num_ctas;
    // Block-level merge: the split kernel merges a split row itself when all
    // its segments lie in one block of kBlockUnits units. It needs every split
    // segment to be its unit's first or last (true of every make_plan cut) and
    // is used when it covers every split row, so no merge launch remains.
    bool block_merge = nseg > static_cast<size_t>(plan.items);
    if (block_merge) {
        std::vector<int32_t> unit_of(nseg, 0);
        for (int u = 0; u < plan.num_ctas; ++u)
            for (int sg = plan.cta_seg_begin[u]; sg < plan.cta_seg_begin[u + 1]; ++sg)
                unit_of[static_cast<size_t>(sg)] = u;
        for (int i = 0; i < plan.items && block_merge; ++i) {
            const int a = plan.item_seg_begin[i], z = plan.item_seg_begin[i + 1];
            if (z - a <= 1) continue;
            if (unit_of[static_cast<size_t>(a)] / pa::kBlockUnits != unit_of[static_cast<size_t>(z - 1)] / pa::kBlockUnits)
                block_merge = false;   // the row spans blocks
            for (int sg = a; sg < z && block_merge; ++sg) {
                const int u = unit_of[static_cast<size_t>(sg)];
                if (sg != plan.cta_seg_begin[u] && sg != plan.cta_seg_begin[u + 1] - 1)
                    block_merge = false;   // a split segment inside a unit
            }
        }
    }
    dp.block_merge = block_merge;
    dp.needs_merge = !block_merge && nseg > static_cast<size_t>(plan.items) ? 1 : 0;
    dp.max_item_segments = 0;
    for (int i = 0; i < plan.items; ++i)
        dp.max_item_segments = std::max(dp.max_item_segments, plan.item_seg_begin[i + 1] - plan.item_seg_begin[i]);
    // The sources are host vectors the caller may free or rebuild right away.
    pa::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

void device_plan_bind(const pa_device_plan& dp, pa_decode_params& p) {
    p.segments       = dp.segments;
    p.cta_seg_begin  = dp.cta_seg_begin;
    p.item_seg_begin = dp.item_seg_begin;
    p.num_ctas       = dp.num_ctas;
    p.needs_merge    = dp.needs_merge;
    p.partial_out    = dp.partial_out;
    p.partial_lse    = dp.partial_lse;
    p.max_item_segments = dp.max_item_segments;
    p.block_merge       = dp.block_merge ? 1 : 0;
}

void device_plan_free(pa_device_plan& dp) {
    (void)hipFree(dp.segments);
    (void)hipFree(dp.cta_seg_begin);
    (void)hipFree(dp.item_seg_begin);
    (void)hipFree(dp.partial_out);
    dp = pa_device_plan{};
}

void decode_impl(int dtype, const pa_decode_params& p, hipStream_t s, bool split, bool merge) {
    if (split) pa::hip_check(pa::launch_decode_split(dtype, p, s), "decode split kernel launch");
    if (merge) pa::hip_check(pa::launch_decode_merge(dtype, p, s), "decode merge kernel launch");
}

void pool_init(pa_pool& pool, int num_pages, int page_size, int max_slots, int max_pages_per_slot) {
    if (num_pages <= 0 || page_size <= 0 || max_slots <= 0 || max_pages_per_slot <= 0)
        throw std::invalid_argument("PagedKVCache: all sizes must be positive");
    pool.page_size          = page_size;
    pool.max_slots          = max_slots;
    pool.max_pages_per_slot = max_pages_per_slot;
    pool.free_pages.resize(static_cast<size_t>(num_pages));
    // Popped from the back, so page 0 is handed out first.
    std::iota(pool.free_pages.rbegin(), pool.free_pages.rend(), 0);
    pool.tables.assign(static_cast<size_t>(max_slots), {});
    pool.seq_lens.assign(static_cast<size_t>(max_slots), 0);
    pool.occupied.assign(static_cast<size_t>(max_slots), 0);
}

bool slot_ok(const pa_pool& pool, int slot) {
    return slot >= 0 && slot < pool.max_slots && pool.occupied[static_cast<size_t>(slot)];
}

int pool_admit(pa_pool& pool) {
    for (int s = 0; s < pool.max_slots; ++s) {
        if (!pool.occupied[static_cast<size_t>(s)]) {
            pool.occupied[static_cast<size_t>(s)] = 1;
            pool.seq_lens[static_cast<size_t>(s)] = 0;
            return s;
        }
    }
    return -1;
}

// Append bookkeeping: returns false (nothing changed) when out of pages.
bool pool_reserve(pa_pool& pool, int slot, int n, int& first_new, int& num_new) {
    if (!slot_ok(pool, slot)) throw std::invalid_argument("append: slot is not admitted");
    auto& table = pool.tables[static_cast<size_t>(slot)];
    first_new   = static_cast<int>(table.size());
    num_new     = 0;
    if (n <= 0) return true;
    const long new_len = static_cast<long>(pool.seq_lens[static_cast<size_t>(slot)]) + n;
    const long need    = (new_len + pool.page_size - 1) / pool.page_size;
    if (need > pool.max_pages_per_slot) throw std::length_error("append: sequence exceeds max_pages_per_slot");
    const long grow = need - static_cast<long>(table.size());
    if (grow > static_cast<long>(pool.free_pages.size())) return false;
    for (long i = 0; i < grow; ++i) {
        table.push_back(pool.free_pages.back());
        pool.free_pages.pop_back();
    }
    pool.seq_lens[static_cast<size_t>(slot)] = static_cast<int32_t>(new_len);
    num_new = static_cast<int>(grow);
    return true;
}

// Entry i of a batched append: the slot's length before it, and the table
// entries it added.
struct reserve_entry {
    int old_len   = 0;
    int first_new = 0;
    int num_new   = 0;
};

// Batched append bookkeeping: the same as pool_reserve(slots[i], counts[i])
// for i = 0..n-1 in order (a slot may repeat), except all-or-nothing: returns
// false with nothing changed when the pool lacks pages for the whole batch, and
// throws before changing anything for a bad slot, a negative count or a slot
// that would exceed max_pages_per_slot.
bool pool_reserve_batch(pa_pool& pool, const int32_t* slots, const int32_t* counts, int n,
                        std::vector<reserve_entry>* entries) {
    if (n < 0) throw std::invalid_argument("append_batch: negative batch size");
    if (n > 0 && (!slots || !counts)) throw std::invalid_argument("append_batch: slots or counts is null");
    std::vector<long> len(pool.seq_lens.begin(), pool.seq_lens.end());
    std::vector<long> pages(static_cast<size_t>(pool.max_slots));
    for (int s = 0; s < pool.max_slots; ++s) pages[static_cast<size_t>(s)] = static_cast<long>(pool.tables[static_cast<size_t>(s)].size());
    long grow = 0;
    for (int i = 0; i < n; ++i) {
        if (!slot_ok(pool, slots[i])) throw std::invalid_argument("append_batch: slot is not admitted");
        if (counts[i] < 0) throw std::invalid_argument("append_batch: negative token count");
        const size_t s = static_cast<size_t>(slots[i]);
        len[s] += counts[i];
        const long need = (len[s] + pool.page_size - 1) / pool.page_size;
        if (need > pool.max_pages_per_slot) throw std::length_error("append_batch: sequence exceeds max_pages_per_slot");
        if (need > pages[s]) {
            grow += need - pages[s];
            pages[s] = need;
        }
    }
    if (grow > static_cast<long>(pool.free_pages.size())) return false;
    if (entries) entries->assign(static_cast<size_t>(n), reserve_entry{});
    for (int i = 0; i < n; ++i) {
        reserve_entry e;
        e.old_len = pool.seq_lens[static_cast<size_t>(slots[i])];
        pool_reserve(pool, slots[i], counts[i], e.first_new, e.num_new);
        if (entries) (*entries)[static_cast<size_t>(i)] = e;
    }
    return true;
}

void pool_release(pa_pool& pool, int slot) {
    if (!slot_ok(pool, slot)) throw std::invalid_argument("release: slot is not admitted");
    auto& table = pool.tables[static_cast<size_t>(slot)];
    for (int32_t page : table) pool.free_pages.push_back(page);
    table.clear();
    pool.seq_lens[static_cast<size_t>(slot)] = 0;
    pool.occupied[static_cast<size_t>(slot)] = 0;
}

size_t bytes_per_page_impl(const pa_cache_config& cfg) {
    const int eb = cfg.dtype == PA_KV_FP8_E4M3 ? 1 : 2;
    return 2ull * static_cast<size_t>(cfg.num_kv_heads) * static_cast<size_t>(cfg.page_size) *
           static_cast<size_t>(cfg.head_dim) * static_cast<size_t>(eb);
}

void cache_params(const pa_cache& c, pa_decode_params& p) {
    p = pa_decode_params{};
    p.k_cache            = c.d_k;
    p.v_cache            = c.d_v;
    p.block_table        = c.d_table;
    p.seq_lens           = c.d_seq_lens;
    p.block_table_stride = c.cfg.max_pages_per_slot;
    p.num_kv_heads       = c.cfg.num_kv_heads;
    p.head_dim           = c.cfg.head_dim;
    p.page_size          = c.cfg.page_size;
    p.sm_scale           = 1.0f / std::sqrt(static_cast<float>(c.cfg.head_dim));
    const bool fp8       = c.cfg.dtype == PA_KV_FP8_E4M3;
    p.k_scale            = fp8 ? c.cfg.k_scale : 1.0f;
    p.v_scale            = fp8 ? c.cfg.v_scale : 1.0f;
}

void cache_plan(pa_cache& c, const int32_t* slots, int n, int hq, int num_ctas, hipStream_t s) {
    if (n < 0 || (n > 0 && !slots)) throw std::invalid_argument("plan: bad slot list");
    std::vector<int32_t> lens(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) {
        if (!slot_ok(c.pool, slots[i])) throw std::invalid_argument("plan: slot is not admitted");
        lens[static_cast<size_t>(i)] = c.pool.seq_lens[static_cast<size_t>(slots[i])];
    }
    make_plan_impl(c.plan, c.cfg.dtype, lens.data(), n, hq, c.cfg.num_kv_heads, c.cfg.head_dim, num_ctas);
    device_plan_upload(c.dplan, c.plan, hq / c.cfg.num_kv_heads, c.cfg.head_dim, s);
    upload_grow(c.d_slot_ids, c.slot_ids_cap, slots, static_cast<size_t>(n), s);
    pa::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    c.plan_batch = n;
    c.plan_hq    = hq;
}

void cache_run(pa_cache& c, const uint16_t* q, uint16_t* out, hipStream_t s) {
    pa_decode_params p;
    cache_params(c, p);
    p.q           = q;
    p.out         = out;
    p.slot_ids    = c.d_slot_ids;
    p.batch       = c.plan_batch;
    p.num_q_heads = c.plan_hq;
    device_plan_bind(c.dplan, p);
    decode_impl(c.cfg.dtype, p, s, true, true);
}

}  // namespace

extern "C" {

const char* pa_last_error(void) { return g_last_error.c_str(); }

int pa_kv_dtype_bytes(int dtype) { return dtype == PA_KV_FP16 ? 2 : 1; }
const char* pa_kv_dtype_name(int dtype) { return dtype == PA_KV_FP16 ? "fp16" : "fp8_e4m3"; }

pa_status pa_tile_tokens(int dtype, int head_dim, int group, int* out) {
    return guarded([&] {
        check_shape(dtype, head_dim, group);
        if (!out) throw std::invalid_argument("out is null");
        *out = pa::kernel_tile_tokens(dtype, group);
    });
}

pa_status pa_wave_ctas(int dtype, int head_dim, int group, int* out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("out is null");
        *out = wave_ctas_impl(dtype, head_dim, group);
    });
}

pa_status pa_default_ctas(int dtype, int head_dim, int group, int* out) {
    // One full wave: every resident work unit gets one equal range.
    return pa_wave_ctas(dtype, head_dim, group, out);
}

pa_status pa_plan_build(int dtype, const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                        int head_dim, int num_ctas, pa_plan** out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("out is null");
        auto* plan = new pa_plan;
        try {
            make_plan_impl(*plan, dtype, seq_lens, batch, num_q_heads, num_kv_heads, head_dim, num_ctas);
        } catch (...) {
            delete plan;
            throw;
        }
        *out = plan;
    });
}

pa_status pa_plan_build_tiled(int tile, const int32_t* seq_lens, int batch, int num_kv_heads, int num_ctas,
                              pa_plan** out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("out is null");
        auto* plan = new pa_plan;
        try {
            cut(*plan, tile, seq_lens, batch, num_kv_heads, num_ctas);
        } catch (...) {
            delete plan;
            throw;
        }
        *out = plan;
    });
}

pa_status pa_plan_create(int num_ctas, int tile, const int32_t* segments, int num_segments,
                         const int32_t* cta_seg_begin, const int32_t* item_seg_begin, int num_items,
                         int num_kv_heads, pa_plan** out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("out is null");
        if (num_ctas < 0 || num_segments < 0 || num_items < 0 || tile <= 0 || num_kv_heads < 0)
            throw std::invalid_argument("plan: negative sizes or non-positive tile");
        if ((num_segments && !segments) || !cta_seg_begin || !item_seg_begin)
            throw std::invalid_argument("plan: null array");
        if (num_kv_heads == 0) {   // every (row, kv head) has a segment, so the heads are 0 .. max
            for (int i = 0; i < num_segments; ++i) num_kv_heads = std::max(num_kv_heads, segments[4 * i + 1] + 1);
            num_kv_heads = std::max(num_kv_heads, 1);
        }
        if (num_items % num_kv_heads != 0) throw std::invalid_argument("plan: items must be batch * num_kv_heads");
        auto prefix_ok = [&](const int32_t* a, int n) {
            if (a[0] != 0 || a[n] != num_segments) return false;
            for (int i = 0; i < n; ++i)
                if (a[i + 1] < a[i]) return false;
            return true;
        };
        if (!prefix_ok(cta_seg_begin, num_ctas) || !prefix_ok(item_seg_begin, num_items))
            throw std::invalid_argument("plan: segment prefix arrays must rise from 0 to num_segments");
        for (int i = 0; i < num_items; ++i)
            if (item_seg_begin[i + 1] == item_seg_begin[i])
                throw std::invalid_argument("plan: every (row, kv head) needs a segment");
        for (int i = 0; i < num_segments; ++i) {
            const int32_t* sg = segments + 4 * static_cast<size_t>(i);
            const long item = static_cast<long>(sg[0]) * num_kv_heads + sg[1];
            if (sg[0] < 0 || sg[1] < 0 || sg[1] >= num_kv_heads || item >= num_items)
                throw std::invalid_argument("plan: segment row / kv head out of range");
            if (sg[2] < 0 || sg[3] <= sg[2]) throw std::invalid_argument("plan: empty or negative segment");
            if (i < item_seg_begin[item] || i >= item_seg_begin[item + 1])
                throw std::invalid_argument("plan: segment is not listed under its (row, kv head)");
        }
        auto* plan = new pa_plan;
        plan->num_ctas = num_ctas;
        plan->tile     = tile;
        plan->items    = num_items;
        plan->segments.assign(segments, segments + 4 * static_cast<size_t>(num_segments));
        plan->cta_seg_begin.assign(cta_seg_begin, cta_seg_begin + num_ctas + 1);
        plan->item_seg_begin.assign(item_seg_begin, item_seg_begin + num_items + 1);
        *out = plan;
    });
}

void pa_plan_destroy(pa_plan* plan) { delete plan; }
int  pa_plan_num_ctas(const pa_plan* plan) { return plan ? plan->num_ctas : 0; }
int  pa_plan_tile(const pa_plan* plan) { return plan ? plan->tile : 0; }
int  pa_plan_num_segments(const pa_plan* plan) { return plan ? static_cast<int>(plan->segments.size() / 4) : 0; }
int  pa_plan_num_items(const pa_plan* plan) { return plan ? plan->items : 0; }

pa_status pa_plan_copy(const pa_plan* plan, int32_t* segments, int32_t* cta_seg_begin, int32_t* item_seg_begin) {
    return guarded([&] {
        if (!plan) throw std::invalid_argument("plan is null");
        if (segments) std::copy(plan->segments.begin(), plan->segments.end(), segments);
        if (cta_seg_begin) std::copy(plan->cta_seg_begin.begin(), plan->cta_seg_begin.end(), cta_seg_begin);
        if (item_seg_begin) std::copy(plan->item_seg_begin.begin(), plan->item_seg_begin.end(), item_seg_begin);
    });
}

pa_status pa_device_plan_create(pa_device_plan** out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("out is null");
        *out = new pa_device_plan;
    });
}

void pa_device_plan_destroy(pa_device_plan* dp) {
    if (!dp) return;
    device_plan_free(*dp);
    delete dp;
}

pa_status pa_device_plan_upload(pa_device_plan* dp, const pa_plan* plan, int group, int head_dim, void* stream) {
    return guarded([&] {
        if (!dp || !plan) throw std::invalid_argument("device plan or plan is null");
        device_plan_upload(*dp, *plan, group, head_dim, as_stream(stream));
    });
}

pa_status pa_device_plan_bind(const pa_device_plan* dp, pa_decode_params* p) {
    return guarded([&] {
        if (!dp || !p) throw std::invalid_argument("device plan or params is null");
        device_plan_bind(*dp, *p);
    });
}

pa_status pa_decode(int dtype, const pa_decode_params* p, void* stream) {
    return guarded([&] {
        if (!p) throw std::invalid_argument("params is null");
        decode_impl(dtype, *p, as_stream(stream), true, true);
    });
}

pa_status pa_decode_split(int dtype, const pa_decode_params* p, void* stream) {
    return guarded([&] {
        if (!p) throw std::invalid_argument("params is null");
        decode_impl(dtype, *p, as_stream(stream), true, false);
    });
}

pa_status pa_decode_merge(int dtype, const pa_decode_params* p, void* stream) {
    return guarded([&] {
        if (!p) throw std::invalid_argument("params is null");
        decode_impl(dtype, *p, as_stream(stream), false, true);
    });
}

pa_status pa_append_quantize(int dtype, const uint16_t* k, const uint16_t* v, void* k_cache, void* v_cache,
                             const int32_t* block_table_row, int start_pos, int n, int num_kv_heads, int head_dim,
                             int page_size, float inv_k_scale, float inv_v_scale, void* stream) {
    return guarded([&] {
        check_dtype(dtype);
        if (head_dim != pa::kHeadDim) throw std::invalid_argument("unsupported head_dim " + std::to_string(head_dim));
        if (num_kv_heads <= 0 || page_size <= 0 || start_pos < 0 || n < 0)
            throw std::invalid_argument("append: bad sizes");
        if (n > 0 && (!k || !v || !k_cache || !v_cache || !block_table_row))
            throw std::invalid_argument("append: null pointer");
        pa::hip_check(pa::launch_append(dtype, k, v, k_cache, v_cache, block_table_row, start_pos, n, num_kv_heads,
                                        page_size, inv_k_scale, inv_v_scale, as_stream(stream)),
                      "append kernel launch");
    });
}

pa_status pa_gather_kv(int dtype, const void* cache, const int32_t* block_table_row, int num_kv_heads, int head_dim,
                       int page_size, int kv_head, int len, void* out, void* stream) {
    return guarded([&] {
        check_dtype(dtype);
        if (head_dim != pa::kHeadDim) throw std::invalid_argument("unsupported head_dim " + std::to_string(head_dim));
        if (num_kv_heads <= 0 || page_size <= 0 || kv_head < 0 || kv_head >= num_kv_heads || len < 0)
            throw std::invalid_argument("gather: bad sizes");
        pa::hip_check(pa::launch_gather(dtype, cache, block_table_row, num_kv_heads, page_size, kv_head, len, out,
                                        as_stream(stream)),
                      "gather kernel launch");
    });
}

pa_status pa_stream_read(const void* buf, size_t bytes, int blocks, uint32_t* sink, void* stream) {
    return pa_stream_read_ex(buf, bytes, blocks, 256, 1, 0, sink, stream);
}

pa_status pa_stream_read_chunked(const void* buf, size_t bytes, int blocks, int threads, int unroll, uint32_t* sink,
                                 void* stream) {
    return guarded([&] {
        if (!buf || !sink) throw std::invalid_argument("stream_read_chunked: null pointer");
        pa::hip_check(pa::launch_stream_read_chunked(buf, bytes, blocks, threads, unroll, sink, as_stream(stream)),
                      "stream_read_chunked launch");
    });
}

pa_status pa_stream_read_ex(const void* buf, size_t bytes, int blocks, int threads, int unroll, int nontemporal,
                            uint32_t* sink, void* stream) {
    return guarded([&] {
        if (bytes % 16 != 0 || blocks <= 0 || !buf || !sink) throw std::invalid_argument("stream_read: bad arguments");
        pa::hip_check(pa::launch_stream_read(buf, bytes, blocks, threads, unroll, nontemporal != 0, sink,
                                             as_stream(stream)),
                      "read kernel launch");
    });
}

pa_status pa_fill_bytes(void* buf, size_t bytes, int value, void* stream) {
    return guarded([&] {
        if (bytes % 16 != 0 || (bytes && !buf)) throw std::invalid_argument("fill_bytes: bad arguments");
        pa::hip_check(pa::launch_fill_bytes(buf, bytes, value, as_stream(stream)), "fill kernel launch");
    });
}

// ---- pool

pa_status pa_pool_create(int num_pages, int page_size, int max_slots, int max_pages_per_slot, pa_pool** out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("out is null");
        auto* pool = new pa_pool;
        try {
            pool_init(*pool, num_pages, page_size, max_slots, max_pages_per_slot);
        } catch (...) {
            delete pool;
            throw;
        }
        *out = pool;
    });
}

void pa_pool_destroy(pa_pool* pool) { delete pool; }
int  pa_pool_admit(pa_pool* pool) { return pool ? pool_admit(*pool) : -1; }

pa_status pa_pool_reserve(pa_pool* pool, int slot, int n, int* ok, int* first_new, int* num_new) {
    return guarded([&] {
        if (!pool) throw std::invalid_argument("pool is null");
        int f = 0, m = 0;
        const bool r = pool_reserve(*pool, slot, n, f, m);
        if (ok) *ok = r ? 1 : 0;
        if (first_new) *first_new = f;
        if (num_new) *num_new = m;
    });
}

pa_status pa_pool_reserve_batch(pa_pool* pool, const int32_t* slots, const int32_t* counts, int n, int* ok) {
    return guarded([&] {
        if (!pool) throw std::invalid_argument("pool is null");
        const bool r = pool_reserve_batch(*pool, slots, counts, n, nullptr);
        if (ok) *ok = r ? 1 : 0;
    });
}

pa_status pa_pool_release(pa_pool* pool, int slot) {
    return guarded([&] {
        if (!pool) throw std::invalid_argument("pool is null");
        pool_release(*pool, slot);
    });
}

void pa_pool_shuffle_free_pages(pa_pool* pool, unsigned seed) {
    if (!pool) return;
    std::mt19937 rng(seed);
    std::shuffle(pool->free_pages.begin(), pool->free_pages.end(), rng);
}

int pa_pool_free_pages(const pa_pool* pool) { return pool ? static_cast<int>(pool->free_pages.size()) : 0; }
int pa_pool_seq_len(const pa_pool* pool, int slot) {
    return pool && slot >= 0 && slot < pool->max_slots ? pool->seq_lens[static_cast<size_t>(slot)] : 0;
}
int pa_pool_occupied(const pa_pool* pool, int slot) {
    return pool && slot >= 0 && slot < pool->max_slots ? pool->occupied[static_cast<size_t>(slot)] : 0;
}
int pa_pool_max_seq_len(const pa_pool* pool) {
    if (!pool || pool->seq_lens.empty()) return 0;
    return *std::max_element(pool->seq_lens.begin(), pool->seq_lens.end());
}
int pa_pool_num_pages_of(const pa_pool* pool, int slot) {
    return pool && slot >= 0 && slot < pool->max_slots
               ? static_cast<int>(pool->tables[static_cast<size_t>(slot)].size())
               : 0;
}

pa_status pa_pool_block_table(const pa_pool* pool, int slot, int32_t* out, int cap) {
    return guarded([&] {
        if (!pool || slot < 0 || slot >= pool->max_slots) throw std::invalid_argument("block_table: bad slot");
        const auto& t = pool->tables[static_cast<size_t>(slot)];
        const size_t n = std::min(t.size(), static_cast<size_t>(std::max(cap, 0)));
        if (n && !out) throw std::invalid_argument("out is null");
        std::copy(t.begin(), t.begin() + static_cast<long>(n), out);
    });
}

// ---- cache

size_t pa_cache_bytes_per_page(const pa_cache_config* cfg) { return cfg ? bytes_per_page_impl(*cfg) : 0; }

int pa_cache_pages_for_budget(const pa_cache_config* cfg, size_t budget_bytes) {
    if (!cfg) return 0;
    const size_t per = bytes_per_page_impl(*cfg);
    return per ? static_cast<int>(budget_bytes / per) : 0;
}

pa_status pa_cache_create(const pa_cache_config* cfg, pa_cache** out) {
    return guarded([&] {
        if (!cfg || !out) throw std::invalid_argument("config or out is null");
        check_dtype(cfg->dtype);
        if (cfg->num_pages <= 0 || cfg->page_size <= 0 || cfg->num_kv_heads <= 0 || cfg->max_slots <= 0 ||
            cfg->max_pages_per_slot <= 0)
            throw std::invalid_argument("PagedKVCache: all sizes must be positive");
        if (cfg->head_dim != pa::kHeadDim) throw std::invalid_argument("PagedKVCache: head_dim must be 128");
        auto* c = new pa_cache;
        try {
            c->cfg = *cfg;
            pool_init(c->pool, cfg->num_pages, cfg->page_size, cfg->max_slots, cfg->max_pages_per_slot);
            const size_t half_bytes = bytes_per_page_impl(*cfg) / 2 * static_cast<size_t>(cfg->num_pages);
            const size_t table = sizeof(int32_t) * static_cast<size_t>(cfg->max_slots) * cfg->max_pages_per_slot;
            pa::hip_check(hipMalloc(&c->d_k, half_bytes), "hipMalloc k pool");
            pa::hip_check(hipMalloc(&c->d_v, half_bytes), "hipMalloc v pool");
            pa::hip_check(hipMalloc(reinterpret_cast<void**>(&c->d_table), table), "hipMalloc block table");
            pa::hip_check(hipMalloc(reinterpret_cast<void**>(&c->d_seq_lens), sizeof(int32_t) * cfg->max_slots),
                          "hipMalloc seq_lens");
            pa::hip_check(hipMemset(c->d_table, 0, table), "hipMemset");
            pa::hip_check(hipMemset(c->d_seq_lens, 0, sizeof(int32_t) * cfg->max_slots), "hipMemset");
        } catch (...) {
            (void)hipFree(c->d_k);
            (void)hipFree(c->d_v);
            (void)hipFree(c->d_table);
            (void)hipFree(c->d_seq_lens);
            delete c;
            throw;
        }
        *out = c;
    });
}

void pa_cache_destroy(pa_cache* c) {
    if (!c) return;
    (void)hipFree(c->d_k);
    (void)hipFree(c->d_v);
    (void)hipFree(c->d_table);
    (void)hipFree(c->d_seq_lens);
    (void)hipFree(c->d_slot_ids);
    for (pa_stage& st : c->stage) {
        if (st.done) (void)hipEventSynchronize(st.done);
        (void)hipHostFree(st.host);
        (void)hipFree(st.dev);
        if (st.done) (void)hipEventDestroy(st.done);
    }
    device_plan_free(c->dplan);
    delete c;
}

pa_pool* pa_cache_pool(pa_cache* c) { return c ? &c->pool : nullptr; }
int      pa_cache_admit(pa_cache* c) { return c ? pool_admit(c->pool) : -1; }

pa_status pa_cache_append(pa_cache* c, int slot, const uint16_t* d_k, const uint16_t* d_v, int n, void* stream,
                          int* appended) {
    return guarded([&] {
        if (!c) throw std::invalid_argument("cache is null");
        if (appended) *appended = 0;
        const int old_len = slot_ok(c->pool, slot) ? c->pool.seq_lens[static_cast<size_t>(slot)] : 0;
        int first_new = 0, num_new = 0;
        if (!pool_reserve(c->pool, slot, n, first_new, num_new)) return;   // out of pages: nothing appended
        if (appended) *appended = 1;
        if (n <= 0) return;
        const hipStream_t s = as_stream(stream);
        int32_t* row = c->d_table + static_cast<size_t>(slot) * c->cfg.max_pages_per_slot;
        const auto& table = c->pool.tables[static_cast<size_t>(slot)];
        if (num_new > 0)
            pa::hip_check(hipMemcpyAsync(row + first_new, table.data() + first_new, sizeof(int32_t) * num_new,
                                         hipMemcpyHostToDevice, s),
                          "hipMemcpyAsync block table");
        pa::hip_check(hipMemcpyAsync(c->d_seq_lens + slot, &c->pool.seq_lens[static_cast<size_t>(slot)],
                                     sizeof(int32_t), hipMemcpyHostToDevice, s),
                      "hipMemcpyAsync seq_len");
        const bool fp8 = c->cfg.dtype == PA_KV_FP8_E4M3;
        const float inv_k = fp8 ? 1.0f / c->cfg.k_scale : 1.0f;
        const float inv_v = fp8 ? 1.0f / c->cfg.v_scale : 1.0f;
        pa::hip_check(pa::launch_append(c->cfg.dtype, d_k, d_v, c->d_k, c->d_v, row, old_len, n, c->cfg.num_kv_heads,
                                        c->cfg.page_size, inv_k, inv_v, s),
                      "append kernel launch");
        // The copies above read host memory the next call may change.
        pa::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    });
}

namespace {

// Takes the next staging buffer with room for `need` ints, waiting for the
// batch that last used it (its copy and kernel) to finish.
pa_stage& take_stage(pa_cache& c, size_t need) {
    pa_stage& st = c.stage[c.stage_next];
    c.stage_next ^= 1;
    if (!st.done) pa::hip_check(hipEventCreateWithFlags(&st.done, hipEventDisableTiming), "hipEventCreate");
    pa::hip_check(hipEventSynchronize(st.done), "hipEventSynchronize staging");
    if (st.cap < need) {
        const size_t cap = std::max<size_t>(need + need / 2, 4096);
        (void)hipHostFree(st.host);
        (void)hipFree(st.dev);
        st.host = nullptr;
        st.dev  = nullptr;
        st.cap  = 0;
        pa::hip_check(hipHostMalloc(reinterpret_cast<void**>(&st.host), cap * sizeof(int32_t), hipHostMallocDefault),
                      "hipHostMalloc staging");
        pa::hip_check(hipMalloc(reinterpret_cast<void**>(&st.dev), cap * sizeof(int32_t)), "hipMalloc staging");
        st.cap = cap;
    }
    return st;
}

}  // namespace

pa_status pa_cache_append_batch(pa_cache* c, const int32_t* slots, const int32_t* counts, int n, const uint16_t* d_k,
                                const uint16_t* d_v, void* stream, int* appended) {
    return guarded([&] {
        if (!c) throw std::invalid_argument("cache is null");
        if (appended) *appended = 0;
        long n_tok = 0;
        for (int i = 0; i < n && counts; ++i) n_tok += counts[i] > 0 ? counts[i] : 0;
        const int hkv = c->cfg.num_kv_heads;
        if (n_tok * hkv * (pa::kHeadDim / 8) > INT_MAX) throw std::length_error("append_batch: too many tokens");
        if (n_tok > 0 && (!d_k || !d_v)) throw std::invalid_argument("append_batch: k or v is null");
        std::vector<reserve_entry> entries;
        if (!pool_reserve_batch(c->pool, slots, counts, n, &entries)) return;   // out of pages: nothing appended
        if (appended) *appended = 1;
        if (n_tok == 0) return;

        // Staging (layout of pa::AppendBatch::meta): per entry its first
        // token, old length and page-list start; the page lists; the new table
        // entries; one (slot, length) per distinct slot.
        const int P = c->cfg.page_size;
        long n_tab = 0, n_pl = 0;
        for (int i = 0; i < n; ++i) {
            const reserve_entry& e = entries[static_cast<size_t>(i)];
            n_tab += e.num_new;
            if (counts[i] > 0) n_pl += (e.old_len + counts[i] - 1) / P - e.old_len / P + 1;
        }
        std::vector<char> seen(static_cast<size_t>(c->cfg.max_slots), 0);
        long n_len = 0;
        for (int i = 0; i < n; ++i)
            if (!seen[static_cast<size_t>(slots[i])]) seen[static_cast<size_t>(slots[i])] = 1, ++n_len;
        const size_t need = 3 * static_cast<size_t>(n) + static_cast<size_t>(n_pl) + 2 * static_cast<size_t>(n_tab + n_len);
        pa_stage& st = take_stage(*c, need);
        int32_t* tok_begin = st.host;
        int32_t* old_len   = tok_begin + n;
        int32_t* pl_begin  = old_len + n;
        int32_t* pages     = pl_begin + n;
        int32_t* tab       = pages + n_pl;
        int32_t* lens      = tab + 2 * n_tab;
        int32_t  tok = 0, pl = 0;
        for (int i = 0; i < n; ++i) {
            const auto& table = c->pool.tables[static_cast<size_t>(slots[i])];
            const reserve_entry& e = entries[static_cast<size_t>(i)];
            tok_begin[i] = tok;
            old_len[i]   = e.old_len;
            pl_begin[i]  = pl;
            tok += counts[i];
            if (counts[i] > 0)
                for (int k = e.old_len / P; k <= (e.old_len + counts[i] - 1) / P; ++k) pages[pl++] = table[static_cast<size_t>(k)];
            for (int k = e.first_new; k < e.first_new + e.num_new; ++k) {
                *tab++ = slots[i] * c->cfg.max_pages_per_slot + k;
                *tab++ = table[static_cast<size_t>(k)];
            }
        }
        for (int i = 0; i < n; ++i) {
            const size_t sl = static_cast<size_t>(slots[i]);
            if (seen[sl] != 1) continue;
            seen[sl] = 2;
            *lens++ = slots[i];
            *lens++ = c->pool.seq_lens[sl];
        }

        const hipStream_t s = as_stream(stream);
        pa::hip_check(hipMemcpyAsync(st.dev, st.host, need * sizeof(int32_t), hipMemcpyHostToDevice, s),
                      "hipMemcpyAsync append staging");
        const bool fp8 = c->cfg.dtype == PA_KV_FP8_E4M3;
        pa::AppendBatch a{};
        a.k = d_k;
        a.v = d_v;
        a.k_cache = c->d_k;
        a.v_cache = c->d_v;
        a.meta = st.dev;
        a.table = c->d_table;
        a.seq_lens = c->d_seq_lens;
        a.n_ent = n;
        a.n_pl = static_cast<int>(n_pl);
        a.n_tab = static_cast<int>(n_tab);
        a.n_len = static_cast<int>(n_len);
        a.n_tok = static_cast<int>(n_tok);
        a.hkv = hkv;
        a.page_size = P;
        a.inv_k = fp8 ? 1.0f / c->cfg.k_scale : 1.0f;
        a.inv_v = fp8 ? 1.0f / c->cfg.v_scale : 1.0f;
        pa::hip_check(pa::launch_append_batch(c->cfg.dtype, a, s), "append_batch kernel launch");
        pa::hip_check(hipEventRecord(st.done, s), "hipEventRecord staging");
    });
}

pa_status pa_cache_release(pa_cache* c, int slot) {
    return guarded([&] {
        if (!c) throw std::invalid_argument("cache is null");
        pool_release(c->pool, slot);
        // A batched append still in flight may write this slot's length.
        for (pa_stage& st : c->stage)
            if (st.done) pa::hip_check(hipEventSynchronize(st.done), "hipEventSynchronize staging");
        pa::hip_check(hipMemset(c->d_seq_lens + slot, 0, sizeof(int32_t)), "hipMemset seq_len");
    });
}

void pa_cache_shuffle_free_pages(pa_cache* c, unsigned seed) {
    if (c) pa_pool_shuffle_free_pages(&c->pool, seed);
}

pa_status pa_cache_params(const pa_cache* c, pa_decode_params* p) {
    return guarded([&] {
        if (!c || !p) throw std::invalid_argument("cache or params is null");
        cache_params(*c, *p);
    });
}

pa_status pa_cache_plan(pa_cache* c, const int32_t* slots, int n, int num_q_heads, int num_ctas, void* stream) {
    return guarded([&] {
        if (!c) throw std::invalid_argument("cache is null");
        cache_plan(*c, slots, n, num_q_heads, num_ctas, as_stream(stream));
    });
}

pa_status pa_cache_run(pa_cache* c, const uint16_t* d_q, uint16_t* d_out, void* stream) {
    return guarded([&] {
        if (!c) throw std::invalid_argument("cache is null");
        cache_run(*c, d_q, d_out, as_stream(stream));
    });
}

pa_status pa_cache_decode(pa_cache* c, const uint16_t* d_q, uint16_t* d_out, int batch, int num_q_heads, int num_ctas,
                          void* stream) {
    return guarded([&] {
        if (!c) throw std::invalid_argument("cache is null");
        if (batch < 0) throw std::invalid_argument("decode: negative batch");
        std::vector<int32_t> slots(static_cast<size_t>(batch));
        std::iota(slots.begin(), slots.end(), 0);
        cache_plan(*c, slots.data(), batch, num_q_heads, num_ctas, as_stream(stream));
        cache_run(*c, d_q, d_out, as_stream(stream));
    });
}

const pa_plan* pa_cache_last_plan(const pa_cache* c) { return c ? &c->plan : nullptr; }

size_t pa_cache_total_bytes(const pa_cache* c) {
    return c ? bytes_per_page_impl(c->cfg) * static_cast<size_t>(c->cfg.num_pages) : 0;
}

}  // extern "C"
