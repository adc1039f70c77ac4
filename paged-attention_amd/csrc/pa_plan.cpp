// C-ABI host layer, part 1: the persistent planner, the device plan and the
// kernel entry points (decode, append, gather, stream reads) over the gfx950
// kernels in pa_decode.hip and pa_cache.hip. Every exported function catches
// exceptions and returns a pa_status (pa_decode.h maps them to the
// reference's errors).

#include "pa_host.hpp"

#include <algorithm>
#include <climits>
#include <string>
#include <vector>

namespace {

using namespace pa::host;

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

}  // namespace

namespace pa::host {

thread_local std::string g_last_error;

void check_dtype(int dtype) {
    if (dtype != PA_KV_FP16 && dtype != PA_KV_FP8_E4M3)
        throw std::invalid_argument("unknown kv dtype " + std::to_string(dtype));
}
constexpr int kChainMaxBlocks = 8;    // blocks one item may span under block_merge 2
int plan_merge_mode(const pa_plan& plan) {
    const size_t nseg = plan.segments.size() / 4;
    if (nseg <= static_cast<size_t>(plan.items)) return 0;   // no split items
    // The split kernel keeps a unit's split segments in two LDS slots: they
    // must be the unit's first and last segments (true of every make_plan cut).
    std::vector<int32_t> unit_of(nseg, 0);
    for (int u = 0; u < plan.num_ctas; ++u)
        for (int sg = plan.cta_seg_begin[u]; sg < plan.cta_seg_begin[u + 1]; ++sg)
            unit_of[static_cast<size_t>(sg)] = u;
    bool in_block = true, consecutive = true;
    for (int i = 0; i < plan.items; ++i) {
        const int a = plan.item_seg_begin[i], z = plan.item_seg_begin[i + 1];
        if (z - a <= 1) continue;
        const int u0 = unit_of[static_cast<size_t>(a)];
        const int nb = unit_of[static_cast<size_t>(z - 1)] / pa::kBlockUnits - u0 / pa::kBlockUnits + 1;
        if (nb > 1) in_block = false;
        // The split kernel's combine of a spanning item runs on one CU and
        // reads one partial per block: past 8 blocks per item the merge
        // kernel, which spreads every item over many CUs, is as fast or
        // faster (one MI355X: at 16 blocks per item 0.4-1.3 us faster in the
        // split kernel back to back but 0.9-1.6 us slower after a cache
        // flush, and slower either way on half-filled grids; at 32 blocks
        // 0.5-2.7 us slower). It addresses the partial rows with 32-bit
        // offsets (segments x 8 heads x 128 floats).
        if (nb > kChainMaxBlocks || z - a >= (1 << 19)) consecutive = false;
        for (int sg = a; sg < z; ++sg) {
            const int u = unit_of[static_cast<size_t>(sg)];
            if (sg != plan.cta_seg_begin[u] && sg != plan.cta_seg_begin[u + 1] - 1) return 0;
            if (u != u0 + (sg - a)) consecutive = false;
        }
    }
    if (in_block) return 1;
    // Chained merge: a block finds an item's other blocks from the unit of the
    // item's first segment, which needs the item's k-th segment in unit u0 + k.
#if PA_CHAIN_MERGE
    if (consecutive) return 2;
#endif
    return 0;
}
void make_plan_impl(pa_plan& plan, int dtype, const int32_t* lens, int batch, int hq, int hkv, int hd,
                    int num_ctas) {
    const int group = group_of(hq, hkv);
    check_shape(dtype, hd, group);
    const int tile = pa::kernel_tile_tokens(dtype, group);
    if (num_ctas <= 0) num_ctas = wave_ctas_impl(dtype, hd, group);
    cut(plan, tile, lens, batch, hkv, num_ctas);
}
pa_stage& take_stage(pa_stage_pool& sp, size_t need, bool with_device) {
    const size_t n = sp.bufs.size();
    size_t pick = n;
    for (size_t k = 0; k < n && pick == n; ++k) {
        const size_t i = (sp.next + k) % n;
        const hipError_t q = hipEventQuery(sp.bufs[i].done);
        if (q == hipSuccess) pick = i;
        else if (q != hipErrorNotReady) pa::hip_check(q, "hipEventQuery staging");
    }
    if (pick == n) {
        if (n < pa_stage_pool::kMaxStages) {
            sp.bufs.emplace_back();
            pa::hip_check(hipEventCreateWithFlags(&sp.bufs.back().done, hipEventDisableTiming), "hipEventCreate");
        } else {
            pick = sp.next % n;   // every buffer in flight: the oldest
            pa::hip_check(hipEventSynchronize(sp.bufs[pick].done), "hipEventSynchronize staging");
        }
    }
    sp.next = (pick + 1) % sp.bufs.size();
    pa_stage& st = sp.bufs[pick];
    if (st.cap < need || (with_device && !st.dev)) {
        const size_t cap = std::max<size_t>(need + need / 2, 4096);
        (void)hipHostFree(st.host);
        (void)hipFree(st.dev);
        st.host = nullptr;
        st.dev  = nullptr;
        st.cap  = 0;
        pa::hip_check(hipHostMalloc(reinterpret_cast<void**>(&st.host), cap * sizeof(int32_t), hipHostMallocDefault),
                      "hipHostMalloc staging");
        if (with_device)
            pa::hip_check(hipMalloc(reinterpret_cast<void**>(&st.dev), cap * sizeof(int32_t)), "hipMalloc staging");
        st.cap = cap;
    }
    return st;
}
void release_stage(pa_stage& st, hipStream_t s) { pa::hip_check(hipEventRecord(st.done, s), "hipEventRecord staging"); }
void free_stages(pa_stage_pool& sp) {
    for (pa_stage& st : sp.bufs) {
        if (st.done) (void)hipEventSynchronize(st.done);
        (void)hipHostFree(st.host);
        (void)hipFree(st.dev);
        if (st.done) (void)hipEventDestroy(st.done);
    }
    sp = pa_stage_pool{};
}
void device_plan_upload(pa_device_plan& dp, const pa_plan& plan, int group, int head_dim, hipStream_t s,
                        const int32_t* extra, size_t n_extra) {
    if (group <= 0 || head_dim <= 0) throw std::invalid_argument("upload: bad group or head_dim");
    if (n_extra && !extra) throw std::invalid_argument("upload: extra ints are null");
    scratch_prepare();
    const size_t nseg = plan.segments.size() / 4;
    // The kernels read a 16-token group from one page run (page sizes >= 16) or
    // one 1 KiB part from one page: a segment may only start on a group boundary.
    for (size_t i = 0; i < nseg; ++i)
        if (plan.segments[4 * i + 2] % pa::kGroupTokens != 0)
            throw std::invalid_argument("upload: segment starts must be multiples of 16 tokens");
    // One block: segments | cta_seg_begin | item_seg_begin | extra | merge
    // counters, each part starting on a 16-byte boundary (the kernels read
    // segments as int4).
    auto round4 = [](size_t n) { return (n + 3) & ~size_t{3}; };
    const size_t o_cta   = round4(plan.segments.size());
    const size_t o_item  = o_cta + round4(plan.cta_seg_begin.size());
    const size_t o_extra = o_item + round4(plan.item_seg_begin.size());
    const size_t o_ctr   = o_extra + round4(n_extra);   // per-item merge counters, uploaded as zeros
    const size_t total   = o_ctr + round4(static_cast<size_t>(plan.items));
    if (total > dp.ints_cap) {
        // Growing frees the old block, which decodes queued before may still
        // read: wait for them first (growth only happens for a plan larger
        // than every earlier one).
        pa::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        pa::hip_check(hipFree(dp.ints), "hipFree");
        dp.ints = nullptr;
        dp.ints_cap = 0;
        const size_t cap = std::max<size_t>(total + total / 4, 1024);
        pa::hip_check(hipMalloc(reinterpret_cast<void**>(&dp.ints), cap * sizeof(int32_t)), "hipMalloc plan");
        dp.ints_cap = cap;
    }
    pa_stage& st = take_stage(dp.staging, total, false);
    std::copy(plan.segments.begin(), plan.segments.end(), st.host);
    std::copy(plan.cta_seg_begin.begin(), plan.cta_seg_begin.end(), st.host + o_cta);
    std::copy(plan.item_seg_begin.begin(), plan.item_seg_begin.end(), st.host + o_item);
    if (n_extra) std::copy(extra, extra + n_extra, st.host + o_extra);
    std::fill(st.host + o_ctr, st.host + total, 0);
    pa::hip_check(hipMemcpyAsync(dp.ints, st.host, total * sizeof(int32_t), hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync plan");
    release_stage(st, s);
    dp.segments       = dp.ints;
    dp.cta_seg_begin  = dp.ints + o_cta;
    dp.item_seg_begin = dp.ints + o_item;
    dp.extra          = n_extra ? dp.ints + o_extra : nullptr;
    dp.merge_counters = dp.ints + o_ctr;
    const size_t rows = nseg * static_cast<size_t>(group);
    const size_t need = rows * (static_cast<size_t>(head_dim) + 1);
    if (need > dp.part_cap) {
        pa::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");   // queued decodes may still use it
        pa::hip_check(hipFree(dp.partial_out), "hipFree");
        dp.partial_out = nullptr;
        pa::hip_check(hipMalloc(reinterpret_cast<void**>(&dp.partial_out), sizeof(float) * need), "hipMalloc");
        dp.part_cap = need;
    }
    dp.partial_lse = dp.partial_out ? dp.partial_out + rows * head_dim : nullptr;
    dp.num_ctas = plan.num_ctas;
    dp.num_segments = static_cast<int>(nseg);
    dp.block_merge = plan_merge_mode(plan);
    dp.needs_merge = dp.block_merge == 0 && nseg > static_cast<size_t>(plan.items) ? 1 : 0;
    dp.max_item_segments = 0;
    for (int i = 0; i < plan.items; ++i)
        dp.max_item_segments = std::max(dp.max_item_segments, plan.item_seg_begin[i + 1] - plan.item_seg_begin[i]);
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
    p.block_merge       = dp.block_merge;
    p.num_segments      = dp.num_segments;
    p.merge_counters    = dp.merge_counters;
}
void device_plan_free(pa_device_plan& dp) {
    free_stages(dp.staging);
    (void)hipFree(dp.ints);
    (void)hipFree(dp.partial_out);
    dp = pa_device_plan{};
}
void decode_impl(int dtype, const pa_decode_params& p, hipStream_t s, bool split, bool merge) {
    if (split) pa::hip_check(pa::launch_decode_split(dtype, p, s), "decode split kernel launch");
    if (merge) pa::hip_check(pa::launch_decode_merge(dtype, p, s), "decode merge kernel launch");
}

}  // namespace pa::host

using namespace pa::host;

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
            if (sg[2] % pa::kGroupTokens != 0)
                throw std::invalid_argument("plan: segment starts must be multiples of 16 tokens");
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
pa_status pa_plan_merge_mode(const pa_plan* plan, int* out) {
    return guarded([&] {
        if (!plan || !out) throw std::invalid_argument("plan or out is null");
        *out = plan_merge_mode(*plan);
    });
}

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
        // One thread per (token, kv head, 8-dim chunk), indexed in 32 bits.
        if (static_cast<long long>(n) * num_kv_heads * (pa::kHeadDim / 8) > INT_MAX)
            throw std::length_error("append: n * num_kv_heads * 16 exceeds INT_MAX");
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

pa_status pa_f32_to_f16(const float* in, uint16_t* out, size_t n, void* stream) {
    return guarded([&] {
        if (n && (!in || !out)) throw std::invalid_argument("f32_to_f16: null pointer");
        pa::hip_check(pa::launch_convert(in, out, n, true, as_stream(stream)), "convert kernel launch");
    });
}

pa_status pa_f16_to_f32(const uint16_t* in, float* out, size_t n, void* stream) {
    return guarded([&] {
        if (n && (!in || !out)) throw std::invalid_argument("f16_to_f32: null pointer");
        pa::hip_check(pa::launch_convert(in, out, n, false, as_stream(stream)), "convert kernel launch");
    });
}

pa_status pa_fill_bytes(void* buf, size_t bytes, int value, void* stream) {
    return guarded([&] {
        if (bytes % 16 != 0 || (bytes && !buf)) throw std::invalid_argument("fill_bytes: bad arguments");
        pa::hip_check(pa::launch_fill_bytes(buf, bytes, value, as_stream(stream)), "fill kernel launch");
    });
}

}  // extern "C"
