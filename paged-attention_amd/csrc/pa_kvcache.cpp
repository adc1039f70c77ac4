// C-ABI host layer, part 3: the paged KV cache (paged_kv_cache.cu): device
// pools and block table over the host pool, per-slot and batched appends, and
// plan / run / decode over the device plan.

#include "pa_host.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <numeric>
#include <vector>

namespace {

using namespace pa::host;

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
    device_plan_upload(c.dplan, c.plan, hq / c.cfg.num_kv_heads, c.cfg.head_dim, s, slots, static_cast<size_t>(n));
    c.plan_batch = n;
    c.plan_hq    = hq;
}

void cache_run(pa_cache& c, const uint16_t* q, uint16_t* out, hipStream_t s) {
    pa_decode_params p;
    cache_params(c, p);
    p.q           = q;
    p.out         = out;
    p.slot_ids    = c.dplan.extra;
    p.batch       = c.plan_batch;
    p.num_q_heads = c.plan_hq;
    device_plan_bind(c.dplan, p);
    decode_impl(c.cfg.dtype, p, s, true, true);
}

}  // namespace

using namespace pa::host;

extern "C" {

size_t pa_cache_bytes_per_page(const pa_cache_config* cfg) { return cfg ? bytes_per_page_impl(*cfg) : 0; }
size_t pa_kv_pool_stagger(void) { return pa::kPoolStagger; }

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
            // One allocation for both pools, V starting kPoolStagger bytes after
            // the end of K (the K/V bank-conflict gap).
            pa::hip_check(hipMalloc(&c->d_k, 2 * half_bytes + pa::kPoolStagger), "hipMalloc k/v pools");
            c->d_v = static_cast<unsigned char*>(c->d_k) + half_bytes + pa::kPoolStagger;
            pa::hip_check(hipMalloc(reinterpret_cast<void**>(&c->d_table), table), "hipMalloc block table");
            pa::hip_check(hipMalloc(reinterpret_cast<void**>(&c->d_seq_lens), sizeof(int32_t) * cfg->max_slots),
                          "hipMalloc seq_lens");
            pa::hip_check(hipMemset(c->d_table, 0, table), "hipMemset");
            pa::hip_check(hipMemset(c->d_seq_lens, 0, sizeof(int32_t) * cfg->max_slots), "hipMemset");
        } catch (...) {
            (void)hipFree(c->d_k);
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
    (void)hipFree(c->d_k);   // both pools
    (void)hipFree(c->d_table);
    (void)hipFree(c->d_seq_lens);
    free_stages(c->append_staging);
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
        if (static_cast<long long>(n) * c->cfg.num_kv_heads * (pa::kHeadDim / 8) > INT_MAX)
            throw std::length_error("append: n * num_kv_heads * 16 exceeds INT_MAX");
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
        pa_stage& st = take_stage(c->append_staging, need, true);
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
        release_stage(st, s);
    });
}

pa_status pa_cache_release(pa_cache* c, int slot) {
    return guarded([&] {
        if (!c) throw std::invalid_argument("cache is null");
        pool_release(c->pool, slot);
        // A batched append still in flight may write this slot's length.
        for (pa_stage& st : c->append_staging.bufs)
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
