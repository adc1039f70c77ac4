#pragma once
// decode::PagedKVCache (src/decode/paged_kv_cache.hpp:17-93) over
// libpa_decode.so: the same constructor, methods and semantics (admit returns
// -1 when full, append returns false and appends nothing when out of pages,
// std::invalid_argument / std::length_error on bad input).

#include "decode.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>
#include <vector>

namespace decode {

// Multi-head paged KV cache in HND layout: [page][kv_head][slot_in_page][head_dim].
// Pages come from a free list and are mapped per sequence by a device block
// table that is updated incrementally. FP8 caches quantize on append with
// per-tensor scales (stored = value * (1 / scale)).
class PagedKVCache {
public:
    struct Config {
        int     num_pages;
        int     page_size;
        int     num_kv_heads;
        int     head_dim;
        int     max_slots;           // concurrent sequences the block table can hold
        int     max_pages_per_slot;
        KVDtype dtype   = KVDtype::FP16;
        float   k_scale = 1.0f;      // FP8 only
        float   v_scale = 1.0f;
    };

    explicit PagedKVCache(const Config& cfg) : cfg_(cfg) {
        const pa_cache_config c = to_abi(cfg);
        detail::check(pa_cache_create(&c, &h_));
        tables_.resize(static_cast<size_t>(cfg.max_slots));
    }
    ~PagedKVCache() { pa_cache_destroy(h_); }
    PagedKVCache(const PagedKVCache&)            = delete;
    PagedKVCache& operator=(const PagedKVCache&) = delete;

    // Bytes of K+V one page occupies across all kv heads.
    static size_t bytes_per_page(const Config& cfg) {
        const pa_cache_config c = to_abi(cfg);
        return pa_cache_bytes_per_page(&c);
    }
    // Pages that fit in a byte budget.
    static int pages_for_budget(const Config& cfg, size_t budget_bytes) {
        const pa_cache_config c = to_abi(cfg);
        return pa_cache_pages_for_budget(&c, budget_bytes);
    }

    // Claims an empty sequence slot; -1 when every slot is in use.
    int admit() { return pa_cache_admit(h_); }
    // Appends n tokens of fp16 K/V ([n][num_kv_heads][head_dim], device memory),
    // allocating pages as needed; false (nothing appended) when out of pages.
    bool append(int slot, const half* d_k, const half* d_v, int n, hipStream_t stream = 0) {
        int done = 0;
        detail::check(pa_cache_append(h_, slot, reinterpret_cast<const uint16_t*>(d_k),
                                      reinterpret_cast<const uint16_t*>(d_v), n, stream, &done));
        return done != 0;
    }
    // Appends counts[i] tokens to slots[i] for every i with one host-to-device
    // copy and one kernel, without synchronizing the stream. d_k / d_v hold the
    // tokens concatenated in entry order; pages are reserved all-or-nothing.
    bool append_batch(const std::vector<int>& slots, const std::vector<int>& counts, const half* d_k, const half* d_v,
                      hipStream_t stream = 0) {
        if (slots.size() != counts.size()) throw std::invalid_argument("append_batch: slots and counts differ in size");
        int done = 0;
        detail::check(pa_cache_append_batch(h_, slots.data(), counts.data(), static_cast<int>(slots.size()),
                                            reinterpret_cast<const uint16_t*>(d_k),
                                            reinterpret_cast<const uint16_t*>(d_v), stream, &done));
        return done != 0;
    }
    // Returns a slot's pages to the free list.
    void release(int slot) { detail::check(pa_cache_release(h_, slot)); }
    // Randomizes allocation order (std::shuffle with std::mt19937(seed)).
    void shuffle_free_pages(unsigned seed) { pa_cache_shuffle_free_pages(h_, seed); }

    // Schedules one decode step over `slots` (batch row i reads cache slot slots[i]).
    void plan(const std::vector<int>& slots, int num_q_heads, int num_ctas = 0, hipStream_t stream = 0) {
        detail::check(pa_cache_plan(h_, slots.data(), static_cast<int>(slots.size()), num_q_heads, num_ctas, stream));
        plan_ = detail::to_plan(pa_cache_last_plan(h_));
    }
    // Decodes the planned batch. q/out: [batch][num_q_heads][head_dim], device memory.
    void run(const half* d_q, half* d_out, hipStream_t stream = 0) {
        detail::check(pa_cache_run(h_, reinterpret_cast<const uint16_t*>(d_q), reinterpret_cast<uint16_t*>(d_out),
                                   stream));
    }
    // plan() over slots 0..batch-1, then run().
    void decode(const half* d_q, half* d_out, int batch, int num_q_heads, int num_ctas = 0, hipStream_t stream = 0) {
        detail::check(pa_cache_decode(h_, reinterpret_cast<const uint16_t*>(d_q), reinterpret_cast<uint16_t*>(d_out),
                                      batch, num_q_heads, num_ctas, stream));
        plan_ = detail::to_plan(pa_cache_last_plan(h_));
    }
    const DecodePlan& last_plan() const { return plan_; }

    // The cache-side fields of DecodeParams (for callers that drive the kernel directly).
    DecodeParams params() const {
        DecodeParams p{};
        detail::check(pa_cache_params(h_, detail::abi(p)));
        return p;
    }

    int    seq_len(int slot) const { return pa_pool_seq_len(pa_cache_pool(h_), slot); }
    bool   occupied(int slot) const { return pa_pool_occupied(pa_cache_pool(h_), slot) != 0; }
    int    free_pages() const { return pa_pool_free_pages(pa_cache_pool(h_)); }
    int    max_seq_len() const { return pa_pool_max_seq_len(pa_cache_pool(h_)); }
    size_t total_bytes() const { return pa_cache_total_bytes(h_); }
    const Config& config() const { return cfg_; }
    // The slot's physical pages in token order (a host copy, refreshed per call).
    const std::vector<int>& block_table(int slot) const {
        std::vector<int>& t = tables_.at(static_cast<size_t>(slot));
        t.resize(static_cast<size_t>(pa_pool_num_pages_of(pa_cache_pool(h_), slot)));
        detail::check(pa_pool_block_table(pa_cache_pool(h_), slot, t.data(), static_cast<int>(t.size())));
        return t;
    }

private:
    static pa_cache_config to_abi(const Config& c) {
        pa_cache_config a{};
        a.num_pages          = c.num_pages;
        a.page_size          = c.page_size;
        a.num_kv_heads       = c.num_kv_heads;
        a.head_dim           = c.head_dim;
        a.max_slots          = c.max_slots;
        a.max_pages_per_slot = c.max_pages_per_slot;
        a.dtype              = static_cast<int32_t>(c.dtype);
        a.k_scale            = c.k_scale;
        a.v_scale            = c.v_scale;
        return a;
    }

    Config     cfg_;
    pa_cache*  h_ = nullptr;
    DecodePlan plan_;
    mutable std::vector<std::vector<int>> tables_;
};

}  // namespace decode
