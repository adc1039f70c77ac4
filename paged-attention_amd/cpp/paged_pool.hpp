#pragma once
// The legacy single-head interfaces over the new paged cache:
//
//   PagedPool          : KVPool            (src/attention/paged_pool/pool.hpp:9-61)
//   PagedPoolAttention : AttentionBackend  (src/attention/paged_pool/pool.hpp:76-81)
//
// Same constructors, methods and return conventions as the reference's FP32
// pool, but the storage is decode::PagedKVCache (one kv head, HND pages, fp16
// or FP8 E4M3) and decode runs the MI355X split-KV kernels. Differences a
// caller sees:
//   * K/V arrive as fp32 host rows and are stored rounded to fp16 (RNE), or
//     quantized to E4M3 for an FP8 pool; decode returns the kernel's fp16
//     output widened to fp32. Against fp32 attention over the same rows the
//     result is within 2e-3 max-abs (the reference's pool is fp32 end to end).
//   * head_dim must be 128 (std::invalid_argument otherwise).
//   * The reference asserts; this pool throws: std::invalid_argument for a
//     slot that is not admitted, a non-positive length or an append_token
//     position other than the slot's current length (the cache is append-only),
//     std::length_error when append_token finds no free page or a sequence
//     would exceed max_pages_per_seq. admit() returns -1 when no slot or not
//     enough pages are free, as in the reference.
//   * decode_device() takes fp32 device q / out as the reference's does; q is
//     rounded to fp16 on the device and the fp16 output widened back. The
//     three partial buffers are accepted and unused (the plan's own workspace
//     holds the split partials). Like the reference it launches on the default
//     stream and does not synchronize.
//   * kv_K_base() / kv_V_base() return the fp16 (or E4M3) pools as const void*.
//   * paged_max_sequences_for_budget() counts this pool's element size (fp16 by
//     default, one byte for FP8) where the reference's counts fp32.

#include "attention_backend.hpp"
#include "decode/half_host.hpp"
#include "decode/paged_kv_cache.hpp"
#include "hip_check.hpp"
#include "kv_pool.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <vector>

static constexpr int PAGE_SIZE = 16;

class PagedPool : public KVPool {
public:
    PagedPool(int total_pages, int max_sequences, int max_pages_per_seq, int d, int page_size = PAGE_SIZE,
              decode::KVDtype dtype = decode::KVDtype::FP16, float k_scale = 1.0f, float v_scale = 1.0f)
        : cache_(config(total_pages, max_sequences, max_pages_per_seq, d, page_size, dtype, k_scale, v_scale)),
          d_(d) {
        HIP_CHECK(hipMalloc(&d_q_, sizeof(uint16_t) * static_cast<size_t>(d)));
        HIP_CHECK(hipMalloc(&d_out_, sizeof(uint16_t) * static_cast<size_t>(d)));
        // Slot ids 0 .. max_sequences - 1: decode_device points a plan's slot
        // indirection at entry `slot` instead of copying the id per call.
        std::vector<int32_t> ids(static_cast<size_t>(max_sequences));
        for (int i = 0; i < max_sequences; ++i) ids[static_cast<size_t>(i)] = i;
        HIP_CHECK(hipMalloc(&d_slots_, sizeof(int32_t) * ids.size()));
        HIP_CHECK(hipMemcpy(d_slots_, ids.data(), sizeof(int32_t) * ids.size(), hipMemcpyHostToDevice));
    }
    ~PagedPool() override {
        (void)hipFree(d_q_);
        (void)hipFree(d_out_);
        (void)hipFree(d_kv_);
        (void)hipFree(d_slots_);
    }
    PagedPool(const PagedPool&)            = delete;
    PagedPool& operator=(const PagedPool&) = delete;

    // Claims a slot and stores actual_len rows of K and V ([actual_len][d] fp32,
    // host). -1 (nothing changed) when no slot or not enough pages are free.
    int admit(const float* h_K, const float* h_V, int actual_len) override {
        if (actual_len <= 0) throw std::invalid_argument("PagedPool::admit: actual_len must be positive");
        const int slot = cache_.admit();
        if (slot < 0) return -1;
        try {
            stage(h_K, h_V, actual_len);
            if (!cache_.append(slot, half_ptr(d_kv_), half_ptr(d_kv_ + kv_elems(actual_len)), actual_len)) {
                cache_.release(slot);
                return -1;
            }
        } catch (...) {
            cache_.release(slot);
            throw;
        }
        return slot;
    }

    void release(int slot) override { cache_.release(slot); }

    // Stores one K/V row at position actual_len, which must be the slot's
    // current length; the slot grows by one.
    void append_token(int slot, int actual_len, const float* h_k, const float* h_v) override {
        if (!is_occupied(slot)) throw std::invalid_argument("PagedPool::append_token: slot is not admitted");
        if (actual_len != cache_.seq_len(slot))
            throw std::invalid_argument("PagedPool::append_token: actual_len must be the slot's current length");
        stage(h_k, h_v, 1);
        if (!cache_.append(slot, half_ptr(d_kv_), half_ptr(d_kv_ + kv_elems(1)), 1))
            throw std::length_error("PagedPool::append_token: no free page");
    }

    // out[d] = attention of q ([d] fp32, host) over the slot's rows.
    void decode(int slot, const float* h_q, float* h_out) override {
        if (!is_occupied(slot) || actual_len(slot) <= 0)
            throw std::invalid_argument("PagedPool::decode: slot is not admitted or empty");
        std::vector<uint16_t> h(static_cast<size_t>(d_));
        for (int i = 0; i < d_; ++i) h[static_cast<size_t>(i)] = decode::f32_to_f16(h_q[i]);
        HIP_CHECK(hipMemcpy(d_q_, h.data(), sizeof(uint16_t) * h.size(), hipMemcpyHostToDevice));
        cache_.plan({slot}, 1);
        cache_.run(half_ptr(d_q_), reinterpret_cast<half*>(d_out_));
        HIP_CHECK(hipMemcpy(h.data(), d_out_, sizeof(uint16_t) * h.size(), hipMemcpyDeviceToHost));
        for (int i = 0; i < d_; ++i) h_out[i] = decode::f16_to_f32(h[static_cast<size_t>(i)]);
    }

    // pool.hpp:21-24 decode_device: out[d] (fp32, device) = attention of q[d]
    // (fp32, device) over the first actual_len rows of the slot. Launches on the
    // default stream and returns without synchronizing. The partial buffers of
    // the reference's signature are not used.
    void decode_device(int slot, int actual_len, const float* d_q, float* d_out, float* d_partial_out = nullptr,
                       float* d_partial_max = nullptr, float* d_partial_sum = nullptr) const {
        (void)d_partial_out;
        (void)d_partial_max;
        (void)d_partial_sum;
        if (!is_occupied(slot)) throw std::invalid_argument("PagedPool::decode_device: slot is not admitted");
        if (actual_len <= 0 || actual_len > cache_.seq_len(slot))
            throw std::invalid_argument("PagedPool::decode_device: actual_len must be in 1 .. the slot's length");
        if (!d_q || !d_out) throw std::invalid_argument("PagedPool::decode_device: null q or out");
        const decode::KVDtype dt = cache_.config().dtype;
        dplan_.upload(decode::make_plan(dt, {actual_len}, 1, 1, d_), 1, d_, 0);
        decode::detail::check(pa_f32_to_f16(d_q, d_q_, static_cast<size_t>(d_), nullptr));
        decode::DecodeParams p = cache_.params();
        p.q           = half_ptr(d_q_);
        p.out         = reinterpret_cast<half*>(d_out_);
        p.slot_ids    = d_slots_ + slot;
        p.batch       = 1;
        p.num_q_heads = 1;
        dplan_.bind(p);
        decode::paged_decode(dt, p, 0);
        decode::detail::check(pa_f16_to_f32(d_out_, d_out, static_cast<size_t>(d_), nullptr));
    }

    int  actual_len(int slot) const override { return is_occupied(slot) ? cache_.seq_len(slot) : 0; }
    bool is_occupied(int slot) const override {
        return slot >= 0 && slot < cache_.config().max_slots && cache_.occupied(slot);
    }
    int    free_page_count() const { return cache_.free_pages(); }
    int    total_pages() const { return cache_.config().num_pages; }
    int    max_sequences() const { return cache_.config().max_slots; }
    int    d() const { return d_; }
    size_t total_kv_bytes() const { return cache_.total_bytes(); }
    // pool.hpp:34-35: the device K and V pools ([pages][1][page_size][d], fp16
    // or E4M3 bytes).
    const void* kv_K_base() const { return cache_.params().k_cache; }
    const void* kv_V_base() const { return cache_.params().v_cache; }
    // The cache underneath (block tables, params() for the batched kernels).
    decode::PagedKVCache&       cache() { return cache_; }
    const decode::PagedKVCache& cache() const { return cache_; }

private:
    static decode::PagedKVCache::Config config(int total_pages, int max_sequences, int max_pages_per_seq, int d,
                                               int page_size, decode::KVDtype dtype, float k_scale, float v_scale) {
        decode::PagedKVCache::Config c{};
        c.num_pages          = total_pages;
        c.page_size          = page_size;
        c.num_kv_heads       = 1;
        c.head_dim           = d;
        c.max_slots          = max_sequences;
        c.max_pages_per_slot = max_pages_per_seq;
        c.dtype              = dtype;
        c.k_scale            = k_scale;
        c.v_scale            = v_scale;
        return c;
    }
    size_t kv_elems(int n) const { return static_cast<size_t>(n) * static_cast<size_t>(d_); }
    static const half* half_ptr(const uint16_t* p) { return reinterpret_cast<const half*>(p); }

    // Rounds n rows of K and V to fp16 and copies them to the device staging
    // buffer (K rows, then V rows).
    void stage(const float* h_K, const float* h_V, int n) {
        const size_t m = kv_elems(n);
        if (2 * m > cap_) {
            (void)hipFree(d_kv_);
            d_kv_ = nullptr;
            cap_  = 0;
            HIP_CHECK(hipMalloc(&d_kv_, sizeof(uint16_t) * 2 * m));
            cap_ = 2 * m;
        }
        host_.resize(2 * m);
        for (size_t i = 0; i < m; ++i) {
            host_[i]     = decode::f32_to_f16(h_K[i]);
            host_[m + i] = decode::f32_to_f16(h_V[i]);
        }
        HIP_CHECK(hipMemcpy(d_kv_, host_.data(), sizeof(uint16_t) * 2 * m, hipMemcpyHostToDevice));
    }

    decode::PagedKVCache  cache_;
    int                   d_;
    uint16_t*             d_q_   = nullptr;
    uint16_t*             d_out_ = nullptr;
    uint16_t*             d_kv_  = nullptr;
    size_t                cap_   = 0;
    std::vector<uint16_t> host_;
    int32_t*              d_slots_ = nullptr;   // [max_sequences]: i at entry i
    // decode_device's plan (the method is const in the reference's interface).
    mutable decode::DevicePlan dplan_;
};

// pool.hpp:63-67: sequences of actual_len tokens that fit budget_bytes of
// this pool's pages (K and V, page_size x d elements each, 2 bytes per fp16
// element or 1 per E4M3 one).
inline int paged_max_sequences_for_budget(size_t budget_bytes, int actual_len, int d, int page_size = PAGE_SIZE,
                                          decode::KVDtype dtype = decode::KVDtype::FP16) {
    if (actual_len <= 0 || d <= 0 || page_size <= 0)
        throw std::invalid_argument("paged_max_sequences_for_budget: sizes must be positive");
    const int    pages_per_seq = (actual_len + page_size - 1) / page_size;
    const size_t per_page      = 2ull * static_cast<size_t>(decode::kv_dtype_bytes(dtype)) *
                                 static_cast<size_t>(page_size) * static_cast<size_t>(d);
    return static_cast<int>(budget_bytes / per_page) / pages_per_seq;
}

// pool.hpp:69-72: slots left empty in the last page of a sequence.
inline int paged_waste_tokens(int actual_len, int page_size = PAGE_SIZE) {
    const int pages = (actual_len + page_size - 1) / page_size;
    return pages * page_size - actual_len;
}

// One query over T rows through a single-use PagedPool sized to fit them
// (src/attention/paged_pool/pool.cu:159-166).
class PagedPoolAttention : public AttentionBackend {
public:
    void run(const float* q, const float* K, const float* V, float* out, int T, int d) override {
        const int pages = (T + PAGE_SIZE - 1) / PAGE_SIZE;
        PagedPool pool(pages, 1, pages, d);
        const int slot = pool.admit(K, V, T);
        if (slot != 0) throw std::runtime_error("PagedPoolAttention: admit failed");
        pool.decode(slot, q, out);
    }
    const char* name() const override { return "paged_pool"; }
};
