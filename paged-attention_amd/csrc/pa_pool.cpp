// C-ABI host layer, part 2: the host page pool (paged_kv_cache.cu:84-151):
// free list, per-slot block tables and lengths, no device memory.

#include "pa_host.hpp"

#include <algorithm>
#include <numeric>
#include <random>
#include <vector>

namespace pa::host {

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

}  // namespace pa::host

using namespace pa::host;

extern "C" {

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

}  // extern "C"
