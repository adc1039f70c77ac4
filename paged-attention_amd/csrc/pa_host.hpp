#pragma once
// Host-side state behind the C ABI of libpa_decode.so (plans, device plans, the
// page pool, the paged cache) and the helpers the C entry points share. Internal
// to the library; the public interface is include/pa_decode.h.

#include "pa_decode.h"
#include "pa_internal.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <new>
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

// One pinned host staging buffer for host-to-device copies on a stream: pinned
// host ints, optionally their own device copy, and an event recorded after the
// last stream operation that reads them.
struct pa_stage {
    int32_t*   host = nullptr;
    int32_t*   dev  = nullptr;
    size_t     cap  = 0;   // int32 elements
    hipEvent_t done = nullptr;
};

// Staging buffers for copies that may still be in flight while the next one is
// staged: a call takes any buffer whose last copy has finished and adds a buffer
// (up to kMaxStages) when none has, so a caller that runs a few steps ahead of
// the device never waits for it.
struct pa_stage_pool {
    static constexpr size_t kMaxStages = 8;
    std::vector<pa_stage> bufs;
    size_t next = 0;   // where the search for a finished buffer starts
};

// Device copy of a plan plus the partial workspace (decode.hpp:44-63). The
// plan's int arrays share one device block: segments, cta_seg_begin,
// item_seg_begin, then the caller's extra ints (the cache's slot ids).
struct pa_device_plan {
    int32_t* ints           = nullptr;   // the block
    size_t   ints_cap       = 0;         // int32 elements
    int32_t* segments       = nullptr;
    int32_t* cta_seg_begin  = nullptr;
    int32_t* item_seg_begin = nullptr;
    int32_t* extra          = nullptr;
    float*   partial_out    = nullptr;
    float*   partial_lse    = nullptr;
    size_t   part_cap = 0;
    int      num_ctas    = 0;
    int      needs_merge = 0;
    int      max_item_segments = 0;
    int      num_segments = 0;
    int      block_merge = 0;          // pa_decode_params.block_merge of the plan
    int32_t* merge_counters = nullptr;  // per-item counters in `ints`
    pa_stage_pool staging;
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

struct pa_cache {
    pa_cache_config cfg{};
    pa_pool         pool;
    void*           d_k          = nullptr;
    void*           d_v          = nullptr;
    int32_t*        d_table      = nullptr;   // [max_slots][max_pages_per_slot]
    int32_t*        d_seq_lens   = nullptr;   // [max_slots]
    pa_plan         plan;
    pa_device_plan  dplan;                    // its extra ints are the plan's slot ids
    int             plan_batch = 0;
    int             plan_hq    = 0;
    pa_stage_pool   append_staging;           // the batched append's metadata
};

namespace pa::host {

// The message behind this thread's last non-OK status (pa_last_error).
extern thread_local std::string g_last_error;

// Runs f and maps its exception to a status (pa_decode.h): the reference's
// std::invalid_argument / std::length_error, and device errors.
template <class F>
inline pa_status guarded(F&& f) {
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

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// ---- staging (pa_plan.cpp)
// A buffer of the pool with room for `need` ints (and a device copy of that
// size when with_device) whose last use has finished: a free one, else a new
// one, else (kMaxStages in flight) the oldest after waiting for it. Grows a
// buffer by reallocating. The reference is valid until the next take_stage.
pa_stage& take_stage(pa_stage_pool& sp, size_t need, bool with_device);
// Records the buffer's event on s: call after queuing the work that reads it.
void release_stage(pa_stage& st, hipStream_t s);
// Waits for every queued use of the pool and frees its buffers and events.
void free_stages(pa_stage_pool& sp);

// ---- planner and device plan (pa_plan.cpp)
void check_dtype(int dtype);
// pa_decode_params.block_merge for a plan: 0 (merge kernel), 1 (every split
// item inside one block), 2 (items spanning blocks merged by the split kernel).
int  plan_merge_mode(const pa_plan& plan);
void make_plan_impl(pa_plan& plan, int dtype, const int32_t* lens, int batch, int hq, int hkv, int hd,
                    int num_ctas);
// Queues the plan's arrays (and n_extra caller ints, kept at dp.extra) for the
// device on s through pinned staging and returns: no stream synchronization.
// The host plan may change or go right after the call.
void device_plan_upload(pa_device_plan& dp, const pa_plan& plan, int group, int head_dim, hipStream_t s,
                        const int32_t* extra = nullptr, size_t n_extra = 0);
void device_plan_bind(const pa_device_plan& dp, pa_decode_params& p);
void device_plan_free(pa_device_plan& dp);
void decode_impl(int dtype, const pa_decode_params& p, hipStream_t s, bool split, bool merge);

// ---- allocation-free decode (pa_scratch.hip)
// Looks up the device address of pa_decode_static's static scratch array on
// the current device, once per device. Plan uploads call it, so the lookup
// (which may load the library's code object onto the device) happens at set-up,
// outside any graph capture of the decode that follows.
void scratch_prepare();

// ---- page pool (pa_pool.cpp)
// Entry i of a batched append: the slot's length before it, and the table
// entries it added.
struct reserve_entry {
    int old_len   = 0;
    int first_new = 0;
    int num_new   = 0;
};

void pool_init(pa_pool& pool, int num_pages, int page_size, int max_slots, int max_pages_per_slot);
bool slot_ok(const pa_pool& pool, int slot);
int  pool_admit(pa_pool& pool);
// Append bookkeeping: false (nothing changed) when out of pages.
bool pool_reserve(pa_pool& pool, int slot, int n, int& first_new, int& num_new);
bool pool_reserve_batch(pa_pool& pool, const int32_t* slots, const int32_t* counts, int n,
                        std::vector<reserve_entry>* entries);
void pool_release(pa_pool& pool, int slot);

}  // namespace pa::host
