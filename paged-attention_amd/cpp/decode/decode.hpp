#pragma once
// The persistent planner and the decode entry point (src/decode/decode.hpp:21-66)
// over libpa_decode.so: same names and signatures, hipStream_t for
// cudaStream_t, the reference's exception types.

#include "decode_types.hpp"
#include "hip_check.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <memory>
#include <vector>

namespace decode {

// A persistent, load-balanced schedule for one decode step: the flat list of
// (batch row, kv head, tile) work cut into num_ctas contiguous equal ranges,
// one per work unit; each maximal run of one (row, head) inside a range is a
// segment. Build it once per step and reuse it for every layer.
struct DecodePlan {
    int num_ctas = 0;
    int tile     = 0;
    std::vector<int4> segments;
    std::vector<int>  cta_seg_begin;
    std::vector<int>  item_seg_begin;
};

// Tokens per planning tile for this configuration (the kernel's step).
inline int tile_tokens(KVDtype dtype, int head_dim, int group) {
    int v = 0;
    detail::check(pa_tile_tokens(static_cast<int>(dtype), head_dim, group, &v));
    return v;
}

// Work units (waves) resident in one full wave of the decode kernel on the current device.
inline int wave_ctas(KVDtype dtype, int head_dim, int group) {
    int v = 0;
    detail::check(pa_wave_ctas(static_cast<int>(dtype), head_dim, group, &v));
    return v;
}

// Persistent grid size used when a plan does not specify one (one full wave).
inline int default_ctas(KVDtype dtype, int head_dim, int group) {
    int v = 0;
    detail::check(pa_default_ctas(static_cast<int>(dtype), head_dim, group, &v));
    return v;
}

namespace detail {
struct PlanDeleter {
    void operator()(pa_plan* p) const { pa_plan_destroy(p); }
};
using PlanHandle = std::unique_ptr<pa_plan, PlanDeleter>;

inline DecodePlan to_plan(const pa_plan* h) {
    DecodePlan p;
    p.num_ctas = pa_plan_num_ctas(h);
    p.tile     = pa_plan_tile(h);
    p.segments.resize(static_cast<size_t>(pa_plan_num_segments(h)));
    p.cta_seg_begin.resize(static_cast<size_t>(p.num_ctas) + 1);
    p.item_seg_begin.resize(static_cast<size_t>(pa_plan_num_items(h)) + 1);
    check(pa_plan_copy(h, reinterpret_cast<int32_t*>(p.segments.data()), p.cta_seg_begin.data(),
                       p.item_seg_begin.data()));
    return p;
}
}  // namespace detail

// seq_lens[i] is the length of batch row i. num_ctas = 0 uses default_ctas.
inline DecodePlan make_plan(KVDtype dtype, const std::vector<int>& seq_lens, int num_q_heads, int num_kv_heads,
                            int head_dim, int num_ctas = 0) {
    pa_plan* raw = nullptr;
    detail::check(pa_plan_build(static_cast<int>(dtype), seq_lens.data(), static_cast<int>(seq_lens.size()),
                                num_q_heads, num_kv_heads, head_dim, num_ctas, &raw));
    detail::PlanHandle h(raw);
    return detail::to_plan(h.get());
}

// Device copy of a plan plus the partial-result workspace it needs.
class DevicePlan {
public:
    DevicePlan() { detail::check(pa_device_plan_create(&h_)); }
    ~DevicePlan() { pa_device_plan_destroy(h_); }
    DevicePlan(const DevicePlan&)            = delete;
    DevicePlan& operator=(const DevicePlan&) = delete;

    // Uploads `plan` (growing buffers as needed); bind() then points params at it.
    void upload(const DecodePlan& plan, int group, int head_dim, hipStream_t stream = 0) {
        if (plan.cta_seg_begin.empty() || plan.item_seg_begin.empty())
            throw std::invalid_argument("DevicePlan::upload: plan has no prefix arrays");
        const int items = static_cast<int>(plan.item_seg_begin.size()) - 1;
        pa_plan* raw = nullptr;   // validated copy; kv heads inferred from the segments
        detail::check(pa_plan_create(plan.num_ctas, plan.tile, reinterpret_cast<const int32_t*>(plan.segments.data()),
                                     static_cast<int>(plan.segments.size()), plan.cta_seg_begin.data(),
                                     plan.item_seg_begin.data(), items, 0, &raw));
        detail::PlanHandle h(raw);
        detail::check(pa_device_plan_upload(h_, h.get(), group, head_dim, stream));
    }
    void bind(DecodeParams& p) const { detail::check(pa_device_plan_bind(h_, detail::abi(p))); }

private:
    pa_device_plan* h_ = nullptr;
};

// Runs the split kernel and, if any row was split across work units, the merge.
// Supported: head_dim 128; num_q_heads / num_kv_heads in {1, 2, 4, 8}.
inline void paged_decode(KVDtype dtype, const DecodeParams& p, hipStream_t stream = 0) {
    detail::check(pa_decode(static_cast<int>(dtype), detail::abi(p), stream));
}

}  // namespace decode
