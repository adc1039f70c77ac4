#pragma once
// decode::KVDtype and decode::DecodeParams (src/decode/decode_types.hpp:8-45)
// over libpa_decode.so. DecodeParams keeps the reference's field names, types
// and order and is layout-identical to the C ABI's pa_decode_params, so it is
// handed to the library as is.

#include "pa_decode.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>

namespace decode {

enum class KVDtype { FP16 = PA_KV_FP16, FP8_E4M3 = PA_KV_FP8_E4M3 };

inline int kv_dtype_bytes(KVDtype t) { return t == KVDtype::FP16 ? 2 : 1; }
inline const char* kv_dtype_name(KVDtype t) { return t == KVDtype::FP16 ? "fp16" : "fp8_e4m3"; }

// Everything the decode kernels read. All pointers are device pointers.
struct DecodeParams {
    const half* q;                // [batch][num_q_heads][head_dim]
    half*       out;              // [batch][num_q_heads][head_dim]

    const void* k_cache;          // [num_pages][num_kv_heads][page_size][head_dim], fp16 or fp8
    const void* v_cache;
    const int*  block_table;      // [num_slots][block_table_stride] physical page ids
    const int*  seq_lens;         // [num_slots] (carried, not read by the kernels)
    const int*  slot_ids;         // [batch] cache slot of each batch row; nullptr => identity
    int         block_table_stride;

    int batch;
    int num_q_heads;
    int num_kv_heads;
    int head_dim;
    int page_size;

    float sm_scale;               // usually 1/sqrt(head_dim)
    float k_scale;                // FP8 dequantization scales (1.0 for fp16)
    float v_scale;

    // Schedule (see DecodePlan): segment i covers tokens [z, w) of (batch row
    // x, kv head y); work unit c runs segments [cta_seg_begin[c], cta_seg_begin[c+1]).
    const int4* segments;
    const int*  cta_seg_begin;    // [num_ctas + 1]
    const int*  item_seg_begin;   // [batch * num_kv_heads + 1]
    int         num_ctas;
    int         needs_merge;      // some (row, head) spans more than one segment

    float* partial_out;           // [num_segments][group][head_dim]
    float* partial_lse;           // [num_segments][group]

    int max_item_segments = 0;    // most segments of one (row, head); sizes the merge (0 = unknown)
    int block_merge       = 0;    // split rows merged inside the split kernel (set by DevicePlan::bind)
    int num_segments      = 0;    // segments of the bound plan (set by DevicePlan::bind; 0 = unknown)
    int* merge_counters   = nullptr;   // per-item arrival counters of block_merge 2 (set by DevicePlan::bind)
};

static_assert(sizeof(DecodeParams) == sizeof(pa_decode_params), "DecodeParams must match pa_decode_params");
static_assert(offsetof(DecodeParams, block_table_stride) == offsetof(pa_decode_params, block_table_stride));
static_assert(offsetof(DecodeParams, sm_scale) == offsetof(pa_decode_params, sm_scale));
static_assert(offsetof(DecodeParams, segments) == offsetof(pa_decode_params, segments));
static_assert(offsetof(DecodeParams, partial_lse) == offsetof(pa_decode_params, partial_lse));
static_assert(offsetof(DecodeParams, max_item_segments) == offsetof(pa_decode_params, max_item_segments));
static_assert(offsetof(DecodeParams, block_merge) == offsetof(pa_decode_params, block_merge));
static_assert(offsetof(DecodeParams, num_segments) == offsetof(pa_decode_params, num_segments));
static_assert(offsetof(DecodeParams, merge_counters) == offsetof(pa_decode_params, merge_counters));
static_assert(sizeof(int4) == 4 * sizeof(int32_t), "segments are int32 quadruples");

namespace detail {
inline const pa_decode_params* abi(const DecodeParams& p) { return reinterpret_cast<const pa_decode_params*>(&p); }
inline pa_decode_params* abi(DecodeParams& p) { return reinterpret_cast<pa_decode_params*>(&p); }
}  // namespace detail

}  // namespace decode
