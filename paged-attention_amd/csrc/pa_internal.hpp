// Internal interface between the C-ABI host layer (pa_plan.cpp, pa_pool.cpp,
// pa_kvcache.cpp) and the gfx950 kernels (pa_decode.hip, pa_cache.hip). Not
// installed; callers use pa_decode.h.
#pragma once

#include "pa_decode.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace pa {

// Raised by host code for a failed HIP runtime call; the C ABI maps it to
// PA_ERR_DEVICE.
struct DeviceError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw DeviceError(std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

constexpr int kHeadDim     = 128;   // the only head_dim the path supports (decode.cu:31-38)
constexpr int kGroupTokens = 16;    // tokens per MFMA step of the decode kernel
#ifndef PA_BLOCK_UNITS
#define PA_BLOCK_UNITS 8
#endif
constexpr int kBlockUnits  = PA_BLOCK_UNITS;   // work units (waves) per block of the decode kernel
// 1: plans whose split (row, kv head) items span blocks are merged inside the
// split kernel (pa_decode_params.block_merge 2); 0: by the merge kernel.
#ifndef PA_CHAIN_MERGE
#define PA_CHAIN_MERGE 1
#endif

// Byte gap between the end of the K pool and the start of the V pool when both
// share one allocation. A wave reads the same (page, kv head) run of K and of
// V at once; pools at the same offset modulo a large power of two put those
// two reads on the same HBM banks, and on MI355X a decode step is then 3-7%
// slower (32 x 8192 fp16, 16-token pages: 163.2 against 158.4 us). 8 KiB was
// the best or near-best gap for fp16 and FP8 at page sizes 16 to 8192.
#ifndef PA_POOL_STAGGER
#define PA_POOL_STAGGER 8192
#endif
constexpr size_t kPoolStagger = PA_POOL_STAGGER;

inline void check_kv_dtype(int dtype) {
    if (dtype != PA_KV_FP16 && dtype != PA_KV_FP8_E4M3)
        throw std::invalid_argument("unknown kv dtype " + std::to_string(dtype));
}

// Tokens per planning tile (decode.cu:43-45 tile_tokens). The gfx950 kernel
// consumes 16-token groups, so every 16-token boundary is a legal cut.
int kernel_tile_tokens(int dtype, int group);
// Decode work units (waves) resident per CU at the kernel's occupancy.
int kernel_units_per_cu(int dtype, int group);

// Throws std::invalid_argument for unsupported (dtype, head_dim, group);
// returns the launch status otherwise.
hipError_t launch_decode_split(int dtype, const pa_decode_params& p, hipStream_t s);
hipError_t launch_decode_merge(int dtype, const pa_decode_params& p, hipStream_t s);
hipError_t launch_append(int dtype, const uint16_t* k, const uint16_t* v, void* k_cache,
                         void* v_cache, const int32_t* bt_row, int start_pos, int n, int hkv,
                         int page_size, float inv_k, float inv_v, hipStream_t s);
// One launch of the batched append. meta (int32, device), for n_ent entries:
//   tok_begin[n_ent]  first token of each entry in k / v (prefix sums of the counts)
//   old_len[n_ent]    the slot's length before the entry
//   pl_begin[n_ent]   the entry's first page in pages[]
//   pages[n_pl]       per entry, the pages holding positions old_len .. old_len + count - 1
//   tab[2 n_tab]      new block-table entries: flat index, page
//   lens[2 n_len]     new lengths, one per distinct slot: slot, length
struct AppendBatch {
    const uint16_t* k;
    const uint16_t* v;
    void*           k_cache;
    void*           v_cache;
    const int32_t*  meta;
    int32_t*        table;
    int32_t*        seq_lens;
    int             n_ent, n_pl, n_tab, n_len, n_tok;
    int             hkv, page_size;
    float           inv_k, inv_v;
};
hipError_t launch_append_batch(int dtype, const AppendBatch& a, hipStream_t s);
hipError_t launch_gather(int dtype, const void* cache, const int32_t* bt_row, int hkv,
                         int page_size, int kv_head, int len, void* out, hipStream_t s);
hipError_t launch_fill_bytes(void* buf, size_t bytes, int value, hipStream_t s);
// n elements fp32 -> fp16 (RNE) when to_half, else fp16 -> fp32.
hipError_t launch_convert(const void* in, void* out, size_t n, bool to_half, hipStream_t s);
hipError_t launch_stream_read_chunked(const void* buf, size_t bytes, int blocks, int threads, int unroll,
                                     uint32_t* sink, hipStream_t s);
hipError_t launch_stream_read(const void* buf, size_t bytes, int blocks, int threads, int unroll, bool nt,
                              uint32_t* sink, hipStream_t s);

}  // namespace pa
