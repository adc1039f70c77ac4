/*
 * pa_decode.h — C ABI of the MI355X (gfx950) paged flash-decoding library
 * (libpa_decode.so).
 *
 * This is the drop-in boundary for the reference's `src/decode` path
 * (emaanh/paged-attention). Every entry point takes plain pointers, sizes and
 * scalars; device pointers are HIP device addresses and `stream` is a
 * hipStream_t passed as `void*` (NULL = the default stream). No entry point
 * throws: each returns a pa_status and, on failure, leaves a message that
 * pa_last_error() returns (thread-local).
 *
 * Error mapping (reference -> this ABI):
 *   std::invalid_argument             -> PA_ERR_INVALID_ARGUMENT
 *   std::length_error                 -> PA_ERR_LENGTH
 *   CUDA_CHECK abort() (cuda_check.hpp:9-17) -> PA_ERR_DEVICE (the C++ wrapper
 *                                        in paged-attention_amd/cpp aborts, as
 *                                        the reference does)
 *   append() returning false          -> PA_OK with *appended = 0
 *   admit() returning -1              -> return value -1
 *
 * Layouts (HND, as the reference):
 *   q, out        [batch][num_q_heads][head_dim] fp16
 *   k/v cache     [num_pages][num_kv_heads][page_size][head_dim] fp16 or fp8 e4m3
 *   block_table   [num_slots][block_table_stride] int32 physical page ids
 *   segments      [num_segments][4] int32 = (batch row, kv head, tok_begin, tok_end)
 */
#ifndef PA_DECODE_H
#define PA_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum pa_status {
    PA_OK                   = 0,
    PA_ERR_INVALID_ARGUMENT = 1,
    PA_ERR_LENGTH           = 2,
    PA_ERR_DEVICE           = 3
} pa_status;

/* decode_types.hpp:8 `enum class KVDtype { FP16, FP8_E4M3 }` */
typedef enum pa_kv_dtype {
    PA_KV_FP16     = 0,
    PA_KV_FP8_E4M3 = 1
} pa_kv_dtype;

/* decode_types.hpp:14-45 `struct DecodeParams`, with plain C types:
 * half* -> uint16_t*, int4* -> int32_t* ([n][4]). `seq_lens` is carried but,
 * as in the reference, never read by the kernels (lengths come from the
 * segments). */
typedef struct pa_decode_params {
    const uint16_t* q;
    uint16_t*       out;
    const void*     k_cache;
    const void*     v_cache;
    const int32_t*  block_table;
    const int32_t*  seq_lens;
    const int32_t*  slot_ids;          /* NULL => identity */
    int32_t         block_table_stride;
    int32_t         batch;
    int32_t         num_q_heads;
    int32_t         num_kv_heads;
    int32_t         head_dim;
    int32_t         page_size;
    float           sm_scale;
    float           k_scale;
    float           v_scale;
    const int32_t*  segments;          /* [num_segments][4] */
    const int32_t*  cta_seg_begin;     /* [num_ctas + 1] */
    const int32_t*  item_seg_begin;    /* [batch * num_kv_heads + 1] */
    int32_t         num_ctas;
    int32_t         needs_merge;
    float*          partial_out;       /* [num_segments][group][head_dim] */
    float*          partial_lse;       /* [num_segments][group] */
    int32_t         max_item_segments; /* most segments of one (row, kv head); sizes the
                                          merge launch (0 = unknown). Set by bind. */
    int32_t         block_merge;       /* How the split kernel merges split (row, kv head)
                                          items itself (needs_merge is then 0; the launches
                                          refuse both set). Set by bind.
                                          0: it does not (the merge kernel does, if
                                          needs_merge). 1: every split item lies in one
                                          block of 8 work units and is merged there in LDS.
                                          2: items spanning blocks are also merged in the
                                          split kernel: each block writes one partial per
                                          such item to the workspace, and the last block
                                          to finish (merge_counters) combines them. */
    int32_t         num_segments;      /* segments of the bound plan (0 = unknown); sizes the
                                          partial workspace. Set by bind. */
    int32_t*        merge_counters;    /* block_merge 2: one arrival counter per item, zero
                                          between decodes (the plan zeroes them at upload;
                                          every decode leaves them at zero). Set by bind. */
} pa_decode_params;

/* Thread-local message describing the last failed call ("" if none). */
const char* pa_last_error(void);

/* decode_types.hpp:10 kv_dtype_bytes; :11 kv_dtype_name ("fp16" / "fp8_e4m3"). */
int         pa_kv_dtype_bytes(int dtype);
const char* pa_kv_dtype_name(int dtype);

/* ---- planner (decode.hpp:21-41, decode.cu:43-108) ------------------------ */

/* decode.cu:43-45 tile_tokens: tokens per planning tile of the gfx950 kernel. */
pa_status pa_tile_tokens(int dtype, int head_dim, int group, int* out);
/* decode.cu:47-53 wave_ctas: work units (waves) resident in one full wave of
 * the decode kernel on the current device. */
pa_status pa_wave_ctas(int dtype, int head_dim, int group, int* out);
/* decode.cu:55-63 default_ctas: persistent grid used when a plan asks for 0. */
pa_status pa_default_ctas(int dtype, int head_dim, int group, int* out);

typedef struct pa_plan pa_plan;   /* host copy of decode.hpp:21-27 DecodePlan */

/* decode.cu:65-108 make_plan(dtype, seq_lens, hq, hkv, hd, num_ctas).
 * num_ctas <= 0 uses pa_default_ctas (needs a device); otherwise pure host. */
pa_status pa_plan_build(int dtype, const int32_t* seq_lens, int batch, int num_q_heads,
                        int num_kv_heads, int head_dim, int num_ctas, pa_plan** out);
/* The same equal-range cut with an explicit tile and grid (pure host). Used to
 * replay the reference planner at its own tile (64) in tests. */
pa_status pa_plan_build_tiled(int tile, const int32_t* seq_lens, int batch, int num_kv_heads,
                              int num_ctas, pa_plan** out);
/* A plan from caller-built host arrays (decode.hpp:21-27 DecodePlan's fields),
 * validated: prefix arrays rise from 0 to num_segments, every segment is
 * non-empty and listed under its (row, kv head) item = row * num_kv_heads +
 * head, every item has a segment and every segment starts on a multiple of 16
 * tokens (the kernels' step; the reference's plans start on its 64-token
 * tiles). num_kv_heads = 0 infers it (1 + the largest head in the segments).
 * Lets DevicePlan::upload take any DecodePlan. */
pa_status pa_plan_create(int num_ctas, int tile, const int32_t* segments, int num_segments,
                         const int32_t* cta_seg_begin, const int32_t* item_seg_begin, int num_items,
                         int num_kv_heads, pa_plan** out);
void      pa_plan_destroy(pa_plan* plan);
int       pa_plan_num_ctas(const pa_plan* plan);
int       pa_plan_tile(const pa_plan* plan);
int       pa_plan_num_segments(const pa_plan* plan);
int       pa_plan_num_items(const pa_plan* plan);
/* How the split kernel merges this plan's split items, as DevicePlan::bind
 * sets pa_decode_params.block_merge (0, 1 or 2; see there). No counterpart in
 * the reference, whose plans always merge in a second kernel
 * (decode.cu:143 needs_merge). Pure host. */
pa_status pa_plan_merge_mode(const pa_plan* plan, int* out);
/* Copies segments ([n][4]), cta_seg_begin ([num_ctas+1]) and item_seg_begin
 * ([items+1]); any output may be NULL. */
pa_status pa_plan_copy(const pa_plan* plan, int32_t* segments, int32_t* cta_seg_begin,
                       int32_t* item_seg_begin);

typedef struct pa_device_plan pa_device_plan;   /* decode.hpp:44-63 DevicePlan */

pa_status pa_device_plan_create(pa_device_plan** out);
void      pa_device_plan_destroy(pa_device_plan* dp);
/* decode.cu:131-146 DevicePlan::upload: grow-only device copies of the plan plus
 * the partial workspace (segments * group * (head_dim + 1) floats). Rejects a
 * plan whose segments do not start on multiples of 16 tokens. The plan's arrays
 * go through pinned staging as one copy queued on `stream`; the call does not
 * synchronize the stream (it waits only when 8 of its uploads are still in
 * flight, and synchronizes once when a plan outgrows every earlier one), and
 * the host plan may change or go as soon as it returns. Decodes queued earlier
 * on `stream` still see the previous plan. */
pa_status pa_device_plan_upload(pa_device_plan* dp, const pa_plan* plan, int group, int head_dim,
                                void* stream);
/* decode.cu:148-156 DevicePlan::bind: points the schedule fields of *p at it. */
pa_status pa_device_plan_bind(const pa_device_plan* dp, pa_decode_params* p);

/* ---- kernels ------------------------------------------------------------- */

/* decode.cu:158-165 paged_decode: split-KV decode kernel, then the merge
 * kernel when a (row, kv head) spans several segments. head_dim must be 128;
 * num_q_heads / num_kv_heads in {1, 2, 4, 8}. */
pa_status pa_decode(int dtype, const pa_decode_params* p, void* stream);
/* The two launches of decode_kernels.cuh:450-458 separately: the split kernel
 * (paged_decode_kernel) and the LSE merge (merge_segments_kernel; a no-op when
 * p->needs_merge is 0). pa_decode == pa_decode_split + pa_decode_merge. */
pa_status pa_decode_split(int dtype, const pa_decode_params* p, void* stream);
pa_status pa_decode_merge(int dtype, const pa_decode_params* p, void* stream);
/* No counterpart in the reference. pa_decode for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): the same split and merge launches, but the partial
 * workspace of rows split across blocks lives in a fixed 32 MiB device array
 * of the library (one per GPU, held until the process ends) instead of
 * p->partial_out / p->partial_lse, which are ignored. p must be bound to a
 * device plan (pa_device_plan_bind records the plan's segment count in
 * p->num_segments), and num_segments must equal that count
 * (pa_plan_num_segments); anything else is refused with
 * PA_ERR_INVALID_ARGUMENT before any launch. A plan whose workspace,
 * num_segments * group * (head_dim + 1) * 4 bytes, exceeds 32 MiB is refused
 * with PA_ERR_LENGTH; plans without split rows, or merged in the split kernel
 * (p->block_merge = 1), need none. The array's address is looked up by the
 * plan upload on the device (so a first call made under graph capture needs
 * no lookup); a first call on a device that has seen no upload looks it up
 * itself, and refuses to while its stream is being captured. Allocates
 * nothing. Calls on one GPU share its array: calls that overlap on one GPU
 * (two streams, two threads) race. */
pa_status pa_decode_static(int dtype, const pa_decode_params* p, int num_segments, void* stream);

/* paged_kv_cache.cu:15-39 quantize<> + append_kernel, launch at :122-131:
 * scatters n tokens of fp16 K/V ([n][num_kv_heads][head_dim]) into pages
 * resolved through block_table_row, token i going to position start_pos + i.
 * fp16: bit copy; fp8: e4m3(RNE, saturate to +-448)(float(x) * inv_scale). */
pa_status pa_append_quantize(int dtype, const uint16_t* k, const uint16_t* v, void* k_cache,
                             void* v_cache, const int32_t* block_table_row, int start_pos, int n,
                             int num_kv_heads, int head_dim, int page_size, float inv_k_scale,
                             float inv_v_scale, void* stream);

/* Block-table resolution probe (decode_kernels.cuh:175-177's address, with the
 * decode kernel's own device function): copies the raw cache bytes of tokens
 * [0, len) of one kv head into out ([len][head_dim] elements of the cache type). */
pa_status pa_gather_kv(int dtype, const void* cache, const int32_t* block_table_row,
                       int num_kv_heads, int head_dim, int page_size, int kv_head, int len,
                       void* out, void* stream);

/* bench_decode.cu:70-78 read_kernel: 16 B/lane streaming read of `bytes`
 * (multiple of 16) with `blocks` x 256 threads; the cache flush and the
 * plain-copy ceiling. */
pa_status pa_stream_read(const void* buf, size_t bytes, int blocks, uint32_t* sink, void* stream);
/* The same read with threads_per_block in {256, 512}, unroll in {1, 2, 4, 8}
 * independent 16 B loads per lane per trip, and optionally non-temporal loads:
 * the copy-ceiling variants (bench_decode.cu:224-240 uses 512 threads, unroll 1). */
pa_status pa_stream_read_ex(const void* buf, size_t bytes, int blocks, int threads_per_block, int unroll,
                            int nontemporal, uint32_t* sink, void* stream);

/* The same read with each wave streaming one contiguous span: `bytes` splits
 * into blocks x threads/64 equal spans, each a multiple of unroll KiB
 * (unroll in {8, 16}, threads in {256, 512}); non-temporal 16 B loads. The
 * highest-rate read shape on MI355X, reported as the read ceiling beside
 * bench_decode.cu:224-240's grid-stride copy rows. */
pa_status pa_stream_read_chunked(const void* buf, size_t bytes, int blocks, int threads_per_block, int unroll,
                                 uint32_t* sink, void* stream);

/* Streaming write of the byte `value` over `bytes` (a multiple of 16): the
 * write-side counterpart of pa_stream_read (bench_decode.cu:61-68 fills the
 * bench inputs; here it is a write of known size for counter calibration). */
pa_status pa_fill_bytes(void* buf, size_t bytes, int value, void* stream);

/* n device elements fp32 -> fp16 (round to nearest even) and fp16 -> fp32
 * (exact). No counterpart of their own in the reference: the legacy pool's FP32
 * device entry (src/attention/paged_pool/pool.hpp:21-24 decode_device) converts
 * its q and out with them around the fp16 decode. */
pa_status pa_f32_to_f16(const float* in, uint16_t* out, size_t n, void* stream);
pa_status pa_f16_to_f32(const uint16_t* in, float* out, size_t n, void* stream);

/* ---- host page pool (paged_kv_cache.cu:84-151, no device memory) -------- */

typedef struct pa_pool pa_pool;

/* paged_kv_cache.cu:51-74 sizes and free list [N-1..0] (page 0 handed out first). */
pa_status pa_pool_create(int num_pages, int page_size, int max_slots, int max_pages_per_slot,
                         pa_pool** out);
void      pa_pool_destroy(pa_pool* pool);
/* paged_kv_cache.cu:84-93 admit: first free slot, or -1. */
int       pa_pool_admit(pa_pool* pool);
/* paged_kv_cache.cu:95-113 append's bookkeeping: grows `slot` by n tokens.
 * *ok = 0 (nothing changed) when the pool lacks pages; PA_ERR_LENGTH when the
 * slot would exceed max_pages_per_slot; PA_ERR_INVALID_ARGUMENT for a slot
 * that is not admitted. *first_new / *num_new give the new table entries. */
pa_status pa_pool_reserve(pa_pool* pool, int slot, int n, int* ok, int* first_new, int* num_new);
/* paged_kv_cache.cu:138-146 release. */
/* The bookkeeping of append_batch below, one call for many slots:
 * pa_pool_reserve(slots[i], counts[i]) for i = 0..n-1 in order, but
 * all-or-nothing (*ok = 0, nothing changed, when the whole batch does not fit;
 * errors raised before anything changes). Grows the reference's per-call
 * reserve (paged_kv_cache.cu:95-121) to a batch. */
pa_status pa_pool_reserve_batch(pa_pool* pool, const int32_t* slots, const int32_t* counts, int n, int* ok);
pa_status pa_pool_release(pa_pool* pool, int slot);
/* paged_kv_cache.cu:148-151 shuffle_free_pages: std::shuffle(mt19937(seed)). */
void      pa_pool_shuffle_free_pages(pa_pool* pool, unsigned seed);
int       pa_pool_free_pages(const pa_pool* pool);
int       pa_pool_seq_len(const pa_pool* pool, int slot);
int       pa_pool_occupied(const pa_pool* pool, int slot);
int       pa_pool_max_seq_len(const pa_pool* pool);
int       pa_pool_num_pages_of(const pa_pool* pool, int slot);
/* Copies up to cap table entries of `slot` (paged_kv_cache.hpp:73 block_table). */
pa_status pa_pool_block_table(const pa_pool* pool, int slot, int32_t* out, int cap);

/* ---- paged KV cache (paged_kv_cache.hpp:17-93) --------------------------- */

/* paged_kv_cache.hpp:19-29 PagedKVCache::Config. */
typedef struct pa_cache_config {
    int32_t num_pages;
    int32_t page_size;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t max_slots;
    int32_t max_pages_per_slot;
    int32_t dtype;      /* pa_kv_dtype */
    float   k_scale;    /* stored = value * (1/scale), FP8 only */
    float   v_scale;
} pa_cache_config;

typedef struct pa_cache pa_cache;

/* paged_kv_cache.cu:43-45 bytes_per_page; :47-49 pages_for_budget. */
size_t    pa_cache_bytes_per_page(const pa_cache_config* cfg);
int       pa_cache_pages_for_budget(const pa_cache_config* cfg, size_t budget_bytes);
/* paged_kv_cache.cu:51-74 constructor (device pools, table, seq_lens). The K
 * and V pools share one allocation, V starting pa_kv_pool_stagger() bytes
 * after the end of K. */
pa_status pa_cache_create(const pa_cache_config* cfg, pa_cache** out);
/* No counterpart in the reference: the byte gap this library leaves between
 * the end of its K pool and the start of its V pool. A wave reads the same
 * (page, kv head) run of both pools at once, and pools at the same offset
 * modulo a large power of two put those reads on the same HBM banks (a decode
 * step 3-7% slower on MI355X). Callers that allocate their own pools for
 * pa_decode or the torch Decoder get the same placement by allocating both
 * pools at once with V this many bytes after the end of K. */
size_t    pa_kv_pool_stagger(void);
void      pa_cache_destroy(pa_cache* cache);
/* Host bookkeeping view (seq_len, free_pages, block tables, ...). */
pa_pool*  pa_cache_pool(pa_cache* cache);
int       pa_cache_admit(pa_cache* cache);
/* paged_kv_cache.cu:95-136 append (synchronizes `stream`, as the reference). */
pa_status pa_cache_append(pa_cache* cache, int slot, const uint16_t* d_k, const uint16_t* d_v,
                          int n, void* stream, int* appended);
/* paged_kv_cache.cu:95-136 append, batched across sequences: appends counts[i]
 * tokens to slots[i] for i = 0..n-1 (host arrays; a slot may repeat, its
 * tokens then follow in order). d_k / d_v hold every token, concatenated in
 * entry order: [sum(counts)][Hkv][D] fp16. Pages are reserved all-or-nothing
 * (*appended = 0 and nothing changed when the pool lacks pages). The new
 * block-table entries and lengths go over in one pinned host-to-device copy and
 * one kernel writes them together with every token (copy or E4M3 quantize): two
 * stream operations, no stream synchronization. The call returns once its host
 * staging is queued; it waits only when 8 of its batches are still in flight. */
pa_status pa_cache_append_batch(pa_cache* cache, const int32_t* slots, const int32_t* counts, int n,
                                const uint16_t* d_k, const uint16_t* d_v, void* stream, int* appended);
pa_status pa_cache_release(pa_cache* cache, int slot);
void      pa_cache_shuffle_free_pages(pa_cache* cache, unsigned seed);
/* paged_kv_cache.cu:157-171 params(): cache-side fields of DecodeParams. */
pa_status pa_cache_params(const pa_cache* cache, pa_decode_params* p);
/* paged_kv_cache.cu:173-191 plan(slots, num_q_heads, num_ctas). Queues the plan
 * and the slot ids like pa_device_plan_upload: no stream synchronization. */
pa_status pa_cache_plan(pa_cache* cache, const int32_t* slots, int n, int num_q_heads,
                        int num_ctas, void* stream);
/* paged_kv_cache.cu:193-202 run(q, out). */
pa_status pa_cache_run(pa_cache* cache, const uint16_t* d_q, uint16_t* d_out, void* stream);
/* paged_kv_cache.cu:204-210 decode = plan(0..batch-1) + run. */
pa_status pa_cache_decode(pa_cache* cache, const uint16_t* d_q, uint16_t* d_out, int batch,
                          int num_q_heads, int num_ctas, void* stream);
/* paged_kv_cache.hpp:62 last_plan(). Owned by the cache. */
const pa_plan* pa_cache_last_plan(const pa_cache* cache);
/* paged_kv_cache.hpp:71 total_bytes(). */
size_t    pa_cache_total_bytes(const pa_cache* cache);

#ifdef __cplusplus
}
#endif

#endif /* PA_DECODE_H */
