/*
 * pa_oracle.h — CPU oracle for the paged flash-decoding path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or, for cpu_baseline, as the timed CPU restatement). The product
 * (libpa_decode.so) never calls it.
 *
 * Each function restates the reference's algorithm in plain C, citing the
 * file:line it follows (paths relative to the emaanh/paged-attention tree).
 * How each one is pinned is listed in oracle/README (tests name the checks).
 */
#ifndef PA_ORACLE_H
#define PA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE-754 binary16 <-> binary32 (RNE). */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float x);
void     orc_f32_to_f16_array(const float* x, uint16_t* out, size_t n);
void     orc_f16_to_f32_array(const uint16_t* h, float* out, size_t n);

/* OCP OFP8 E4M3 (bias 7, max 448, NaN = S.1111.111). */
float    orc_e4m3_to_f32(uint8_t b);
/* Nearest E4M3 value (search over the code table), ties to even mantissa; |x| beyond the finite range
 * saturates to +-448 (CUDA __nv_fp8_e4m3(float) semantics: satfinite); NaN -> 0x7f|sign. */
uint8_t  orc_f32_to_e4m3(float x);

/* paged_kv_cache.cu:15-39 append_kernel: token i of [n][hkv][hd] fp16 goes to
 * ((page*hkv + h)*P + pos%P)*hd + d with page = bt_row[pos/P], pos = start+i.
 * dtype 0: fp16 bit copy; 1: e4m3(float(x) * inv_scale) (x * reciprocal, :21/:130). */
void orc_append(int dtype, const uint16_t* k, const uint16_t* v, void* k_cache, void* v_cache,
                const int32_t* bt_row, int start_pos, int n, int hkv, int hd, int page_size,
                float inv_k_scale, float inv_v_scale);

/* The FP8 store of orc_append as a table: out[h] = e4m3(float(fp16 code h) *
 * inv_scale) for all 65536 fp16 codes h (paged_kv_cache.cu:20-22 at one fixed
 * scale). Lets a check of a large FP8 pool look each stored byte up. */
void orc_e4m3_quantize_table(float inv_scale, uint8_t* out);

/* decode_kernels.cuh:175-177 address resolution; raw element bytes of tokens
 * [0,len) of kv head h into out ([len][hd] elements). */
void orc_gather_raw(int dtype, const void* cache, const int32_t* bt_row, int hkv, int hd,
                    int page_size, int h, int len, void* out);

/* Gather + dequantize: fp16 -> float(x); fp8 -> float(x) * scale
 * (tests/test_paged_decode.cu:28-31 `stored`). out is [len][hd] fp32. */
void orc_gather_dequant(int dtype, const void* cache, const int32_t* bt_row, int hkv, int hd,
                        int page_size, int h, int len, float scale, float* out);

/* src/attention/cpu/attention.cpp:5-34 cpu_attention: fp32, sequential dot
 * products, scale 1/sqrt(d), max, expf, normalize, then the weighted sum. */
void orc_cpu_attention(const float* q, const float* K, const float* V, float* out, int T, int d);

/* Multi-head paged decode reference (tests/test_paged_decode.cu:111-145 GQA
 * mapping h = hq / G; scripts/compare_flashinfer.py:113-126 fp32 over the
 * dequantized cache): out[b][hq][:] = cpu_attention(q[b][hq], K_h, V_h) for
 * kv head h = hq / G of batch row b's sequence (table row slot_ids[b] or b).
 * Runs (b, kv head) items on `threads` POSIX threads. */
void orc_paged_decode(int dtype, const uint16_t* q, const void* k_cache, const void* v_cache,
                      const int32_t* block_table, int block_table_stride, const int32_t* slot_ids,
                      const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                      int head_dim, int page_size, float k_scale, float v_scale, float* out,
                      int threads);

/* Signature of src/attention/cpu/attention.hpp cpu_attention(q, K, V, out, T, d). */
typedef void (*orc_attention_fn)(const float* q, const float* K, const float* V, float* out, int T, int d);

/* The CPU baseline's timed loop: for every (batch row b, query head hq) pair,
 * fn(q[b][hq], K[item], V[item], out[b][hq], lens[b], head_dim) with
 * item = b * num_kv_heads + hq / G, over already gathered and dequantized fp32
 * K/V ([len][head_dim] per item). fn NULL = orc_cpu_attention. Pairs are taken
 * from a shared counter by `threads` POSIX threads. Returns the wall seconds of
 * the loop (thread start to join, CLOCK_MONOTONIC). */
double orc_attention_pairs(orc_attention_fn fn, const float* q, const float* const* K,
                           const float* const* V, const int32_t* lens, int batch, int num_q_heads,
                           int num_kv_heads, int head_dim, float* out, int threads);

/* decode.cu:65-108 make_plan, restated as interval intersection: unit u owns
 * global tiles [u*per, (u+1)*per), item i owns its tiles in (row, head) order;
 * every non-empty intersection is a segment (row, head, t0, min(t1, len)).
 * Returns the number of segments, or -1 if a length is <= 0 or an output
 * capacity is too small. num_ctas_out gets the unit count. */
int orc_make_plan(int tile, const int32_t* seq_lens, int batch, int num_kv_heads, int requested,
                  int32_t* segments, int seg_cap, int32_t* cta_seg_begin, int cta_cap,
                  int32_t* item_seg_begin, int* num_ctas_out);

#ifdef __cplusplus
}
#endif

#endif
