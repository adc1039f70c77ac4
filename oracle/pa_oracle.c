/*
 * pa_oracle.c — CPU oracle of the paged flash-decoding path (plain C).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg. libpa_decode.so never calls it.
 *
 * Compiled with -ffp-contract=off so every a*b+c is two roundings, as in the
 * reference's CPU path. See pa_oracle.h for the reference lines each function
 * restates.
 */
#define _POSIX_C_SOURCE 200809L
#include "pa_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ---- binary16 ----------------------------------------------------------- */

float orc_f16_to_f32(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0)
        v = ldexpf((float)m, -24);
    else if (e == 31)
        v = m ? NAN : INFINITY;
    else
        v = ldexpf((float)(m + 1024), e - 25);
    return s ? -v : v;
}

uint16_t orc_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;   /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00u;  /* >= 65520 rounds to infinity */
    if (a < 0x38800000u) {                         /* below 2^-14: subnormal grid m * 2^-24 */
        float ax;
        memcpy(&ax, &a, 4);
        return sign | (uint16_t)rintf(ax * 16777216.0f);
    }
    const uint32_t man = a & 0x7fffffu;
    uint32_t q = ((((a >> 23) - 112u)) << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;
    return sign | (uint16_t)q;
}

void orc_f32_to_f16_array(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_to_f32_array(const uint16_t* h, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(h[i]);
}

/* ---- E4M3 ---------------------------------------------------------------- */

float orc_e4m3_to_f32(uint8_t b) {
    const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7)
        v = NAN;
    else if (e == 0)
        v = ldexpf((float)m, -9);
    else
        v = ldexpf((float)(8 + m), e - 10);
    return s ? -v : v;
}

/* Nearest representable magnitude: binary search for the largest finite code
 * (0x00..0x7e, ascending magnitude) not above |x|, then pick the closer of it
 * and the next code; on a tie the even code (even mantissa) wins. */
uint8_t orc_f32_to_e4m3(float x) {
    if (isnan(x)) return signbit(x) ? 0xff : 0x7f;
    const uint8_t sign = signbit(x) ? 0x80 : 0x00;
    const double a = fabs((double)x);
    if (a >= 448.0) return sign | 0x7e;
    int lo = 0, hi = 0x7e;   /* value(lo) <= a < value(hi) */
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if ((double)orc_e4m3_to_f32((uint8_t)mid) <= a)
            lo = mid;
        else
            hi = mid;
    }
    const double dl = a - (double)orc_e4m3_to_f32((uint8_t)lo);
    const double dh = (double)orc_e4m3_to_f32((uint8_t)hi) - a;
    int best;
    if (dl < dh)
        best = lo;
    else if (dh < dl)
        best = hi;
    else
        best = (lo & 1) == 0 ? lo : hi;
    return sign | (uint8_t)best;
}

/* ---- append / gather ---------------------------------------------------- */

static size_t cache_index(int page, int h, int slot, int d, int hkv, int page_size, int hd) {
    return (((size_t)page * hkv + h) * page_size + slot) * hd + d;
}

void orc_append(int dtype, const uint16_t* k, const uint16_t* v, void* k_cache, void* v_cache,
                const int32_t* bt_row, int start_pos, int n, int hkv, int hd, int page_size,
                float inv_k_scale, float inv_v_scale) {
    for (int i = 0; i < n; i++) {
        const int pos = start_pos + i;
        const int page = bt_row[pos / page_size];
        for (int h = 0; h < hkv; h++)
            for (int d = 0; d < hd; d++) {
                const size_t dst = cache_index(page, h, pos % page_size, d, hkv, page_size, hd);
                const size_t src = ((size_t)i * hkv + h) * hd + d;
                if (dtype == 0) {
                    ((uint16_t*)k_cache)[dst] = k[src];
                    ((uint16_t*)v_cache)[dst] = v[src];
                } else {
                    const float kx = orc_f16_to_f32(k[src]) * inv_k_scale;
                    const float vx = orc_f16_to_f32(v[src]) * inv_v_scale;
                    ((uint8_t*)k_cache)[dst] = orc_f32_to_e4m3(kx);
                    ((uint8_t*)v_cache)[dst] = orc_f32_to_e4m3(vx);
                }
            }
    }
}

void orc_e4m3_quantize_table(float inv_scale, uint8_t* out) {
    for (uint32_t h = 0; h < 65536u; h++) out[h] = orc_f32_to_e4m3(orc_f16_to_f32((uint16_t)h) * inv_scale);
}

void orc_gather_raw(int dtype, const void* cache, const int32_t* bt_row, int hkv, int hd,
                    int page_size, int h, int len, void* out) {
    const size_t eb = dtype == 0 ? 2 : 1;
    for (int t = 0; t < len; t++) {
        const int page = bt_row[t / page_size];
        const size_t src = cache_index(page, h, t % page_size, 0, hkv, page_size, hd);
        memcpy((char*)out + (size_t)t * hd * eb, (const char*)cache + src * eb, hd * eb);
    }
}

void orc_gather_dequant(int dtype, const void* cache, const int32_t* bt_row, int hkv, int hd,
                        int page_size, int h, int len, float scale, float* out) {
    for (int t = 0; t < len; t++) {
        const int page = bt_row[t / page_size];
        const size_t src = cache_index(page, h, t % page_size, 0, hkv, page_size, hd);
        for (int d = 0; d < hd; d++) {
            if (dtype == 0)
                out[(size_t)t * hd + d] = orc_f16_to_f32(((const uint16_t*)cache)[src + d]);
            else
                out[(size_t)t * hd + d] = orc_e4m3_to_f32(((const uint8_t*)cache)[src + d]) * scale;
        }
    }
}

/* ---- attention ----------------------------------------------------------- */

void orc_cpu_attention(const float* q, const float* K, const float* V, float* out, int T, int d) {
    float* scores = (float*)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
    const float scale = 1.0f / sqrtf((float)d);
    float max_score = -INFINITY;
    for (int i = 0; i < T; i++) {
        float dot = 0.0f;
        for (int j = 0; j < d; j++) dot += q[j] * K[(size_t)i * d + j];
        scores[i] = dot * scale;
        if (scores[i] > max_score) max_score = scores[i];
    }
    float sum = 0.0f;
    for (int i = 0; i < T; i++) {
        scores[i] = expf(scores[i] - max_score);
        sum += scores[i];
    }
    for (int i = 0; i < T; i++) scores[i] /= sum;
    for (int j = 0; j < d; j++) {
        float s = 0.0f;
        for (int i = 0; i < T; i++) s += scores[i] * V[(size_t)i * d + j];
        out[j] = s;
    }
    free(scores);
}

typedef struct {
    int dtype;
    const uint16_t* q;
    const void* k_cache;
    const void* v_cache;
    const int32_t* block_table;
    int stride;
    const int32_t* slot_ids;
    const int32_t* seq_lens;
    int batch, hq, hkv, hd, page_size;
    float k_scale, v_scale;
    float* out;
    int next;   /* next item, taken under the lock */
    pthread_mutex_t lock;
} decode_job;

static void* decode_worker(void* arg) {
    decode_job* j = (decode_job*)arg;
    const int group = j->hq / j->hkv;
    size_t cap = 0;
    float *K = NULL, *V = NULL;
    float* qf = (float*)malloc(sizeof(float) * (size_t)j->hd);
    for (;;) {
        pthread_mutex_lock(&j->lock);
        const int item = j->next++;
        pthread_mutex_unlock(&j->lock);
        if (item >= j->batch * j->hkv) break;
        const int b = item / j->hkv, h = item % j->hkv;
        const int len = j->seq_lens[b];
        const int slot = j->slot_ids ? j->slot_ids[b] : b;
        const int32_t* row = j->block_table + (size_t)slot * j->stride;
        const size_t need = (size_t)len * j->hd;
        if (need > cap) {
            free(K);
            free(V);
            K = (float*)malloc(sizeof(float) * need);
            V = (float*)malloc(sizeof(float) * need);
            cap = need;
        }
        orc_gather_dequant(j->dtype, j->k_cache, row, j->hkv, j->hd, j->page_size, h, len, j->k_scale, K);
        orc_gather_dequant(j->dtype, j->v_cache, row, j->hkv, j->hd, j->page_size, h, len, j->v_scale, V);
        for (int g = 0; g < group; g++) {
            const int hq = h * group + g;
            const size_t off = ((size_t)b * j->hq + hq) * j->hd;
            for (int d = 0; d < j->hd; d++) qf[d] = orc_f16_to_f32(j->q[off + d]);
            orc_cpu_attention(qf, K, V, j->out + off, len, j->hd);
        }
    }
    free(K);
    free(V);
    free(qf);
    return NULL;
}

void orc_paged_decode(int dtype, const uint16_t* q, const void* k_cache, const void* v_cache,
                      const int32_t* block_table, int block_table_stride, const int32_t* slot_ids,
                      const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                      int head_dim, int page_size, float k_scale, float v_scale, float* out,
                      int threads) {
    decode_job job = {dtype, q, k_cache, v_cache, block_table, block_table_stride, slot_ids, seq_lens,
                      batch, num_q_heads, num_kv_heads, head_dim, page_size,
                      dtype == 0 ? 1.0f : k_scale, dtype == 0 ? 1.0f : v_scale, out, 0,
                      PTHREAD_MUTEX_INITIALIZER};
    if (threads < 1) threads = 1;
    pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int t = 0; t < threads; t++) pthread_create(&tid[t], NULL, decode_worker, &job);
    for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
    free(tid);
    pthread_mutex_destroy(&job.lock);
}

typedef struct {
    orc_attention_fn fn;
    const float* q;
    const float* const* K;
    const float* const* V;
    const int32_t* lens;
    int batch, hq, hkv, hd;
    float* out;
    int next;
    pthread_mutex_t lock;
} pairs_job;

static void* pairs_worker(void* arg) {
    pairs_job* j = (pairs_job*)arg;
    const int group = j->hq / j->hkv;
    for (;;) {
        pthread_mutex_lock(&j->lock);
        const int pair = j->next++;
        pthread_mutex_unlock(&j->lock);
        if (pair >= j->batch * j->hq) break;
        const int b = pair / j->hq, hq = pair % j->hq;
        const int item = b * j->hkv + hq / group;
        const size_t off = (size_t)pair * j->hd;
        j->fn(j->q + off, j->K[item], j->V[item], j->out + off, j->lens[b], j->hd);
    }
    return NULL;
}

double orc_attention_pairs(orc_attention_fn fn, const float* q, const float* const* K,
                           const float* const* V, const int32_t* lens, int batch, int num_q_heads,
                           int num_kv_heads, int head_dim, float* out, int threads) {
    pairs_job job = {fn ? fn : orc_cpu_attention, q, K, V, lens, batch, num_q_heads, num_kv_heads,
                     head_dim, out, 0, PTHREAD_MUTEX_INITIALIZER};
    if (threads < 1) threads = 1;
    pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int t = 0; t < threads; t++) pthread_create(&tid[t], NULL, pairs_worker, &job);
    for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
    clock_gettime(CLOCK_MONOTONIC, &t1);
    free(tid);
    pthread_mutex_destroy(&job.lock);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* ---- planner ------------------------------------------------------------ */

int orc_make_plan(int tile, const int32_t* seq_lens, int batch, int num_kv_heads, int requested,
                  int32_t* segments, int seg_cap, int32_t* cta_seg_begin, int cta_cap,
                  int32_t* item_seg_begin, int* num_ctas_out) {
    const int items = batch * num_kv_heads;
    long total = 0;
    for (int b = 0; b < batch; b++) {
        if (seq_lens[b] <= 0) return -1;
        total += (long)((seq_lens[b] + tile - 1) / tile) * num_kv_heads;
    }
    for (int i = 0; i <= items; i++) item_seg_begin[i] = 0;
    if (total == 0) {
        *num_ctas_out = 0;
        if (cta_cap < 1) return -1;
        cta_seg_begin[0] = 0;
        return 0;
    }
    const long per = (total + requested - 1) / requested;
    const long units = (total + per - 1) / per;
    if (units + 1 > cta_cap) return -1;
    int nseg = 0;
    int item = 0;
    long item_start = 0;   /* global index of item's first tile */
    for (long u = 0; u < units; u++) {
        cta_seg_begin[u] = nseg;
        const long lo = u * per;
        const long hi = lo + per < total ? lo + per : total;
        while (item < items) {
            const int b = item / num_kv_heads;
            const long n_tiles = (seq_lens[b] + tile - 1) / tile;
            const long a = lo > item_start ? lo : item_start;
            const long z = hi < item_start + n_tiles ? hi : item_start + n_tiles;
            if (a < z) {
                if (nseg >= seg_cap) return -1;
                const long t1 = (z - item_start) * tile;
                segments[4 * nseg + 0] = b;
                segments[4 * nseg + 1] = item % num_kv_heads;
                segments[4 * nseg + 2] = (int32_t)((a - item_start) * tile);
                segments[4 * nseg + 3] = (int32_t)(t1 < seq_lens[b] ? t1 : seq_lens[b]);
                item_seg_begin[item + 1]++;
                nseg++;
            }
            if (item_start + n_tiles <= hi) {
                item_start += n_tiles;
                item++;
            } else {
                break;
            }
        }
    }
    cta_seg_begin[units] = nseg;
    for (int i = 0; i < items; i++) item_seg_begin[i + 1] += item_seg_begin[i];
    *num_ctas_out = (int)units;
    return nseg;
}
