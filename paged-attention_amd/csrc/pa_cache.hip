// gfx950 kernels around the decode path:
//
//   append_kernel        fp16 copy / FP8 E4M3 quantize + page scatter (paged_kv_cache.cu:15-39)
//   append_batch_kernel  the same for a whole decode step's appends across sequences, plus the
//                        new block-table entries and lengths, in one launch
//   gather_kernel        block-table resolution probe (the decode kernel's row address function)
//   stream_read_kernel   streaming read: cache flush and plain-copy ceiling (bench_decode.cu:70-78)
//   stream_read_chunked_kernel  the same read with one contiguous span per wave (best read rate)
//   fill_bytes_kernel    streaming write of a byte value (bench_decode.cu:61-68's fill role; the
//                        write-side counterpart of the copy ceiling)
//   f32_to_f16_kernel, f16_to_f32_kernel  element conversions for the legacy pool's fp32 device entry

#include "pa_device.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <type_traits>

namespace pa {
namespace {

// ---------------------------------------------------------------------------
// FP8 E4M3 encoder, written from the OCP OFP8 definition (bias 7, max normal
// 448 = S.1111.110, NaN = S.1111.111, subnormals m * 2^-9): round to nearest
// even, finite overflow and infinities saturate to +-448, NaN stays NaN.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
    const uint32_t u    = __builtin_bit_cast(uint32_t, x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a    = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7fu;    // NaN
    if (a >= 0x43e00000u) return sign | 0x7eu;   // |x| >= 448: saturate
    if (a < 0x3c800000u) {                       // |x| < 2^-6: subnormal grid
        const float ax = __builtin_bit_cast(float, a);
        return sign | static_cast<uint32_t>(rintf(ax * 512.0f));   // 0..8; 8 is the min normal
    }
    const uint32_t man = a & 0x7fffffu;
    uint32_t q = (((a >> 23) - 120u) << 3) | (man >> 20);
    const uint32_t rem = man & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q += 1u;
    return sign | q;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h16)));
}

// Streaming (non-temporal) loads of the new tokens and stores into the pages:
// both are touched once per append.
#ifndef PA_APPEND_NT
#define PA_APPEND_NT 1
#endif
constexpr bool kAppendNT = PA_APPEND_NT != 0;

// E4M3 encode of eight products float(x) * inv through gfx950's OCP FP8
// conversion (v_cvt_scalef32_pk_fp8_f32, scale 1): each product is rounded to
// fp32 first, as e4m3_encode's argument is. Finite values are clamped to
// +-448 beforehand (saturation, and infinities). The instruction writes every
// NaN as 0xff; a chunk holding a NaN takes e4m3_encode instead, which keeps
// the sign (0x7f | sign), as the software path and the oracle do.
#ifndef PA_APPEND_HWCVT
#define PA_APPEND_HWCVT 1
#endif
constexpr bool kAppendHwCvt = PA_APPEND_HWCVT != 0;

typedef short v2i16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float sat448(float x) { return __builtin_fminf(__builtin_fmaxf(x, -448.0f), 448.0f); }

__device__ __forceinline__ u32x2 encode8_hw(const u32x4 in, float inv) {
    float f[8];
    bool  nan = false;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        f[e] = f16_bits_to_f32((in[e >> 1] >> (16 * (e & 1))) & 0xffffu) * inv;
        nan |= f[e] != f[e];
    }
    u32x2 out = {0u, 0u};
    if (__builtin_expect(nan, 0)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e >> 2] |= e4m3_encode(f[e]) << (8 * (e & 3));
        return out;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = sat448(f[e]);
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        v2i16 r = {0, 0};
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, f[4 * w + 0], f[4 * w + 1], 1.0f, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, f[4 * w + 2], f[4 * w + 3], 1.0f, true);
        out[w] = __builtin_bit_cast(uint32_t, r);
    }
    return out;
}

// E4M3 bytes of eight products float(x) * inv, in software (e4m3_encode).
[[maybe_unused]] __device__ __forceinline__ u32x2 encode8_sw(const u32x4 in, float inv) {
    u32x2 out = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e)
        out[e >> 2] |= e4m3_encode(f16_bits_to_f32((in[e >> 1] >> (16 * (e & 1))) & 0xffffu) * inv) << (8 * (e & 3));
    return out;
}

__device__ __forceinline__ u32x2 encode8(const u32x4 in, float inv) {
    if constexpr (kAppendHwCvt) return encode8_hw(in, inv);
    else return encode8_sw(in, inv);
}

// Dims of one row that one thread appends: 8 for fp16 (one 16-byte load and
// one 16-byte store per pool), 16 for FP8 (two 16-byte loads of fp16, one
// 16-byte store of E4M3 bytes).
template <int EB>
constexpr int kAppendDims = EB == 2 ? 8 : 16;

template <bool NT, typename T>
__device__ __forceinline__ void store_raw(T x, unsigned char* p) {
    if constexpr (NT) __builtin_nontemporal_store(x, reinterpret_cast<T*>(p));
    else *reinterpret_cast<T*>(p) = x;
}

// One kAppendDims-dim chunk of fp16 K and V (one or two 16-byte words each).
template <int EB>
struct ChunkIn {
    u32x4 k[EB == 2 ? 1 : 2], v[EB == 2 ? 1 : 2];
};

// Loads the chunk at element offset src of k / v. The kernels issue these
// loads before they look up the destination page, so the two overlap, and
// before any store: a store may alias the inputs as far as the compiler
// knows, so a load after it would wait for it.
template <int EB>
__device__ __forceinline__ ChunkIn<EB> load_chunk(const uint16_t* k, const uint16_t* v, size_t src) {
    ChunkIn<EB> in;
#pragma unroll
    for (int w = 0; w < (EB == 2 ? 1 : 2); ++w) {
        in.k[w] = load16<kAppendNT>(k + src + 8 * w);
        in.v[w] = load16<kAppendNT>(v + src + 8 * w);
    }
    return in;
}

// Stores a chunk at byte offset dst of the pools, as a bit copy (fp16) or
// e4m3(float(x) * inv_scale) (FP8, paged_kv_cache.cu:15-22).
template <int EB>
__device__ __forceinline__ void store_chunk(const ChunkIn<EB>& in, void* k_cache, void* v_cache, size_t dst,
                                            float inv_k, float inv_v) {
    unsigned char* kc = static_cast<unsigned char*>(k_cache) + dst;
    unsigned char* vc = static_cast<unsigned char*>(v_cache) + dst;
    if constexpr (EB == 2) {
        store_raw<kAppendNT>(in.k[0], kc);
        store_raw<kAppendNT>(in.v[0], vc);
    } else {
        const u32x2 ka = encode8(in.k[0], inv_k), kb = encode8(in.k[1], inv_k);
        const u32x2 va = encode8(in.v[0], inv_v), vb = encode8(in.v[1], inv_v);
        store_raw<kAppendNT>(u32x4{ka[0], ka[1], kb[0], kb[1]}, kc);
        store_raw<kAppendNT>(u32x4{va[0], va[1], vb[0], vb[1]}, vc);
    }
}

// One thread per (token, kv head, chunk of kAppendDims dims); token i goes to
// position start_pos + i of the sequence whose block-table row is bt_row.
template <int EB>
__global__ __launch_bounds__(256) void append_kernel(const uint16_t* __restrict__ k,
                                                     const uint16_t* __restrict__ v, void* k_cache,
                                                     void* v_cache, const int32_t* __restrict__ bt_row,
                                                     int start_pos, int n, int hkv, int page_size,
                                                     float inv_k, float inv_v) {
    constexpr int DIMS = kAppendDims<EB>, CPR = kHeadDim / DIMS;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n * hkv * CPR) return;
    const int chunk = static_cast<unsigned>(idx) % CPR;   // idx >= 0: a mask and a shift
    const int th    = static_cast<unsigned>(idx) / CPR;
    const int h     = th % hkv;
    const int i     = th / hkv;
    const ChunkIn<EB> in = load_chunk<EB>(k, v, (static_cast<size_t>(i) * hkv + h) * kHeadDim + DIMS * chunk);
    const int pos   = start_pos + i;
    const int page  = bt_row[pos / page_size];
    const size_t dst = kv_row_offset<EB>(page, h, pos % page_size, page_size, hkv) + DIMS * EB * chunk;
    store_chunk<EB>(in, k_cache, v_cache, dst, inv_k, inv_v);
}

// The chunk of thread idx of append_batch_kernel.
template <int EB>
__device__ __forceinline__ void append_batch_chunk(const AppendBatch& a, int idx) {
    constexpr int DIMS = kAppendDims<EB>, CPR = kHeadDim / DIMS;
    const int32_t* tok_begin = a.meta;
    const int32_t* old_len   = a.meta + a.n_ent;
    const int32_t* pl_begin  = a.meta + 2 * a.n_ent;
    const int32_t* pages     = a.meta + 3 * a.n_ent;
    const int chunk = static_cast<unsigned>(idx) % CPR;
    const int th    = static_cast<unsigned>(idx) / CPR;
    const int h     = th % a.hkv;
    const int t     = th / a.hkv;
    const ChunkIn<EB> in = load_chunk<EB>(a.k, a.v, (static_cast<size_t>(t) * a.hkv + h) * kHeadDim + DIMS * chunk);
    // The last entry with tok_begin <= t (zero-count entries share the next
    // one's). Entry t * n_ent / n_tok is tried first (one round of loads): it
    // is the one when every entry holds the same number of tokens (one in a
    // decode step, the prompt length in a uniform prefill); otherwise a
    // binary search.
    const int g  = min(static_cast<int>(static_cast<int64_t>(t) * a.n_ent / a.n_tok), a.n_ent - 1);
    const int tg = tok_begin[g];
    const int tn = g + 1 < a.n_ent ? tok_begin[g + 1] : INT_MAX;
    int lo = g;
    if (tg > t || tn <= t) {
        lo = 0;
        int hi = a.n_ent;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (tok_begin[mid] <= t) lo = mid;
            else hi = mid;
        }
    }
    const int first = old_len[lo];
    const int pos   = first + (t - tok_begin[lo]);
    const int page  = pages[pl_begin[lo] + pos / a.page_size - first / a.page_size];
    const size_t dst = kv_row_offset<EB>(page, h, pos % a.page_size, a.page_size, a.hkv) + DIMS * EB * chunk;
    store_chunk<EB>(in, a.k_cache, a.v_cache, dst, a.inv_k, a.inv_v);
}

// A whole batch of appends in one launch (layout of AppendBatch::meta in
// pa_internal.hpp). Threads cover max(n_tok * hkv * chunks per row, n_tab,
// n_len); each writes its chunk, table entry and length where it has one. A token
// finds its entry by binary search over the entries' first-token offsets, then
// its page in the entry's page list: table entries are read from the staging
// copy, never from the block table this launch is writing.
template <int EB>
__global__ __launch_bounds__(256) void append_batch_kernel(const AppendBatch a) {
    constexpr int CPR = kHeadDim / kAppendDims<EB>;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int32_t* tab       = a.meta + 3 * a.n_ent + a.n_pl;
    const int32_t* lens      = tab + 2 * a.n_tab;
    // A thread's table entry and length are read first and written last, so
    // that every load of the thread is issued before its first store. Both
    // are 8-byte pairs read through buffer resources sized to their arrays:
    // threads past an array read zeros without a branch (a branch around the
    // load would make the thread wait for it where the paths join).
    const u32x2 tabv = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(buffer_rsrc(tab, 8 * a.n_tab), 8 * min(idx, a.n_tab), 0, 0));
    const u32x2 lenv = __builtin_bit_cast(
        u32x2, __builtin_amdgcn_raw_buffer_load_b64(buffer_rsrc(lens, 8 * a.n_len), 8 * min(idx, a.n_len), 0, 0));
    if (idx < a.n_tok * a.hkv * CPR) append_batch_chunk<EB>(a, idx);
    if (idx < a.n_tab) a.table[tabv[0]] = static_cast<int32_t>(tabv[1]);
    if (idx < a.n_len) a.seq_lens[lenv[0]] = static_cast<int32_t>(lenv[1]);
}

// One thread per (token, 8-dim chunk) of one kv head: raw cache bytes out,
// addressed with kv_row_offset, the row function the decode kernel uses.
template <int EB>
__global__ __launch_bounds__(256) void gather_kernel(const void* cache, const int32_t* __restrict__ bt_row,
                                                     int hkv, int page_size, int kv_head, int len, void* out) {
    using Raw = std::conditional_t<EB == 2, u32x4, u32x2>;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= len * 16) return;
    const int chunk = idx & 15;
    const int t     = idx >> 4;
    const int page  = bt_row[t / page_size];
    const size_t off = kv_row_offset<EB>(page, kv_head, t % page_size, page_size, hkv) + 8 * EB * chunk;
    *reinterpret_cast<Raw*>(static_cast<unsigned char*>(out) + static_cast<size_t>(t) * kRowBytes<EB> +
                            8 * EB * chunk) =
        *reinterpret_cast<const Raw*>(static_cast<const unsigned char*>(cache) + off);
}

// Streaming read of n 16-byte words, U independent loads per lane per trip
// (U = 1 is bench_decode.cu:70-78's read_kernel); NT marks the loads
// non-temporal so they bypass cache allocation. Every lane folds its words
// into one value and stores it to *sink only when `publish` is nonzero:
// the launchers pass 0, and since the compiler cannot know that, the loads
// stay.
template <int U, bool NT>
__global__ __launch_bounds__(512) void stream_read_kernel(const u32x4* __restrict__ x, size_t n,
                                                          uint32_t* sink, int publish) {
    uint32_t acc = 0;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (; i + (U - 1) * stride < n; i += U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(x + i + u * stride) : x[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < n; i += stride) {
        const u32x4 v = x[i];
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    if (publish) *sink = acc;
}

// Streaming read where each wave reads its own contiguous `per`-byte span
// (U KiB per trip, 16 B per lane per KiB, non-temporal raw buffer loads):
// the access shape that reaches the highest read rate on this part, since a
// wave's requests stay within few DRAM pages. `per` is a multiple of U KiB.
template <int U>
__global__ __launch_bounds__(512) void stream_read_chunked_kernel(const unsigned char* __restrict__ x, size_t per,
                                                                  uint32_t* sink, int publish) {
    const int    lane = threadIdx.x & 63;
    const size_t wave = (static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(x + wave * per), 0, static_cast<int>(per), 0x00020000);
    uint32_t acc = 0;
    for (size_t off = 0; off < per; off += U * 1024) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 r, static_cast<int>(off) + u * 1024 + 16 * lane, 0, 2));
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (publish) *sink = acc;   // as in stream_read_kernel: never taken, keeps the loads
}

// fp32 -> fp16 (round to nearest even) and fp16 -> fp32 (exact), n elements.
__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                                         size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(in[i]));
}
__global__ __launch_bounds__(256) void f16_to_f32_kernel(const uint16_t* __restrict__ in, float* __restrict__ out,
                                                         size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = static_cast<float>(__builtin_bit_cast(_Float16, in[i]));
}

// Streaming write: every 16-byte word of x gets `word` repeated.
__global__ __launch_bounds__(256) void fill_bytes_kernel(u32x4* __restrict__ x, size_t n, uint32_t word) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        x[i] = u32x4{word, word, word, word};
}

}  // namespace

hipError_t launch_append(int dtype, const uint16_t* k, const uint16_t* v, void* k_cache, void* v_cache,
                         const int32_t* bt_row, int start_pos, int n, int hkv, int page_size, float inv_k,
                         float inv_v, hipStream_t s) {
    check_kv_dtype(dtype);
    if (n <= 0) return hipSuccess;
    const long threads = static_cast<long>(n) * hkv * (kHeadDim / (dtype == PA_KV_FP16 ? kAppendDims<2> : kAppendDims<1>));
    const int blocks   = static_cast<int>((threads + 255) / 256);
    if (dtype == PA_KV_FP16)
        hipLaunchKernelGGL(append_kernel<2>, dim3(blocks), dim3(256), 0, s, k, v, k_cache, v_cache, bt_row,
                           start_pos, n, hkv, page_size, inv_k, inv_v);
    else
        hipLaunchKernelGGL(append_kernel<1>, dim3(blocks), dim3(256), 0, s, k, v, k_cache, v_cache, bt_row,
                           start_pos, n, hkv, page_size, inv_k, inv_v);
    return hipGetLastError();
}

hipError_t launch_append_batch(int dtype, const AppendBatch& a, hipStream_t s) {
    check_kv_dtype(dtype);
    const int  cpr     = kHeadDim / (dtype == PA_KV_FP16 ? kAppendDims<2> : kAppendDims<1>);
    const long threads = std::max<long>(static_cast<long>(a.n_tok) * a.hkv * cpr, std::max(a.n_tab, a.n_len));
    if (threads <= 0) return hipSuccess;
    const int blocks = static_cast<int>((threads + 255) / 256);
    if (dtype == PA_KV_FP16)
        hipLaunchKernelGGL(append_batch_kernel<2>, dim3(blocks), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(append_batch_kernel<1>, dim3(blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gather(int dtype, const void* cache, const int32_t* bt_row, int hkv, int page_size,
                         int kv_head, int len, void* out, hipStream_t s) {
    check_kv_dtype(dtype);
    if (len <= 0) return hipSuccess;
    const int blocks = (len * 16 + 255) / 256;
    if (dtype == PA_KV_FP16)
        hipLaunchKernelGGL(gather_kernel<2>, dim3(blocks), dim3(256), 0, s, cache, bt_row, hkv, page_size, kv_head,
                           len, out);
    else
        hipLaunchKernelGGL(gather_kernel<1>, dim3(blocks), dim3(256), 0, s, cache, bt_row, hkv, page_size, kv_head,
                           len, out);
    return hipGetLastError();
}

hipError_t launch_convert(const void* in, void* out, size_t n, bool to_half, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const size_t want = (n + 255) / 256;
    const int blocks = static_cast<int>(want < 4096 ? want : 4096);
    if (to_half)
        hipLaunchKernelGGL(f32_to_f16_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const float*>(in),
                           static_cast<uint16_t*>(out), n);
    else
        hipLaunchKernelGGL(f16_to_f32_kernel, dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(in),
                           static_cast<float*>(out), n);
    return hipGetLastError();
}

hipError_t launch_fill_bytes(void* buf, size_t bytes, int value, hipStream_t s) {
    const size_t n = bytes / 16;
    if (n == 0) return hipSuccess;
    const uint32_t b = static_cast<uint32_t>(value) & 0xffu;
    const size_t want = (n + 255) / 256;
    const int blocks = static_cast<int>(want < 16384 ? want : 16384);
    hipLaunchKernelGGL(fill_bytes_kernel, dim3(blocks), dim3(256), 0, s, static_cast<u32x4*>(buf), n,
                       b | (b << 8) | (b << 16) | (b << 24));
    return hipGetLastError();
}

hipError_t launch_stream_read_chunked(const void* buf, size_t bytes, int blocks, int threads, int unroll,
                                     uint32_t* sink, hipStream_t s) {
    if (threads != 256 && threads != 512) throw std::invalid_argument("stream_read_chunked: threads must be 256 or 512");
    if (unroll != 8 && unroll != 16) throw std::invalid_argument("stream_read_chunked: unroll must be 8 or 16");
    const size_t waves = static_cast<size_t>(blocks) * (threads / 64);
    const size_t trip  = static_cast<size_t>(unroll) * 1024;
    if (blocks <= 0 || bytes % (waves * trip) != 0 || bytes / waves > static_cast<size_t>(INT32_MAX))
        throw std::invalid_argument("stream_read_chunked: bytes must split into equal spans of whole trips per wave");
    const auto*  x   = static_cast<const unsigned char*>(buf);
    const size_t per = bytes / waves;
    if (unroll == 8)
        hipLaunchKernelGGL(stream_read_chunked_kernel<8>, dim3(blocks), dim3(threads), 0, s, x, per, sink, 0);
    else
        hipLaunchKernelGGL(stream_read_chunked_kernel<16>, dim3(blocks), dim3(threads), 0, s, x, per, sink, 0);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* buf, size_t bytes, int blocks, int threads, int unroll, bool nt,
                              uint32_t* sink, hipStream_t s) {
    if (threads != 256 && threads != 512) throw std::invalid_argument("stream_read: threads must be 256 or 512");
    const auto* x = static_cast<const u32x4*>(buf);
    const size_t n = bytes / 16;
#define PA_READ(U, NT) hipLaunchKernelGGL((stream_read_kernel<U, NT>), dim3(blocks), dim3(threads), 0, s, x, n, sink, 0)
    switch (unroll * 2 + (nt ? 1 : 0)) {
        case 2: PA_READ(1, false); break;
        case 3: PA_READ(1, true); break;
        case 4: PA_READ(2, false); break;
        case 5: PA_READ(2, true); break;
        case 8: PA_READ(4, false); break;
        case 9: PA_READ(4, true); break;
        case 16: PA_READ(8, false); break;
        case 17: PA_READ(8, true); break;
        default: throw std::invalid_argument("stream_read: unroll must be 1, 2, 4 or 8");
    }
#undef PA_READ
    return hipGetLastError();
}

}  // namespace pa
