// Device-side helpers shared by the gfx950 kernels (pa_decode.hip, pa_cache.hip).
#pragma once

#include "pa_internal.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pa {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float    f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Bytes of one token's head_dim row in an HND pool of element width EB.
template <int EB>
constexpr int kRowBytes = kHeadDim * EB;

// Byte offset of (page, kv head, slot in page) in an HND pool
// ([page][kv_head][slot][dim], decode_kernels.cuh:175-177 / paged_kv_cache.cu:34).
template <int EB>
__device__ __forceinline__ size_t kv_row_offset(int page, int h, int slot, int page_size, int hkv) {
    return ((static_cast<size_t>(page) * hkv + h) * page_size + slot) * static_cast<size_t>(kRowBytes<EB>);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// dword 3 of a raw buffer resource (32-bit data format, no swizzle).
constexpr int kBufferFlags = 0x00020000;

// Raw buffer resource over [base, base + bytes): loads past the end read
// zeros and touch no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferFlags);
}

// Orders LDS accesses that lanes of one wave use to trade data: every access
// before the call (e.g. one lane's ds_write) happens before every access after
// it (another lane's ds_read of the same bytes). LDS runs a wave's operations
// in issue order, so on gfx950 this emits no instruction; the wavefront-scope
// fences and the wave barrier keep the compiler from moving LDS accesses
// across the call.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Two FP8 E4M3 bytes (byte pair HI of w) -> two fp16, exactly (every E4M3
// value is an fp16 value; scale 1.0).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_f16x2(uint32_t w) {
    const f16x2 h = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI);
    return __builtin_bit_cast(uint32_t, h);
}

// Eight FP8 bytes -> eight fp16.
__device__ __forceinline__ f16x8 fp8x8_to_f16x8(uint32_t lo, uint32_t hi) {
    u32x4 r;
    r[0] = fp8x2_to_f16x2<false>(lo);
    r[1] = fp8x2_to_f16x2<true>(lo);
    r[2] = fp8x2_to_f16x2<false>(hi);
    r[3] = fp8x2_to_f16x2<true>(hi);
    return __builtin_bit_cast(f16x8, r);
}

// 16-byte / 8-byte global loads, optionally non-temporal (streamed data that
// is read once should not displace reusable lines).
template <bool NT>
__device__ __forceinline__ u32x4 load16(const void* p) {
    if constexpr (NT) return __builtin_nontemporal_load(static_cast<const u32x4*>(p));
    else return *static_cast<const u32x4*>(p);
}
template <bool NT>
__device__ __forceinline__ u32x2 load8(const void* p) {
    if constexpr (NT) return __builtin_nontemporal_load(static_cast<const u32x2*>(p));
    else return *static_cast<const u32x2*>(p);
}

}  // namespace pa
