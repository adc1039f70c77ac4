// Allocation-free decode entry point (pa_decode_static): pa_decode with the
// partial workspace (the normalized fp32 partial rows and base-2 LSEs of rows
// split across blocks, which the merge kernel combines) in a fixed device
// array of this library instead of the caller's pa_decode_params workspace.
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc). It launches
// the same split and merge kernels as pa_decode.
//
// The array: PA_SCRATCH_BYTES (32 MiB) per device, held by every GPU the
// library runs on until the process ends. Its device address is looked up
// once per device (hipGetSymbolAddress, on the entry point's first call with
// that device current) and only that address reaches the kernels. Every call
// on one GPU shares that GPU's array: calls that overlap on one GPU (two
// streams, two host threads) race on it. Nothing in it needs to start at
// zero: the split kernel writes every partial the merge kernel reads.

#include "pa_host.hpp"

#include <hip/hip_runtime.h>

#include <array>
#include <cstddef>
#include <mutex>
#include <string>

#ifndef PA_SCRATCH_BYTES
#define PA_SCRATCH_BYTES (32u << 20)
#endif

namespace {

constexpr size_t kScratchBytes = PA_SCRATCH_BYTES;
constexpr int    kMaxDevices   = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex                          g_scratch_mu;
std::array<void*, kMaxDevices>      g_scratch_ptr{};   // per device: the array's device address

// The device address of `scratch` on the current device (looked up once).
void* scratch_on_current_device() {
    int dev = 0;
    pa::hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw std::invalid_argument("decode_static: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    void*& ptr = g_scratch_ptr[static_cast<size_t>(dev)];
    if (!ptr) {
        void* addr = nullptr;
        pa::hip_check(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!addr) throw pa::DeviceError("hipGetSymbolAddress(scratch) returned a null address");
        ptr = addr;
    }
    return ptr;
}

}  // namespace

using namespace pa::host;

extern "C" {

pa_status pa_decode_static(int dtype, const pa_decode_params* p, int num_segments, void* stream) {
    return guarded([&] {
        if (!p) throw std::invalid_argument("params is null");
        check_dtype(dtype);
        if (p->num_kv_heads <= 0 || p->num_q_heads <= 0 || p->num_q_heads % p->num_kv_heads != 0)
            throw std::invalid_argument("num_q_heads must be a multiple of num_kv_heads");
        if (p->head_dim != pa::kHeadDim) throw std::invalid_argument("unsupported head_dim " + std::to_string(p->head_dim));
        // The kernels write one partial per split segment of the bound plan,
        // which only the caller knows here; reject counts no plan can have
        // (every (row, kv head) holds at least one segment, no row more than
        // the plan's most).
        const long items = static_cast<long>(p->batch) * p->num_kv_heads;
        if (num_segments < 0 || (p->num_ctas > 0 && (num_segments < items || num_segments < p->max_item_segments)))
            throw std::invalid_argument("decode_static: num_segments must be the plan's segment count");
        const size_t group = static_cast<size_t>(p->num_q_heads / p->num_kv_heads);
        const size_t rows  = static_cast<size_t>(num_segments) * group;
        // Plans merged inside the split kernel keep their partials in LDS; every
        // other plan with split rows writes rows * (head_dim + 1) floats.
        const size_t need = p->block_merge ? 0 : rows * (static_cast<size_t>(pa::kHeadDim) + 1) * sizeof(float);
        if (need > kScratchBytes)
            throw std::length_error("decode_static: the plan's partial workspace (" + std::to_string(need) +
                                    " bytes) exceeds the static scratch (" + std::to_string(kScratchBytes) +
                                    " bytes)");
        pa_decode_params q = *p;
        float* base = static_cast<float*>(scratch_on_current_device());
        q.partial_out = base;
        q.partial_lse = need ? base + rows * pa::kHeadDim : base;   // unused by merged plans
        decode_impl(dtype, q, as_stream(stream), true, true);
    });
}

}  // extern "C"
