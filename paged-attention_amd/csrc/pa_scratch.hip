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
// once per device (hipGetSymbolAddress) at set-up: by every plan upload on
// that device (scratch_prepare), else by the entry point's first call there,
// which refuses to do it while its stream is being captured. Only that
// address reaches the kernels. The workspace is sized from the bound plan's
// own segment count (pa_decode_params.num_segments, set by
// pa_device_plan_bind); a count from the caller that disagrees is refused
// before anything is launched. Every call on one GPU shares that GPU's array:
// calls that overlap on one GPU (two streams, two host threads) race on it.
// Nothing in it needs to start at zero: the split kernel writes every partial
// that is read back (the merge counters of block_merge 2 live in the plan).

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

// The device address of `scratch` on the current device, looked up once per
// device. `lookup` = false only reports it (null when not looked up yet).
void* scratch_on_current_device(bool lookup) {
    int dev = 0;
    pa::hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw std::invalid_argument("decode_static: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    void*& ptr = g_scratch_ptr[static_cast<size_t>(dev)];
    if (!ptr && lookup) {
        void* addr = nullptr;
        pa::hip_check(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!addr) throw pa::DeviceError("hipGetSymbolAddress(scratch) returned a null address");
        ptr = addr;
    }
    return ptr;
}

}  // namespace

using namespace pa::host;

namespace pa::host {
void scratch_prepare() { (void)scratch_on_current_device(true); }
}  // namespace pa::host

extern "C" {

pa_status pa_decode_static(int dtype, const pa_decode_params* p, int num_segments, void* stream) {
    return guarded([&] {
        if (!p) throw std::invalid_argument("params is null");
        check_dtype(dtype);
        if (p->num_kv_heads <= 0 || p->num_q_heads <= 0 || p->num_q_heads % p->num_kv_heads != 0)
            throw std::invalid_argument("num_q_heads must be a multiple of num_kv_heads");
        if (p->head_dim != pa::kHeadDim) throw std::invalid_argument("unsupported head_dim " + std::to_string(p->head_dim));
        // The kernels write one partial per split segment of the bound plan:
        // the workspace is sized from the count the plan's bind recorded, and a
        // caller's count must agree with it.
        if (p->num_ctas > 0 && p->num_segments <= 0)
            throw std::invalid_argument("decode_static: params are not bound to a device plan (num_segments unset)");
        if (num_segments != p->num_segments)
            throw std::invalid_argument("decode_static: num_segments (" + std::to_string(num_segments) +
                                        ") differs from the bound plan's (" + std::to_string(p->num_segments) + ")");
        const long items      = static_cast<long>(p->batch) * p->num_kv_heads;
        const bool split_rows = p->num_segments > items;
        if (split_rows && !p->block_merge && !p->needs_merge)
            throw std::invalid_argument("decode_static: a plan with split rows needs needs_merge or block_merge");
        const size_t group = static_cast<size_t>(p->num_q_heads / p->num_kv_heads);
        const size_t rows  = static_cast<size_t>(p->num_segments) * group;
        // Plans merged by the merge kernel, or across blocks inside the split
        // kernel (block_merge 2), write partials to the workspace, at most
        // rows * (head_dim + 1) floats; plans merged inside one block keep
        // theirs in LDS, and plans without split rows write none.
        const bool   hbm_partials = split_rows && p->block_merge != 1;
        const size_t need = hbm_partials ? rows * (static_cast<size_t>(pa::kHeadDim) + 1) * sizeof(float) : 0;
        if (need > kScratchBytes)
            throw std::length_error("decode_static: the plan's partial workspace (" + std::to_string(need) +
                                    " bytes) exceeds the static scratch (" + std::to_string(kScratchBytes) +
                                    " bytes)");
        void* addr = scratch_on_current_device(false);
        if (!addr) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            pa::hip_check(hipStreamIsCapturing(as_stream(stream), &cs), "hipStreamIsCapturing");
            if (cs != hipStreamCaptureStatusNone)
                throw std::invalid_argument(
                    "decode_static: the static scratch of this device is not set up; upload a plan on the device "
                    "(pa_device_plan_upload, pa_cache_plan) outside graph capture first");
            addr = scratch_on_current_device(true);
        }
        pa_decode_params q = *p;
        float* base   = static_cast<float*>(addr);
        q.partial_out = base;
        q.partial_lse = need ? base + rows * pa::kHeadDim : base;   // unused without HBM partials
        decode_impl(dtype, q, as_stream(stream), true, true);
    });
}

}  // extern "C"
