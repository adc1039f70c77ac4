#pragma once
// RAII contiguous fp32 K/V store on the device (include/kv_store.hpp:6-27)
// with HIP allocations; accessor() hands out the device pointers.

#include "hip_check.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>

// Device pointers to a contiguous [T][d] fp32 K and V (include/kv_layout.hpp:4-6).
struct ContiguousKV {
    const float* K;
    const float* V;
};

struct ContiguousKVStore {
    float* d_K;
    float* d_V;

    ContiguousKVStore(const float* h_K, const float* h_V, int T, int d) {
        const size_t bytes = sizeof(float) * static_cast<size_t>(T) * static_cast<size_t>(d);
        HIP_CHECK(hipMalloc(&d_K, bytes));
        HIP_CHECK(hipMalloc(&d_V, bytes));
        HIP_CHECK(hipMemcpy(d_K, h_K, bytes, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(d_V, h_V, bytes, hipMemcpyHostToDevice));
    }

    ~ContiguousKVStore() {
        (void)hipFree(d_K);
        (void)hipFree(d_V);
    }

    ContiguousKVStore(const ContiguousKVStore&)            = delete;
    ContiguousKVStore& operator=(const ContiguousKVStore&) = delete;

    ContiguousKV accessor() const { return {d_K, d_V}; }
};
