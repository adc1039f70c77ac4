#pragma once
// HIP_CHECK (the reference's CUDA_CHECK, include/cuda_check.hpp:9-17) and the
// C-ABI status -> C++ error mapping used by the header-only wrappers.

#include "pa_decode.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <stdexcept>

// Evaluate expr exactly once and abort on failure (not assert(): release
// builds define NDEBUG).
#define HIP_CHECK(expr)                                                                        \
    do {                                                                                       \
        hipError_t _hip_err = (expr);                                                          \
        if (_hip_err != hipSuccess) {                                                          \
            std::fprintf(stderr, "HIP error %s at %s:%d: %s\n", hipGetErrorName(_hip_err),     \
                         __FILE__, __LINE__, hipGetErrorString(_hip_err));                     \
            std::abort();                                                                      \
        }                                                                                      \
    } while (0)

namespace decode::detail {

// PA_ERR_INVALID_ARGUMENT -> std::invalid_argument, PA_ERR_LENGTH ->
// std::length_error (the reference's exception types); a device error aborts,
// as CUDA_CHECK does in the reference.
inline void check(pa_status s) {
    switch (s) {
        case PA_OK: return;
        case PA_ERR_INVALID_ARGUMENT: throw std::invalid_argument(pa_last_error());
        case PA_ERR_LENGTH: throw std::length_error(pa_last_error());
        default:
            std::fprintf(stderr, "paged decode device error: %s\n", pa_last_error());
            std::abort();
    }
}

}  // namespace decode::detail
