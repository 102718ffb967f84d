// Shared helpers of the MI355X (gfx950) RDT4quant kernels: the status /
// last-error convention of the C ABI and small device utilities.
//
// Status convention (mirrors montlok_status + a thread-local last error,
// include/montlok/montlok.h:16-17,43-52 of the reference): every entry point
// returns an mlk_status; on failure mlk_last_error() names the argument or
// the HIP call that failed, with the same wording as the reference's
// TORCH_CHECK messages where one exists.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/mlk_hip.h"

namespace mlk {

void set_error(const std::string& message);
void clear_error();

// Validation helper: `MLK_CHECK(cond, "message")` returns MLK_ERR_INVALID_ARGUMENT.
#define MLK_CHECK(cond, msg)                                   \
    do {                                                       \
        if (!(cond)) {                                         \
            ::mlk::set_error(msg);                             \
            return MLK_ERR_INVALID_ARGUMENT;                   \
        }                                                      \
    } while (0)

// Kernel launch epilogue: turns a launch error into MLK_ERR_RUNTIME.
mlk_status launch_status(const char* what);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Device utilities
// ---------------------------------------------------------------------------

constexpr int kWave = 64;

__device__ __forceinline__ double shfl_xor_d(double v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ __forceinline__ double shfl_d(double v, int src) { return __shfl(v, src, kWave); }

// Sum over aligned groups of `width` lanes (width a power of two <= 64);
// every lane of a group receives the group total.
template <int width>
__device__ __forceinline__ double group_sum_d(double v) {
#pragma unroll
    for (int mask = width / 2; mask > 0; mask >>= 1) {
        v += shfl_xor_d(v, mask);
    }
    return v;
}

}  // namespace mlk
