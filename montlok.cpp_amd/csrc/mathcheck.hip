// Diagnostic entry point: evaluates the device math helpers of the kernels
// (exp, tanh, sigmoid in double) on caller data so tests can bound their
// error against a correctly rounded host library. The reference tests its own
// polynomial exp the same way (rdt4quant_cpu/montlok_selftest.cpp:770-790).
#include "mlk_common.h"

namespace mlk {
namespace {

__global__ void math_check_kernel(const double* __restrict__ x, int64_t count, double* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const double v = x[i];
    out[i] = exp_d(v);
    out[count + i] = tanh_d(v);
    out[2 * count + i] = sigmoid_fast(v);
    out[3 * count + i] = recip_pos(v);
}

}  // namespace
}  // namespace mlk

extern "C" mlk_status mlk_math_check(const double* x, int64_t count, double* out, mlk_stream_t stream) {
    MLK_CHECK(count >= 0, "count must be non-negative");
    MLK_CHECK(count == 0 || (x != nullptr && out != nullptr), "null tensor pointer");
    if (count == 0) return MLK_OK;
    hipLaunchKernelGGL(mlk::math_check_kernel, dim3(mlk::ceil_div(count, 256)), dim3(256), 0, stream, x, count, out);
    return mlk::launch_status("math_check");
}
