// Thread-local last-error state and introspection of the C ABI.
#include <cstring>
#include <string>

#include "mlk_common.h"

namespace mlk {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }

void clear_error() { g_last_error.clear(); }

mlk_status launch_status(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error(std::string(what) + ": " + hipGetErrorString(err));
        return MLK_ERR_RUNTIME;
    }
    return MLK_OK;
}

// A kernel that does nothing: graph nodes of it with a kernel's launch shape
// time the floor that launch pays before any of its work.
__global__ void empty_kernel() {}

}  // namespace mlk

extern "C" {

mlk_status mlk_empty_kernel(int64_t blocks, int64_t threads, size_t dynamic_lds_bytes, mlk_stream_t stream) {
    MLK_CHECK(blocks > 0 && blocks <= (int64_t{1} << 31) - 1, "blocks must be in [1, 2^31)");
    MLK_CHECK(threads > 0 && threads <= 1024, "threads must be in [1, 1024]");
    MLK_CHECK(dynamic_lds_bytes <= 160 * 1024, "dynamic LDS must be at most 160 KiB");
    hipLaunchKernelGGL(mlk::empty_kernel, dim3(static_cast<unsigned>(blocks)), dim3(static_cast<unsigned>(threads)),
                       dynamic_lds_bytes, reinterpret_cast<hipStream_t>(stream));
    return mlk::launch_status("empty_kernel");
}

const char* mlk_last_error(void) { return mlk::g_last_error.c_str(); }

int mlk_abi_version(void) { return 1; }

mlk_status mlk_build_info(char* buffer, size_t capacity) {
    MLK_CHECK(buffer != nullptr && capacity > 0, "buffer must be non-empty");
    int device = 0;
    hipDeviceProp_t prop{};
    std::string arch = "unknown";
    int cus = 0;
    if (hipGetDevice(&device) == hipSuccess && hipGetDeviceProperties(&prop, device) == hipSuccess) {
        arch = prop.gcnArchName;
        cus = prop.multiProcessorCount;
    }
    const std::string json = std::string("{\"variant\": \"gfx950\", \"compiled_arch\": \"gfx950\", \"device_arch\": \"") +
                             arch + "\", \"compute_units\": " + std::to_string(cus) +
                             ", \"wavefront\": 64, \"abi\": 1, \"hip_version\": " + std::to_string(HIP_VERSION) + "}";
    std::strncpy(buffer, json.c_str(), capacity - 1);
    buffer[capacity - 1] = '\0';
    return MLK_OK;
}

}  // extern "C"
