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

}  // namespace mlk

extern "C" {

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
