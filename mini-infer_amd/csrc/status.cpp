// status.cpp -- status strings and ABI version of libmi_kernels.so.
#include <hip/hip_runtime.h>

#include <atomic>

#include "mi_kernels.h"

extern "C" const char* mi_status_string(int status) {
    switch (status) {
        case MI_OK: return "ok";
        case MI_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer or bad size)";
        case MI_ERR_UNSUPPORTED: return "shape not supported by the kernels";
        case MI_ERR_ALIASING: return "buffers overlap where they must not";
        default: break;
    }
    if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
    return "unknown status";
}

extern "C" int mi_abi_version(void) { return MI_KERNELS_ABI_VERSION; }

// The one-launch kernels' exchange mode (row_exchange.h), read at each
// launch; only the test hook below changes it.
namespace mi {
std::atomic<int>& exchange_test_mode() {
    static std::atomic<int> mode{0};
    return mode;
}
}  // namespace mi

extern "C" int mi_exchange_test_mode(int mode) {
    if (mode != 0 && mode != 1) return MI_ERR_INVALID_ARGUMENT;
    return mi::exchange_test_mode().exchange(mode);
}
