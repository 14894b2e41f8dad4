// mi_host.h -- host-side helpers for the C-ABI entry points: argument
// checks, alignment and overlap tests, launch-status mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mi_kernels.h"

namespace mi {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// True when [a, a+abytes) and [b, b+bbytes) share at least one byte.
inline bool overlaps(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + static_cast<uintptr_t>(bbytes) && b0 < a0 + static_cast<uintptr_t>(abytes);
}

// Maps the outcome of the launches just issued to the ABI's status code.
inline int launch_status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MI_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int64_t kMaxGridX = 2147483647;  // HIP grid.x limit (2^31 - 1)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace mi
