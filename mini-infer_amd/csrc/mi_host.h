// mi_host.h -- host-side helpers for the C-ABI entry points: argument
// checks, alignment and overlap tests, launch-status mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>
#include <map>
#include <mutex>
#include <utility>

#include "mi_kernels.h"

namespace mi {

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// True when [a, a+abytes) and [b, b+bbytes) share at least one byte.
inline bool overlaps(const void* a, int64_t abytes, const void* b, int64_t bbytes) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + static_cast<uintptr_t>(bbytes) && b0 < a0 + static_cast<uintptr_t>(abytes);
}

// True when every factor is non-negative and their product stays within
// 2^62 (byte counts formed from it, and sums of two such, cannot overflow
// int64).  Entry points check their size products with it before forming
// them and return MI_ERR_INVALID_ARGUMENT otherwise: no real buffer is that
// large.
inline bool product_fits(std::initializer_list<int64_t> factors) {
    int64_t p = 1;
    for (int64_t f : factors) {
        if (f < 0 || __builtin_mul_overflow(p, f, &p) || p > (int64_t{1} << 62)) return false;
    }
    return true;
}

// Maps the outcome of the launches just issued to the ABI's status code.
inline int launch_status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MI_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int64_t kMaxGridX = 2147483647;  // HIP grid.x limit (2^31 - 1)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroups of `kernel` (launched with `threads` lanes) the current device
// holds at once: occupancy per CU x CU count, queried once per
// (kernel, device) and cached.  0 if the runtime cannot say.
inline int64_t resident_workgroups(const void* kernel, int threads) {
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, int64_t> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(kernel, dev * 4096 + threads);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    int64_t cap = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
        cap = static_cast<int64_t>(per_cu) * cus;
    cache[key] = cap;
    return cap;
}

// Compute units of the current device, queried once per device (0 if the
// runtime cannot say).
inline int device_cus() {
    static std::mutex mu;
    static std::map<int, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 0;
    cache[dev] = cus;
    return cus;
}

// A zeroed device region of `bytes` that the library holds for the current
// device's legacy default stream (stream 0), one per `tag`: allocated and
// zeroed on stream 0 at its first use, never freed.  Calls on stream 0 run in
// order, so a region that each call leaves valid for the next (the one-launch
// softmax / argmax row records) can be shared by all of them.  Other streams
// get nullptr -- a stream handle can be reused by a new stream while work of
// the old one is pending, and hipStreamPerThread names a different stream in
// every thread -- as do runtime errors (the error is cleared, so it is not
// reported by a later launch).  The caller then takes a path that needs no
// such region.
inline void* default_stream_region(int tag, int64_t bytes, hipStream_t s) {
    if (s != nullptr || bytes <= 0) return nullptr;
    static std::mutex mu;
    static std::map<std::pair<int, int>, void*> regions;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(dev, tag);
    auto it = regions.find(key);
    if (it != regions.end()) return it->second;
    void* p = nullptr;
    if (hipMalloc(&p, static_cast<size_t>(bytes)) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (hipMemsetAsync(p, 0, static_cast<size_t>(bytes), nullptr) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(p);
        return nullptr;
    }
    regions[key] = p;
    return p;
}
enum RegionTag { kRegionSoftmax = 1, kRegionArgmax = 2 };

// How full the GPU's last round of workgroups is when `groups` workgroups
// run `cap` at a time: groups / (rounds * cap), 1.0 = no idle tail.
inline double round_fill(int64_t groups, int64_t cap) {
    if (cap <= 0 || groups <= 0) return 0.0;
    const int64_t rounds = (groups + cap - 1) / cap;
    return static_cast<double>(groups) / static_cast<double>(rounds * cap);
}

}  // namespace mi
