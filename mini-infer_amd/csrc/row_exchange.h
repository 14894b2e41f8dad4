// row_exchange.h -- placement and record traffic of the one-launch kernels
// (split-row softmax, greedy argmax, fused softmax + argmax), whose chunk
// workgroups exchange per-row partial results through tagged 64-bit record
// words in a caller workspace.
//
// Placement.  The command processor hands the workgroups of a launch to the
// XCDs (each with its own L2) round robin by linear workgroup index: index i
// runs on XCD i mod 8 (measured on MI355X: the hardware XCC id of workgroup
// i equals that of workgroup i mod 8 for every i of a 4096-workgroup grid).
// The one-launch grids are 1-D and order their workgroups so that every chunk
// of a row slot has the same index modulo kXcds (chunk_of below): a row's
// chunks share one XCD and one L2.
//
// Records.  Each chunk publishes its words twice:
//   * into the row's L2 set, with plain (work-group scope) stores, which land
//     in the XCD's L2 through the write-through L1;
//   * into the row's mirror set, with device-scope write-through stores.
// Pollers first read the L2 set with L1-missing non-temporal loads served by
// the L2 (local_load): with the row on one XCD that is an L2 round trip, not
// a trip to the memory side.  If the L2 set does not show every chunk within
// kLocalPollTicks (the placement above did not hold, or a row-mate started
// late), they read the mirror at device scope, which is correct for any
// placement.  Tags make stale words harmless either way, and the callers'
// own bounds and fallbacks still apply.
//
// Measured at [64, 152064] / [32, 152064] (graph replay): softmax 9.8 -> 9.7
// / 7.5 -> 7.1 us, fused softmax + argmax 12.1 -> 11.1 / 11.9 -> 8.4 us
// against device-scope exchange.  (Device-scope polls with the row on one
// XCD were slower than spread rows, 11.4 us: every poll of a row misses in
// the same L2 channel.)
#pragma once

#include <atomic>

#include "mi_device.h"

namespace mi {

constexpr int kXcds = 8;

// Words of one record set start on their own 128-byte line, apart from the
// epoch header that device-scope atomics update.
constexpr int64_t kRecordHeaderBytes = 128;

// Wall-clock bound of the L2 phase of a poll: 2000 ticks of the 100 MHz
// constant clock (20 us), several times a normal exchange.
constexpr uint64_t kLocalPollTicks = 2000;

// Wall-clock bound of a row's whole poll, both phases: 5000 ticks (50 us),
// some 10 times a normal exchange.  A poll that runs out costs only time
// (its row is computed from x), so the bound is what a call pays when a
// row-mate cannot run -- the grid not resident because other work holds
// CUs.
constexpr uint64_t kPollTicks = 5000;

// Chunk `split` and row slot `slot` of workgroup L in a 1-D grid of
// splits * R workgroups (R a multiple of kXcds): rows in groups of kXcds,
// chunk c of slot g * kXcds + q at index g * kXcds * splits + c * kXcds + q.
__device__ __forceinline__ void chunk_of(int L, int splits, int& split, int& slot) {
    const int per_group = kXcds * splits;
    const int grp = L / per_group;
    const int j = L - grp * per_group;
    split = j / kXcds;
    slot = grp * kXcds + (j - split * kXcds);
}

// Publish stores: into the XCD's L2, and through to memory.
__device__ __forceinline__ void local_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void device_store(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll loads of one record slot of SW 64-bit words (2 or 4; 16-byte
// aligned) at `byte_off` from a workgroup-uniform `base`: an SGPR base and a
// 32-bit lane offset, 16-byte loads, one wait for all of them.  Each 64-bit
// word was written whole by one store, and an aligned 16-byte load reads it
// whole.  LOCAL: "sc0 nt", which misses the CU's L1 and is served by the
// XCD's L2 (a work-group scope atomic load, "sc0", hits a stale L1 line and
// never sees a row-mate's store: measured, every poll ran to its bound);
// else "sc1", the device-scope load that a relaxed agent-scope atomic load
// is.  The wait also covers any other outstanding vector memory operation
// of the wave.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#define MI_POLL_LD(BITS) "global_load_dwordx4 %0, %2, %3 " BITS "\n\t"
#define MI_POLL_LD16(BITS) "global_load_dwordx4 %1, %2, %3 offset:16 " BITS "\n\t"
template <bool LOCAL, int SW>
__device__ __forceinline__ void load_slot(const uint64_t* base, uint32_t byte_off,
                                          uint64_t (&w)[SW]) {
    static_assert(SW == 2 || SW == 4, "a slot is 2 or 4 words");
    u32x4 a, b;
    if constexpr (SW == 2) {
        if constexpr (LOCAL)
            asm volatile(MI_POLL_LD("sc0 nt") "s_waitcnt vmcnt(0)"
                         : "=&v"(a), "=v"(b) : "v"(byte_off), "s"(base) : "memory");
        else
            asm volatile(MI_POLL_LD("sc1") "s_waitcnt vmcnt(0)"
                         : "=&v"(a), "=v"(b) : "v"(byte_off), "s"(base) : "memory");
    } else {
        if constexpr (LOCAL)
            asm volatile(MI_POLL_LD("sc0 nt") MI_POLL_LD16("sc0 nt") "s_waitcnt vmcnt(0)"
                         : "=&v"(a), "=&v"(b) : "v"(byte_off), "s"(base) : "memory");
        else
            asm volatile(MI_POLL_LD("sc1") MI_POLL_LD16("sc1") "s_waitcnt vmcnt(0)"
                         : "=&v"(a), "=&v"(b) : "v"(byte_off), "s"(base) : "memory");
    }
    w[0] = (static_cast<uint64_t>(a.y) << 32) | a.x;
    w[1] = (static_cast<uint64_t>(a.w) << 32) | a.z;
    if constexpr (SW == 4) {
        w[2] = (static_cast<uint64_t>(b.y) << 32) | b.x;
        w[3] = (static_cast<uint64_t>(b.w) << 32) | b.z;
    }
}
#undef MI_POLL_LD
#undef MI_POLL_LD16

// Test hook (mi_exchange_test_mode): 0 = L2 set first, then the mirror;
// 1 = the mirror only (device scope from the first poll).
std::atomic<int>& exchange_test_mode();

}  // namespace mi
