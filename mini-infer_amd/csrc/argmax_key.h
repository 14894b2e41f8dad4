// argmax_key.h -- the 64-bit order keys of greedy argmax and their wave
// reduction, shared by the argmax kernels (kv_argmax.hip) and the fused
// softmax + argmax pass (softmax.hip).
//
// The reference lets each of 256 threads keep its first strict maximum over
// a stride-256 slice, then tree-reduces pairs (t, t + offset) for offset =
// 128 .. 1, keeping the lower slot on ties (src/kernels/sampling_kernel.cu:
// 14-38): among tied elements the one whose index i has the smallest 8-bit
// bit reversal of i mod 256 wins, then the smallest i.  One key per element
// encodes that order --
//   [ordered fp16 value : 16 | 255 - bitrev8(i mod 256) : 16 | ~i : 32]
// -- larger is better, 0 = never chosen (NaN, -inf), so any reduction order
// gives the reference's answer.
#pragma once

#include "mi_device.h"

namespace mi {

// Order key of element i with fp16 bits h (see the file header); 0 when the
// element can never be chosen (NaN or -inf).
__device__ __forceinline__ uint64_t argmax_key(uint16_t h, int64_t i) {
    if ((h & 0x7fffu) > 0x7c00u || h == 0xfc00u) return 0;  // NaN, -inf
    if (h == 0x8000u) h = 0;                                 // -0 == +0
    const uint32_t ord = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
    const uint32_t tie = 255u - (__builtin_bitreverse32(static_cast<uint32_t>(i & 255)) >> 24);
    return (static_cast<uint64_t>(ord) << 48) | (static_cast<uint64_t>(tie) << 32) |
           static_cast<uint64_t>(~static_cast<uint32_t>(i));
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// The largest 64-bit key of the wave, in every lane: DPP within 16-lane
// rows (both halves of the key move together), then the permlane swaps
// across rows (no LDS).  Every lane must be active.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xF, 0xF, false);
    const uint32_t hi = __builtin_amdgcn_mov_dpp(static_cast<int>(v >> 32), CTRL, 0xF, 0xF, false);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
template <int STRIDE>
__device__ __forceinline__ uint64_t max_xor_u64(uint64_t v) {
    uint32_t la, lb, ha, hb;
    if constexpr (STRIDE == 16) {
        pair_xor16(static_cast<uint32_t>(v), la, lb);
        pair_xor16(static_cast<uint32_t>(v >> 32), ha, hb);
    } else {
        pair_xor32(static_cast<uint32_t>(v), la, lb);
        pair_xor32(static_cast<uint32_t>(v >> 32), ha, hb);
    }
    return max_u64((static_cast<uint64_t>(ha) << 32) | la, (static_cast<uint64_t>(hb) << 32) | lb);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_u64(v, dpp_u64<0xB1>(v));   // xor 1
    v = max_u64(v, dpp_u64<0x4E>(v));   // xor 2
    v = max_u64(v, dpp_u64<0x141>(v));  // other quad of the half row
    v = max_u64(v, dpp_u64<0x140>(v));  // other half of the row
    v = max_xor_u64<16>(v);
    return max_xor_u64<32>(v);
}

__device__ __forceinline__ int32_t key_index(uint64_t key) {
    return key == 0 ? -1 : static_cast<int32_t>(~static_cast<uint32_t>(key));
}

// Best key among a lane's U vectors a[j] = elements t0 + (lane + 256 j) * 8
// + k (k < 8) of a row, t0 a multiple of 256; vectors past the row hold -inf.
// Lane maximum first (packed fp16 max, which passes over NaN), then the
// element equal to it that the tie order prefers: bitrev8(i mod 256) =
// bitrev3(k) << 5 | bitrev5(lane mod 32), so within a lane a smaller
// bitrev3(k) wins, then a smaller j.  Only that one element's key is formed.
template <int U>
__device__ __forceinline__ uint64_t lane_best_key(const h8 (&a)[U], int64_t t0) {
    h2 m2 = h2(-__builtin_huge_valf16());
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
        for (int k = 0; k < 8; k += 2) m2 = __builtin_elementwise_max(m2, h2{a[j][k], a[j][k + 1]});
    }
    const half_t M = __builtin_elementwise_max(m2.x, m2.y);
    if (!(M > -__builtin_huge_valf16())) return 0;  // NaN and -inf: nothing eligible
    constexpr int kLowToHigh[8] = {7, 3, 5, 1, 6, 2, 4, 0};  // k by falling bitrev3
    int code = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
#pragma unroll
        for (int j = U - 1; j >= 0; --j)
            if (a[j][kLowToHigh[q]] == M) code = j * 8 + kLowToHigh[q];
    }
    const int64_t i = t0 + (threadIdx.x + (code >> 3) * 256) * 8 + (code & 7);
    return argmax_key(__builtin_bit_cast(uint16_t, M), i);
}

// A chunk of one tile (elements t0 .. t0 + 2048 U of a row, t0 a multiple of
// 2048, end - t0 a multiple of 8 and >= 8): lane j's vectors t0 + (j + 256 u)
// * 8, those at or past `end` reading the chunk's last in-range vector and
// then set to -inf.  Every load is unconditional -- straight-line code, so
// the compiler's later waits count exactly the loads issued before them.
template <int U>
__device__ __forceinline__ void chunk_load(const half_t* xr, int64_t t0, int64_t end, h8 (&a)[U]) {
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const int64_t i = t0 + (threadIdx.x + j * 256) * 8;
        a[j] = ld8_stream(xr + (i < end ? i : end - 8));
    }
    if (t0 + 2048 * U > end) {  // workgroup-uniform: only a row's last chunk
#pragma unroll
        for (int j = 0; j < U; ++j)
            if (t0 + (threadIdx.x + j * 256) * 8 >= end) a[j] = h8(-__builtin_huge_valf16());
    }
}

// The workgroup's best key of a chunk loaded by chunk_load (one barrier).
template <int U>
__device__ __forceinline__ uint64_t chunk_best_of(const h8 (&a)[U], int64_t t0, uint64_t* slots) {
    uint64_t best = wave_max_u64(lane_best_key<U>(a, t0));
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) slots[wave] = best;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x / kWave); ++w) t = max_u64(t, slots[w]);
    return t;
}

// Best key of elements [begin, end) of a row, over the workgroup.  The range
// is walked in tiles of 256 * VEC * U elements; every load of a tile is
// issued before any arithmetic, so a workgroup whose chunk is one tile waits
// for HBM once.  With VEC = 8, begin is a multiple of 2048 and end - begin a
// multiple of 16.
template <int VEC, int U>
__device__ __forceinline__ uint64_t chunk_best(const half_t* xr, int64_t begin, int64_t end,
                                               uint64_t* slots) {
    uint64_t best = 0;
    constexpr int64_t kTile = 256 * VEC * U;
    for (int64_t t0 = begin; t0 < end; t0 += kTile) {
        if constexpr (VEC == 8) {
            h8 a[U];
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int64_t i = t0 + (threadIdx.x + j * 256) * 8;
                a[j] = i < end ? ld8_stream(xr + i) : h8(-__builtin_huge_valf16());
            }
            best = max_u64(best, lane_best_key<U>(a, t0));
        } else {
            uint16_t a[U];
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int64_t i = t0 + threadIdx.x + j * 256;
                a[j] = i < end ? __builtin_bit_cast(uint16_t, xr[i]) : uint16_t(0);
            }
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int64_t i = t0 + threadIdx.x + j * 256;
                if (i < end) best = max_u64(best, argmax_key(a[j], i));
            }
        }
    }
    best = wave_max_u64(best);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) slots[wave] = best;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x / kWave); ++w) t = max_u64(t, slots[w]);
    return t;
}

}  // namespace mi
