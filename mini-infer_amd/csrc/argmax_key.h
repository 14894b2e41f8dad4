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
// Lane maximum first, then the element equal to it that the tie order
// prefers: bitrev8(i mod 256) = bitrev3(k) << 5 | bitrev5(lane mod 32), so
// within a lane a smaller bitrev3(k) wins, then a smaller j.  Only that one
// element's key is formed.
//
// Both steps are shallow trees (the tail after a wave's last load is
// latency, not VALU throughput): a NaN-propagating packed maximum
// (v_pk_maximum3_f16, no canonicalisation), and for the tie search one
// packed subtract and one OR per pair of elements -- x - m is +0 exactly
// when x == m (m normal and finite) and has its sign bit set otherwise, so
// (x - m) | rank is the element's rank when it matches and >= 0x8000 when
// not -- and a packed-u16 minimum tree over those.  A lane whose maximum is
// NaN, infinite, zero or subnormal (where that subtraction might not
// separate) takes the element-by-element search (lane_best_exact).
//
// The lane's pick: false when nothing is eligible; else its value bits mb
// (never NaN or -inf) and its place, element k of vector j.
template <int U>
__device__ __forceinline__ bool lane_best_exact(const h8 (&a)[U], uint16_t& mb, int& j, int& k) {
    h2 m2 = h2(-__builtin_huge_valf16());
#pragma unroll
    for (int q = 0; q < U; ++q) {
#pragma unroll
        for (int t = 0; t < 8; t += 2) m2 = __builtin_elementwise_max(m2, h2{a[q][t], a[q][t + 1]});
    }
    const half_t M = __builtin_elementwise_max(m2.x, m2.y);
    if (!(M > -__builtin_huge_valf16())) return false;  // NaN and -inf: nothing eligible
    constexpr int kLowToHigh[8] = {7, 3, 5, 1, 6, 2, 4, 0};  // k by falling bitrev3
    int code = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
#pragma unroll
        for (int t = U - 1; t >= 0; --t)
            if (a[t][kLowToHigh[q]] == M) code = t * 8 + kLowToHigh[q];
    }
    mb = __builtin_bit_cast(uint16_t, M);
    j = code >> 3;
    k = code & 7;
    return true;
}

template <int U>
__device__ __forceinline__ bool lane_best(const h8 (&a)[U], uint16_t& mb, int& j, int& k) {
    static_assert(8 * U <= 0x8000, "ranks must stay below the sign bit");
    typedef unsigned short u2 __attribute__((ext_vector_type(2)));
    constexpr int N = 4 * U;  // element pairs
    h2 p[N];
#pragma unroll
    for (int q = 0; q < U; ++q) {
#pragma unroll
        for (int c = 0; c < 4; ++c) p[4 * q + c] = h2{a[q][2 * c], a[q][2 * c + 1]};
    }
    h2 t[N];
#pragma unroll
    for (int q = 0; q < N; ++q) t[q] = p[q];
#pragma unroll
    for (int s = 1; s < N; s *= 2) {
#pragma unroll
        for (int q = 0; q + s < N; q += 2 * s) t[q] = __builtin_elementwise_maximum(t[q], t[q + s]);
    }
    const half_t M = __builtin_elementwise_maximum(t[0].x, t[0].y);
    mb = __builtin_bit_cast(uint16_t, M);
    // NaN, +-inf, zero or subnormal: the exact search (rare; skipped when no
    // lane needs it)
    const uint32_t ex = mb & 0x7c00u;
    if (ex == 0x7c00u || ex == 0) return lane_best_exact<U>(a, mb, j, k);
    const h2 mm = h2{M, M};
    u2 d[N];
#pragma unroll
    for (int q = 0; q < U; ++q) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            // ranks of elements 2c and 2c + 1 of vector q: bitrev3(element) * U + q
            constexpr int kBrev3[8] = {0, 4, 2, 6, 1, 5, 3, 7};
            const u2 rank = u2{static_cast<unsigned short>(kBrev3[2 * c] * U + q),
                               static_cast<unsigned short>(kBrev3[2 * c + 1] * U + q)};
            d[4 * q + c] = __builtin_bit_cast(u2, p[4 * q + c] - mm) | rank;
        }
    }
#pragma unroll
    for (int s = 1; s < N; s *= 2) {
#pragma unroll
        for (int q = 0; q + s < N; q += 2 * s) d[q] = __builtin_elementwise_min(d[q], d[q + s]);
    }
    const int r = d[0].x < d[0].y ? d[0].x : d[0].y;
    j = r % U;
    k = static_cast<int>(__builtin_bitreverse32(static_cast<uint32_t>(r / U)) >> 29);
    return true;
}

template <int U>
__device__ __forceinline__ uint64_t lane_best_key(const h8 (&a)[U], int64_t t0) {
    uint16_t mb;
    int j, k;
    if (!lane_best<U>(a, mb, j, k)) return 0;
    return argmax_key(mb, t0 + (threadIdx.x + j * 256) * 8 + k);
}

// The same pick as a 32-bit code inside one chunk of a 256-lane workgroup
// with U <= 4 (chunk offset o = (lane + 256 j) * 8 + k < 8192):
//   [ordered value : 16 | 255 - bitrev8(o mod 256) : 8 | 31 - o / 256 : 5]
// -- the 64-bit key's order restricted to the chunk (its start a multiple
// of 256), so a 32-bit wave maximum replaces the 64-bit one.  0 = nothing.
template <int U>
__device__ __forceinline__ uint32_t lane_best_code(const h8 (&a)[U]) {
    static_assert(U <= 4, "chunk offsets must stay below 8192");
    uint16_t mb;
    int j, k;
    if (!lane_best<U>(a, mb, j, k)) return 0;
    uint32_t h = mb == 0x8000u ? 0u : mb;  // -0 == +0
    const uint32_t ord = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
    const uint32_t lo = ((threadIdx.x & 31u) << 3) | static_cast<uint32_t>(k);
    const uint32_t tie = 255u - (__builtin_bitreverse32(lo) >> 24);
    const uint32_t hi = (threadIdx.x >> 5) + 8u * static_cast<uint32_t>(j);
    return (ord << 16) | (tie << 8) | (31u - hi);
}

// The 64-bit key of chunk code c for a chunk starting at t0 (a multiple of
// 256).
__device__ __forceinline__ uint64_t code_key(uint32_t c, int64_t t0) {
    if (c == 0) return 0;
    const uint32_t tie = (c >> 8) & 255u;
    const uint32_t lo = __builtin_bitreverse32(255u - tie) >> 24;
    const int64_t i = t0 + ((31 - static_cast<int64_t>(c & 31u)) << 8) + lo;
    return (static_cast<uint64_t>(c >> 16) << 48) | (static_cast<uint64_t>(tie) << 32) |
           static_cast<uint64_t>(~static_cast<uint32_t>(i));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xB1, 0xF, 0xF, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x4E, 0xF, 0xF, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x141, 0xF, 0xF, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x140, 0xF, 0xF, false)));
    uint32_t x, y;
    pair_xor16(v, x, y);
    v = max(x, y);
    pair_xor32(v, x, y);
    return max(x, y);
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
    const uint32_t best = wave_max_u32(lane_best_code<U>(a));
    const int wave = threadIdx.x / kWave;
    uint32_t* s32 = reinterpret_cast<uint32_t*>(slots);
    if ((threadIdx.x & (kWave - 1)) == 0) s32[wave] = best;
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < 256 / kWave; ++w) t = max(t, s32[w]);
    return code_key(t, t0);
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
