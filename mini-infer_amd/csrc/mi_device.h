// mi_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// fp16 streams are moved as 16-byte vectors (8 halves, one global_load_dwordx4
// per lane), math is fp32, reductions are wave64: DPP within a 16-lane row,
// cross-row shuffles for lanes 16/32, and one LDS slot per wave for a
// workgroup total.  Nothing here allocates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

typedef _Float16 half_t;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// s_waitcnt immediate (gfx9 family) that waits for every outstanding vector
// memory operation: vmcnt = 0 (bits 3:0 and 15:14), expcnt = 7 (bits 6:4)
// and lgkmcnt = 15 (bits 11:8) left unconstrained.
constexpr int kDrainVmem = 0x0F70;  // __builtin_amdgcn_s_waitcnt(kDrainVmem)

__device__ __forceinline__ h8 ld8(const half_t* p) {
    return *reinterpret_cast<const h8*>(p);
}
__device__ __forceinline__ void st8(half_t* p, h8 v) {
    *reinterpret_cast<h8*>(p) = v;
}
// Streaming variants for data a kernel touches exactly once: the nt hint
// marks the lines for early eviction instead of keeping them in L2 / MALL.
// Measured on MI355X (1 GiB streams): read-only 6.4 -> 7.0 TB/s, copy
// 5.7 -> 6.0 TB/s, two reads + one write 5.6 -> 6.1 TB/s.
#ifndef MI_NT_LOAD
#define MI_NT_LOAD 1
#endif
#ifndef MI_NT_STORE
#define MI_NT_STORE 1
#endif
__device__ __forceinline__ h8 ld8_stream(const half_t* p) {
#if MI_NT_LOAD
    return __builtin_nontemporal_load(reinterpret_cast<const h8*>(p));
#else
    return ld8(p);
#endif
}
__device__ __forceinline__ void st8_stream(half_t* p, h8 v) {
#if MI_NT_STORE
    __builtin_nontemporal_store(v, reinterpret_cast<h8*>(p));
#else
    st8(p, v);
#endif
}
// Streaming store at device scope ("nt sc1"): written through the XCD's L2
// instead of left there dirty.  Faster where a kernel's writes are scattered
// or its launch is short (paged KV scatter, in-place Q/K passes); slower for
// the long dense streams, which keep st8_stream.
// A VALU write to the data registers of a store wider than 8 bytes needs a
// wait state after the store on gfx9.  The compiler's hazard pass does not
// see a store inside inline asm, so the asm carries the wait states itself
// (without them, following VALU code overwrote the data before the store
// read it).
// MI_WT_FORM picks the cache-policy bits of that store from the forms
// measured on the GPU (no other text can reach the asm):
//   0 = "nt sc1" (default: fastest for the in-place RoPE / Q/K-norm stores),
//   1 = "sc1", 2 = "sc0 sc1", 3 = "sc0 sc1 nt", 4 = "sc0 nt".
// Each form is followed by the same two wait states (s_nop 1).
#ifndef MI_WT_FORM
#define MI_WT_FORM 0
#endif
#if MI_WT_FORM == 0
#define MI_WT_ASM "global_store_dwordx4 %0, %1, off nt sc1\n\ts_nop 1"
#elif MI_WT_FORM == 1
#define MI_WT_ASM "global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1"
#elif MI_WT_FORM == 2
#define MI_WT_ASM "global_store_dwordx4 %0, %1, off sc0 sc1\n\ts_nop 1"
#elif MI_WT_FORM == 3
#define MI_WT_ASM "global_store_dwordx4 %0, %1, off sc0 sc1 nt\n\ts_nop 1"
#elif MI_WT_FORM == 4
#define MI_WT_ASM "global_store_dwordx4 %0, %1, off sc0 nt\n\ts_nop 1"
#else
#error "MI_WT_FORM must be 0-4"
#endif
__device__ __forceinline__ void st8_stream_wt(half_t* p, h8 v) {
    asm volatile(MI_WT_ASM : : "v"(p), "v"(v) : "memory");
}
// A wait for every outstanding vector-memory operation, placed after a
// store when S: each store then waits for the one before it.
template <bool S>
__device__ __forceinline__ void store_gap() {
    if constexpr (S) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// Store selected per kernel at compile time.
template <bool WT>
__device__ __forceinline__ void st8_out(half_t* p, h8 v) {
    if constexpr (WT) st8_stream_wt(p, v); else st8_stream(p, v);
}

// Pins a value to an fp32 register.  The compiler may otherwise fold
// "fp32 result, then fp16 conversion" into one mixed-precision FMA
// (v_fma_mixlo_f16 a, b, 0) that rounds the exact product straight to fp16;
// reference kernels round to fp32 first (e.g. __float2half(a * b - c * d)),
// and the two differ in rare ties -- and in the sign of a zero product,
// since the fused form adds +0 to it.
__device__ __forceinline__ float fp32_rounded(float f) {
    asm volatile("" : "+v"(f));
    return f;
}

// Round-to-nearest-even fp32 -> fp16 of a value first rounded to fp32
// (v_cvt_f16_f32 under the default mode): RN16(RN32(expression)), as the
// reference's __float2half(expression) computes it.
__device__ __forceinline__ half_t to_half(float f) { return (half_t)fp32_rounded(f); }

// --- DPP helpers ------------------------------------------------------------
// dpp_ctrl encodings (GFX9 DPP): quad_perm = 8-bit lane map within a quad,
// 0x141 = row_half_mirror (lane i of 8 reads 7-i), 0x140 = row_mirror (lane i
// of 16 reads 15-i).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Lane i's value and lane (i ^ 16)'s, or (i ^ 32)'s, through gfx950's
// v_permlane16_swap / v_permlane32_swap (VALU, no LDS round trip as a
// ds_bpermute shuffle takes).  Swapping a register with itself leaves, in
// the two results, lane i's own value and its partner's (in one order or the
// other); callers combine them with a commutative operation, so both lanes
// of a pair get the same bits.  Every lane of the wave must be active.
// (Used by the 64-bit argmax reduction, where it replaced twelve shuffles:
// 7.7 -> 7.3 us at [64, 152064].  For the fp32 reductions below it measured
// no better -- softmax [64, 152064] 9.8 -> 10.2 us -- so they keep
// __shfl_xor across rows.)
__device__ __forceinline__ void pair_xor16(uint32_t v, uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}
__device__ __forceinline__ void pair_xor32(uint32_t v, uint32_t& a, uint32_t& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}

// Sum across aligned groups of G lanes (G a power of two, 1..64); every lane
// of a group receives the group total.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "G must be a power of two <= 64");
    if constexpr (G >= 2) v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]: xor 1
    if constexpr (G >= 4) v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]: xor 2
    if constexpr (G >= 8) v += dpp_f<0x141>(v);   // other quad of the 8-lane half row
    if constexpr (G >= 16) v += dpp_f<0x140>(v);  // other half of the 16-lane row
    if constexpr (G >= 32) v += __shfl_xor(v, 16, kWave);
    if constexpr (G >= 64) v += __shfl_xor(v, 32, kWave);
    return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "G must be a power of two <= 64");
    if constexpr (G >= 2) v = fmaxf(v, dpp_f<0xB1>(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp_f<0x4E>(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp_f<0x141>(v));
    if constexpr (G >= 16) v = fmaxf(v, dpp_f<0x140>(v));
    if constexpr (G >= 32) v = fmaxf(v, __shfl_xor(v, 16, kWave));
    if constexpr (G >= 64) v = fmaxf(v, __shfl_xor(v, 32, kWave));
    return v;
}

// Workgroup-wide sum with a single barrier: each wave reduces in registers,
// lane 0 publishes to LDS, then every lane folds the per-wave partials in the
// same fixed order (so all lanes agree bit for bit).  `slots` needs one float
// per wave; blockDim.x must be a multiple of 64.
__device__ __forceinline__ float block_sum(float v, float* slots) {
    v = group_sum<kWave>(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) slots[wave] = v;
    __syncthreads();
    const int nwaves = blockDim.x / kWave;
    float t = 0.0f;
    for (int i = 0; i < nwaves; ++i) t += slots[i];
    return t;
}

// RPW independent workgroup-wide sums with one barrier; `slots` needs
// RPW floats per wave.
template <int RPW>
__device__ __forceinline__ void block_sum_n(float (&v)[RPW], float* slots) {
    const int wave = threadIdx.x / kWave;
#pragma unroll
    for (int r = 0; r < RPW; ++r) v[r] = group_sum<kWave>(v[r]);
    if ((threadIdx.x & (kWave - 1)) == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) slots[wave * RPW + r] = v[r];
    }
    __syncthreads();
    const int nwaves = blockDim.x / kWave;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float t = 0.0f;
        for (int i = 0; i < nwaves; ++i) t += slots[i * RPW + r];
        v[r] = t;
    }
}

__device__ __forceinline__ float block_max(float v, float* slots) {
    v = group_max<kWave>(v);
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) slots[wave] = v;
    __syncthreads();
    const int nwaves = blockDim.x / kWave;
    float t = -INFINITY;
    for (int i = 0; i < nwaves; ++i) t = fmaxf(t, slots[i]);
    return t;
}

// Sum of squares of a head's slice pair, x1 (first half) and x2 (second half)
// of 8 halves each, as every fused Q/K-norm + RoPE kernel forms it (they must
// agree bit for bit: the one-launch attention pre-processing is checked
// against the separate launches).  MI_SUMSQ_FORM 2 (default): packed fp16
// dot products accumulated in fp32 (v_dot2_f32_f16) over x1 then x2 -- 8
// instructions instead of 16 conversions and 16 fma, Q/K-norm + RoPE at
// T = 6064 18.0 -> 17.8 us; the products of fp16 values are exact and the
// hardware accumulation's rounding differs from an fma chain's by an fp32
// ulp or so, far inside the norm's tolerance.  0: one fma chain over
// (x1[e], x2[e]) pairs.
#ifndef MI_SUMSQ_FORM
#define MI_SUMSQ_FORM 2
#endif
__device__ __forceinline__ float pair_sumsq(const h8& x1, const h8& x2) {
    float ss = 0.0f;
#if MI_SUMSQ_FORM == 2
#pragma unroll
    for (int e = 0; e < 8; e += 2) ss = __builtin_amdgcn_fdot2(h2{x1[e], x1[e + 1]}, h2{x1[e], x1[e + 1]}, ss, false);
#pragma unroll
    for (int e = 0; e < 8; e += 2) ss = __builtin_amdgcn_fdot2(h2{x2[e], x2[e + 1]}, h2{x2[e], x2[e + 1]}, ss, false);
#else
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float f1 = (float)x1[e], f2 = (float)x2[e];
        ss = fmaf(f1, f1, ss);
        ss = fmaf(f2, f2, ss);
    }
#endif
    return ss;
}

// floor(u / d) for integers 0 <= u < 2^22 and d >= 1, given inv_d = 1.0f / d
// (correctly rounded): (u + 0.5) * inv_d lies within (u + 0.5) * 2^-23 of
// (u + 0.5) / d, which is less than the 0.5 / d separating that value from
// the integers on either side.  A few instructions instead of a runtime
// integer division.
__device__ __forceinline__ int small_div(int u, float inv_d) {
    return static_cast<int>((static_cast<float>(u) + 0.5f) * inv_d);
}

// exp(x) through the hardware base-2 exponential (v_exp_f32, ~1 ulp).
__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// x / (1 + exp(-y)): shared tail of silu (y = x) and of gelu_tanh, which is
// exactly x * sigmoid(2u) since 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)).
// exp overflow to +inf gives x / inf = 0, the correct limit.
__device__ __forceinline__ float x_sigmoid(float x, float y) {
    return x * __builtin_amdgcn_rcpf(1.0f + fast_exp(-y));
}

__device__ __forceinline__ float silu_mul(float g, float u) { return x_sigmoid(g, g) * u; }

__device__ __forceinline__ float gelu_tanh(float x) {
    const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
    const float k1 = 0.044715f;
    const float inner = k0 * (x + k1 * x * x * x);
    return x_sigmoid(x, 2.0f * inner);
}

}  // namespace mi
