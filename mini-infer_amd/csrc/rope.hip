// rope.hip -- NeoX half-rotation RoPE for gfx950: table-driven rotation,
// table generation, and the fused in-place Q+K rotation with cos/sin made in
// registers.
//
// Arithmetic follows the reference (src/kernels/rope_kernel.cu:27-54, 65-77;
// src/layers/rope.cpp:20-28):
//   angle  = float(pos) * inv_freq[i]           (fp32 product)
//   c, s   = half(cos(angle)), half(sin(angle))  (fp16-rounded table values)
//   y[i]   = x[i] * c - x[i + h] * s,  y[i + h] = x[i + h] * c + x[i] * s
// Both products in a rotation are exact in fp32 (11-bit x 11-bit
// significands), so the fp32 result is one rounding of the exact value, which
// is then rounded to fp16 -- the same two roundings the reference performs, so
// outputs match it bit for bit given equal tables.
//
// cos/sin: a compact fp32 sin/cos (rope_sincos.h: Cody-Waite reduction,
// Taylor polynomials; a few ulp) is rounded to fp16; when the value lies
// within 2^-20 (relative, 2^-29 absolute floor) of an fp16 rounding boundary
// the angle is re-evaluated in fp64, so the fp16 value always equals
// half(RN32(cos(angle))) computed from the exact cosine.
//
// Design (HBM-bound: 8 bytes/element in place, + 8 bytes/token of positions):
//   a 256-lane workgroup takes 1-8 tokens.  Every lane first issues
//   the 16-byte loads of its (token, head, 8-element) units -- x[i..i+7] and
//   x[h+i..h+i+7] -- then the workgroup builds each token's cos/sin row in LDS
//   once (instead of once per head), and after a single barrier each lane
//   rotates its units.  For Qwen2.5 (28 + 4 heads x 8 units) a token is 256
//   units, so with 2 tokens per workgroup each lane has two units in flight.
#include <math.h>

#include "mi_device.h"
#include "mi_host.h"
#include "rope_sincos.h"

// Stores of the in-place RoPE and fused Q/K-norm + RoPE kernels: write-through
// ("nt sc1", st8_stream_wt) measured 1-3 points faster than plain non-temporal.
#ifndef MI_WT_ROPE
#define MI_WT_ROPE 1
#endif
#ifndef MI_WT_QKNR
#define MI_WT_QKNR 1
#endif

namespace mi {
namespace {

constexpr int kMaxHalf = 256;  // head_dim <= 512

// LDS position of element i of a half-row of n entries (n a multiple of 8),
// for lanes that each read the 8 entries c*8 .. c*8+7 as two 16-byte LDS
// reads: entries 0-3 of every lane's group sit together in the first n/2
// slots and entries 4-7 in the second, so lane c reads slots 4c .. 4c+3 and
// n/2 + 4c .. n/2 + 4c+3.  Eight consecutive lanes then cover 32 distinct
// banks per read; with the plain layout (lane c at 8c) lanes c and c+4 fall
// on the same banks and every read took a second pass (rocprof
// LdsBankConflict 0.97 conflicts per access).
__device__ __forceinline__ int quad_split(int i, int n) {
    return ((i & 4) ? (n >> 1) : 0) + ((i >> 3) << 2) + (i & 3);
}

// Host-computed inverse frequencies travel by value in the kernel arguments.
struct InvFreq {
    float v[kMaxHalf];
};

// fp16 cos/sin of an fp32 angle, equal to half(RN32(exact)) (see file header).
// |ang| <= 2^20: the fp32 Cody-Waite form, re-evaluated in fp64 when a value
// lies within rope_guard_width of an fp16 rounding boundary; larger angles
// (positions beyond 2^20 / inv_freq) go straight to the fp64 form
// (rope_sincos_any: Cody-Waite to 2^24, Payne-Hanek above), which covers
// every fp32 angle -- so every int64 position -- with no range limit.
__device__ __forceinline__ bool near_half_boundary(float v) {
    const float d = rope_guard_width(v);
    return to_half(v - d) != to_half(v + d);
}

__device__ __forceinline__ void cos_sin_half(float ang, half_t& hc, half_t& hs) {
    float s, c;
    rope_sincos_f32(ang, &s, &c);
    if (!rope_sincos_f32_ok(ang) || near_half_boundary(c) || near_half_boundary(s)) {
        double sd, cd;
        rope_sincos_any(ang, &sd, &cd);
        c = static_cast<float>(cd);
        s = static_cast<float>(sd);
    }
    hc = to_half(c);
    hs = to_half(s);
}

template <int VEC>
struct HVec;
template <>
struct HVec<8> {
    typedef h8 T;
    __device__ static T load(const half_t* p) { return ld8(p); }
    __device__ static void store(half_t* p, T v) { st8(p, v); }
};
template <>
struct HVec<1> {
    typedef half_t T;
    __device__ static T load(const half_t* p) { return *p; }
    __device__ static void store(half_t* p, T v) { *p = v; }
};

template <int VEC>
__device__ __forceinline__ float elem(const typename HVec<VEC>::T& v, int k) {
    if constexpr (VEC == 1) return (float)v; else return (float)v[k];
}
template <int VEC>
__device__ __forceinline__ void set_elem(typename HVec<VEC>::T& v, int k, float f) {
    if constexpr (VEC == 1) v = to_half(f); else v[k] = to_half(f);
}

// Tokens per 256-lane workgroup, chosen per launch from {1, 2, 4, 8} (see
// fill_tokens_per_wg); each lane issues the loads of TPW units (one per
// token for a 256-unit token, the Qwen2.5 case) before the table work.

// TPW tokens per 256-lane workgroup.  Sources q_in/k_in, destinations
// q_out/k_out (may equal the sources).  FROM_POS: cos/sin from positions +
// inv_freq, else from fp16 tables [T, half].  A unit is one (token, head,
// VEC-element slice) pair: x[i..i+VEC) and x[h+i..h+i+VEC).  BIAS: the
// projection bias bq [Hq * hd] / bk [Hkv * hd] is added first, rounded to
// fp16 as the reference's launch_add_bias stores it
// (src/kernels/model_utils_kernel.cu:19), and the sum rotated.
// (8 tokens: held to 128 VGPRs, 4 waves per SIMD; the compiler otherwise
// settles at 130 and the residency drops to 3)
template <int VEC, bool FROM_POS, int TPW, bool BIAS = false>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(TPW == 8 ? 4 : 1))) void rope_kernel(const half_t* q_in, half_t* q_out, int Hq,
                                                   const half_t* k_in, half_t* k_out, int Hkv,
                                                   const int64_t* __restrict__ positions,
                                                   const half_t* __restrict__ cos_t,
                                                   const half_t* __restrict__ sin_t, int64_t T,
                                                   int hd, InvFreq inv,
                                                   const half_t* __restrict__ bq = nullptr,
                                                   const half_t* __restrict__ bk = nullptr) {
    typedef HVec<VEC> V;
    __shared__ float cs[TPW][2 * kMaxHalf];
    const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * TPW;
    const int ntok = static_cast<int>(T - tok0 < TPW ? T - tok0 : TPW);
    const int half = hd >> 1;
    const int cph = half / VEC;                // units per head
    const int upt = (Hq + Hkv) * cph;          // units per token
    const int units = ntok * upt;

    const float inv_upt = 1.0f / static_cast<float>(upt);
    const float inv_cph = 1.0f / static_cast<float>(cph);
    // units < 2^22 (checked at launch), so small_div is exact
    auto locate = [&](int u, const half_t*& src, half_t*& dst, const half_t** bias = nullptr) {
        const int t = small_div(u, inv_upt);
        const int rem = u - t * upt;
        const int h = small_div(rem, inv_cph);
        const int c = rem - h * cph;
        const int64_t tok = tok0 + t;
        if (h < Hq) {
            const int64_t base = (tok * Hq + h) * static_cast<int64_t>(hd) + c * VEC;
            src = q_in + base;
            dst = q_out + base;
            if (BIAS && bias) *bias = bq + h * hd + c * VEC;
        } else {
            const int64_t base = (tok * Hkv + (h - Hq)) * static_cast<int64_t>(hd) + c * VEC;
            src = k_in + base;
            dst = k_out + base;
            if (BIAS && bias) *bias = bk + (h - Hq) * hd + c * VEC;
        }
        // offset of this unit's first cos entry in cs (quad_split layout for VEC = 8)
        return t * (2 * kMaxHalf) + (VEC == 8 ? c * 4 : c * VEC);
    };

    // 1. issue up to TPW units' loads per lane before the table work,
    //    so HBM latency overlaps the sincos evaluation
    typename V::T x1[TPW], x2[TPW];
    typename V::T b1[BIAS ? TPW : 1], b2[BIAS ? TPW : 1];  // bias slices (BIAS)
#pragma unroll
    for (int p = 0; p < TPW; ++p) {
        const int u = threadIdx.x + p * 256;
        if (u < units) {
            const half_t* src;
            half_t* dst;
            const half_t* bp = nullptr;
            locate(u, src, dst, &bp);
            if constexpr (VEC == 8) {
                x1[p] = ld8_stream(src);
                x2[p] = ld8_stream(src + half);
            } else {
                x1[p] = V::load(src);
                x2[p] = V::load(src + half);
            }
            if constexpr (BIAS) {  // a few KB every token re-reads: plain loads
                b1[p] = V::load(bp);
                b2[p] = V::load(bp + half);
            }
        }
    }

    // 2. each token's cos/sin row, once per token (not once per head)
    for (int idx = threadIdx.x; idx < ntok * half; idx += 256) {
        const int t = idx / half;
        const int i = idx - t * half;
        const int64_t tok = tok0 + t;
        half_t hc, hs;
        if constexpr (FROM_POS) {
            const float ang = static_cast<float>(positions[tok]) * inv.v[i];
            cos_sin_half(ang, hc, hs);
        } else {
            hc = cos_t[tok * half + i];
            hs = sin_t[tok * half + i];
        }
        const int li = VEC == 8 ? quad_split(i, half) : i;
        cs[t][li] = (float)hc;
        cs[t][kMaxHalf + li] = (float)hs;
    }
    __syncthreads();

    // 3. rotate: y1 = x1 c - x2 s, y2 = x2 c + x1 s
    const float* csf = &cs[0][0];
    auto rotate = [&](int u, const typename V::T& a1, const typename V::T& a2,
                      const typename V::T* c1, const typename V::T* c2) {
        const half_t* src;
        half_t* dst;
        const int off = locate(u, src, dst);
        typename V::T y1, y2;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            // VEC = 8: entries 4-7 sit half/2 slots on (quad_split)
            const int kk = (VEC == 8 && (k & 4)) ? ((half >> 3) << 2) + (k & 3) : k;
            const float cv = csf[off + kk];
            const float sv = csf[off + kMaxHalf + kk];
            float a = elem<VEC>(a1, k), b = elem<VEC>(a2, k);
            if constexpr (BIAS) {
                a = (float)to_half(a + elem<VEC>(*c1, k));
                b = (float)to_half(b + elem<VEC>(*c2, k));
            }
            set_elem<VEC>(y1, k, fp32_rounded(a * cv - b * sv));
            set_elem<VEC>(y2, k, fp32_rounded(b * cv + a * sv));
        }
        if constexpr (VEC == 8) {
            st8_out<MI_WT_ROPE>(dst, y1);
            st8_out<MI_WT_ROPE>(dst + half, y2);
        } else {
            V::store(dst, y1);
            V::store(dst + half, y2);
        }
    };
#pragma unroll
    for (int p = 0; p < TPW; ++p) {
        const int u = threadIdx.x + p * 256;
        if (u < units) rotate(u, x1[p], x2[p], &b1[BIAS ? p : 0], &b2[BIAS ? p : 0]);
    }
    for (int u = threadIdx.x + TPW * 256; u < units; u += 256) {
        const half_t* src;
        half_t* dst;
        const half_t* bp = nullptr;
        locate(u, src, dst, &bp);
        typename V::T c1{}, c2{};
        if constexpr (BIAS) {
            c1 = V::load(bp);
            c2 = V::load(bp + half);
        }
        rotate(u, V::load(src), V::load(src + half), &c1, &c2);
    }
}

// ---------------------------------------------------------------------------
// Fused per-head RMSNorm + RoPE, in place, for Q and K: the reference runs
// launch_rmsnorm on the Q rows and the K rows (D = head_dim, in place,
// src/layers/attention.cpp:757-768) and then RoPE on both (:779-780).  Here
// a head's elements are held by CPH = head_dim/16 lanes -- each lane owns
// x[i..i+7] and x[h+i..h+i+7] -- so the sum of squares is a CPH-lane DPP
// reduction, the normalised value is rounded to fp16 exactly where the
// reference writes it, and the rotation consumes it from registers: one HBM
// read and one write of Q and K instead of two of each.
// ---------------------------------------------------------------------------
template <int CPH, int TPW>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(half_t* q, int Hq, half_t* k, int Hkv,
                                                           const half_t* __restrict__ wq,
                                                           const half_t* __restrict__ wk,
                                                           const int64_t* __restrict__ positions,
                                                           int64_t T, float eps, float w_bias,
                                                           InvFreq inv) {
    constexpr int HALF = CPH * 8;
    constexpr int HD = 2 * HALF;
    __shared__ float cs[TPW][2 * kMaxHalf];
    __shared__ h8 wl[2][HD / 8];  // Q and K weights, read at use (no registers held)
    const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * TPW;
    const int ntok = static_cast<int>(T - tok0 < TPW ? T - tok0 : TPW);
    const int upt = (Hq + Hkv) * CPH;  // units per token
    const int units = ntok * upt;
    const int c = threadIdx.x & (CPH - 1);  // a lane's slice is the same for every unit

    if (threadIdx.x < HD / 8)
        wl[0][threadIdx.x] = ld8(wq + threadIdx.x * 8);
    else if (threadIdx.x < HD / 4 && Hkv > 0)
        wl[1][threadIdx.x - HD / 8] = ld8(wk + (threadIdx.x - HD / 8) * 8);

    // unit u -> (token, head); returns the head's base pointer (units < 2^22,
    // checked at launch, so small_div is exact)
    const float inv_upt = 1.0f / static_cast<float>(upt);
    auto head_ptr = [&](int u, bool& is_k, int& t) -> half_t* {
        t = small_div(u, inv_upt);
        const int h = (u - t * upt) / CPH;
        const int64_t tok = tok0 + t;
        is_k = h >= Hq;
        return is_k ? k + (tok * Hkv + (h - Hq)) * static_cast<int64_t>(HD)
                    : q + (tok * Hq + h) * static_cast<int64_t>(HD);
    };

    h8 x1[TPW], x2[TPW];
#pragma unroll
    for (int p = 0; p < TPW; ++p) {
        const int u = threadIdx.x + p * 256;
        x1[p] = h8(0);
        x2[p] = h8(0);
        if (u < units) {
            bool is_k;
            int t;
            half_t* hp = head_ptr(u, is_k, t);
            x1[p] = ld8_stream(hp + c * 8);
            x2[p] = ld8_stream(hp + HALF + c * 8);
        }
    }

    for (int idx = threadIdx.x; idx < ntok * HALF; idx += 256) {
        const int t = idx / HALF;
        const int i = idx - t * HALF;
        half_t hc, hs;
        cos_sin_half(static_cast<float>(positions[tok0 + t]) * inv.v[i], hc, hs);
        cs[t][i] = (float)hc;
        cs[t][kMaxHalf + i] = (float)hs;
    }
    __syncthreads();

    // Every lane runs process() for every step (the DPP reduction needs the
    // whole wave); lanes past `units` contribute zeros and store nothing.
    auto process = [&](int u, const h8& a1, const h8& a2) {
        const bool valid = u < units;
        float ss = pair_sumsq(a1, a2);
        ss = group_sum<CPH>(ss);
        if (!valid) return;
        bool is_k;
        int t;
        half_t* hp = head_ptr(u, is_k, t);
        const float rrms = rsqrtf(ss / static_cast<float>(HD) + eps);
        const h8 w1 = wl[is_k][c], w2 = wl[is_k][CPH + c];
        const float* cst = &cs[t][0];
        h8 y1, y2;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // the normalised value as the reference stores it (fp16)
            const float n1 = (float)to_half((float)a1[e] * rrms * ((float)w1[e] + w_bias));
            const float n2 = (float)to_half((float)a2[e] * rrms * ((float)w2[e] + w_bias));
            const float cv = cst[c * 8 + e], sv = cst[kMaxHalf + c * 8 + e];
            y1[e] = to_half(fp32_rounded(n1 * cv - n2 * sv));
            y2[e] = to_half(fp32_rounded(n2 * cv + n1 * sv));
        }
        st8_out<MI_WT_QKNR>(hp + c * 8, y1);
        st8_out<MI_WT_QKNR>(hp + HALF + c * 8, y2);
    };
#pragma unroll
    for (int p = 0; p < TPW; ++p) process(threadIdx.x + p * 256, x1[p], x2[p]);
    for (int base = TPW * 256; base < units; base += 256) {
        const int u = base + threadIdx.x;
        h8 a1 = h8(0), a2 = h8(0);
        if (u < units) {
            bool is_k;
            int t;
            half_t* hp = head_ptr(u, is_k, t);
            a1 = ld8_stream(hp + c * 8);
            a2 = ld8_stream(hp + HALF + c * 8);
        }
        process(u, a1, a2);
    }
}

// Persistent, software-pipelined form of qk_norm_rope_kernel: a grid of
// about the resident capacity walks groups of G tokens (G * units-per-token
// <= 256 * P, G * head_dim/2 <= 256), and while it normalises and rotates
// group g it already holds the loads of the next group in flight and builds
// that group's cos/sin rows in the other half of a double-buffered LDS table.
// HBM reads of the next group overlap the writes of the current one, which a
// single round of load-everything / barrier / store-everything workgroups
// cannot do.
//
// The vector-memory counter retires loads and stores in issue order, so the
// loop is arranged so that no wait drains more than it needs to:
//   * each step begins with one full drain -- the current group's data and
//     the next group's positions, both issued a step earlier, and the last
//     step's stores -- and only then issues its prefetch, so nothing inside
//     the step waits for the loads just issued (with loads and stores both
//     outstanding, the compiler can only wait for a load with a full drain);
//   * the two register buffers are used ping-pong (no loop-carried copies);
//   * each lane's table entry (token-in-group, frequency index) is the same in
//     every group, so its inv_freq is read once.
// One barrier per group: the table half written in a step was last read in
// the step before, ahead of this step's barrier.

template <int CPH, int P>
__global__ __launch_bounds__(256) void qk_norm_rope_pipe_kernel(
    half_t* q, int Hq, half_t* k, int Hkv, const half_t* __restrict__ wq,
    const half_t* __restrict__ wk, const int64_t* __restrict__ positions, int64_t T, int G,
    float eps, float w_bias, InvFreq inv) {
    constexpr int HALF = CPH * 8;
    constexpr int HD = 2 * HALF;
    constexpr int kTab = 256;  // cos (or sin) entries per table half: G * HALF <= kTab
    __shared__ float cs[2][2 * kTab];
    // (w + bias) in fp32 for Q heads (row 0) and K heads (row 1), read from
    // LDS per unit rather than held in 32 registers across the loop; the
    // loop's first barrier orders these writes before any read.
    __shared__ float wt[2][HD];
    for (int i = threadIdx.x; i < 2 * HD; i += 256) {
        const int r = i / HD, j = i - r * HD;
        const int hh = j >= HALF ? HALF : 0;  // quad_split within each half
        wt[r][hh + quad_split(j - hh, HALF)] =
            (r == 0 || Hkv > 0) ? (float)(r == 0 ? wq : wk)[j] + w_bias : 0.0f;
    }
    const int upt = (Hq + Hkv) * CPH;
    const int c = threadIdx.x & (CPH - 1);
    const int64_t ngroups = (T + G - 1) / G;
    const int64_t stride = gridDim.x;

    // A lane's slots are the same (token-in-group, head) pairs in every
    // group; only the group's first token moves.
    int slot_t[P];
    int64_t slot_off[P];  // element offset of the head at token 0 of the group
    bool slot_k[P], slot_on[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int u = threadIdx.x + p * 256;
        const int t = u / upt;
        const int h = (u - t * upt) / CPH;
        slot_t[p] = t;
        slot_on[p] = t < G;
        slot_k[p] = h >= Hq;
        slot_off[p] = slot_k[p] ? (static_cast<int64_t>(t) * Hkv + (h - Hq)) * HD + c * 8
                                : (static_cast<int64_t>(t) * Hq + h) * HD + c * 8;
    }
    // This lane's table entry.
    const bool tab_on = static_cast<int>(threadIdx.x) < G * HALF;
    const int tab_t = threadIdx.x / HALF;
    const float tab_f = inv.v[threadIdx.x % HALF];

    auto slot_ptr = [&](int p, int64_t tok0) -> half_t* {
        return slot_k[p] ? k + tok0 * Hkv * HD + slot_off[p] : q + tok0 * Hq * HD + slot_off[p];
    };
    auto load_position = [&](int64_t g) -> int64_t {
        const int64_t tok = g * G + tab_t;
        return (g < ngroups && tab_on && tok < T) ? positions[tok] : 0;
    };
    auto load_group = [&](int64_t g, h8* a1, h8* a2) {
        const int64_t tok0 = g * G;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            a1[p] = h8(0);
            a2[p] = h8(0);
            if (slot_on[p] && tok0 + slot_t[p] < T) {
                const half_t* hp = slot_ptr(p, tok0);
                a1[p] = ld8_stream(hp);
                a2[p] = ld8_stream(hp + HALF);
            }
        }
    };
    auto build_table = [&](int64_t pos, float* tab) {
        if (tab_on) {
            half_t hc, hs;
            cos_sin_half(static_cast<float>(pos) * tab_f, hc, hs);
            const int li = tab_t * HALF + quad_split(threadIdx.x - tab_t * HALF, HALF);
            tab[li] = (float)hc;
            tab[kTab + li] = (float)hs;
        }
    };
    auto process = [&](int64_t g, const float* tab, const h8* a1, const h8* a2) {
        const int64_t tok0 = g * G;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            float ss = pair_sumsq(a1[p], a2[p]);
            ss = group_sum<CPH>(ss);
            if (!slot_on[p] || tok0 + slot_t[p] >= T) continue;
            const float rrms = rsqrtf(ss / static_cast<float>(HD) + eps);
            // weights and table in the quad_split layout: entry e of this
            // lane's group at c*4 + (e & 3), plus HALF/2 for e >= 4
            const float* w = &wt[slot_k[p] ? 1 : 0][c * 4];
            const float* cst = tab + slot_t[p] * HALF + c * 4;
            h8 y1, y2;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int le = (e & 4) ? HALF / 2 + (e & 3) : e;
                const float v1 = (float)to_half((float)a1[p][e] * rrms * w[le]);
                const float v2 = (float)to_half((float)a2[p][e] * rrms * w[HALF + le]);
                const float cv = cst[le], sv = cst[kTab + le];
                y1[e] = to_half(fp32_rounded(v1 * cv - v2 * sv));
                y2[e] = to_half(fp32_rounded(v2 * cv + v1 * sv));
            }
            half_t* hp = slot_ptr(p, tok0);
            st8_out<MI_WT_QKNR>(hp, y1);
            st8_out<MI_WT_QKNR>(hp + HALF, y2);
        }
    };

    int64_t g = blockIdx.x;
    if (g >= ngroups) return;  // whole workgroup: no barrier is skipped by part of it
    h8 a1[P], a2[P], b1[P], b2[P];
    int64_t pos = load_position(g);
    load_group(g, a1, a2);
    int64_t pos_next = load_position(g + stride);
    build_table(pos, cs[0]);
    // One step: prefetch group g + stride into (n1, n2) and its table into
    // cs[nb], prefetch the positions of g + 2 * stride, then process g.
    auto step = [&](int cb, const h8* c1, const h8* c2, h8* n1, h8* n2) -> bool {
        // Drain here, before the next loads are issued: with stores in
        // flight every wait on a load is a full drain, so the only wait of a
        // step must come before its prefetch, not after it.
        __builtin_amdgcn_s_waitcnt(kDrainVmem);
        const int64_t gn = g + stride;
        const bool more = gn < ngroups;
        if (more) {
            const int64_t pn = pos_next;
            pos_next = load_position(gn + stride);
            load_group(gn, n1, n2);
            build_table(pn, cs[cb ^ 1]);
        }
        __syncthreads();
        process(g, cs[cb], c1, c2);
        g = gn;
        return more;
    };
    for (;;) {
        if (!step(0, a1, a2, b1, b2)) break;
        if (!step(1, b1, b2, a1, a2)) break;
    }
}

__global__ __launch_bounds__(256) void rope_table_kernel(const int64_t* __restrict__ positions,
                                                         half_t* __restrict__ cos_t,
                                                         half_t* __restrict__ sin_t, int64_t N,
                                                         int half, InvFreq inv) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= N * half) return;
    const int64_t n = idx / half;
    const int i = static_cast<int>(idx - n * half);
    half_t hc, hs;
    cos_sin_half(static_cast<float>(positions[n]) * inv.v[i], hc, hs);
    cos_t[idx] = hc;
    sin_t[idx] = hs;
}

bool load_inv_freq(const float* host, int64_t half, InvFreq& out) {
    if (!host || half <= 0 || half > kMaxHalf) return false;
    for (int64_t i = 0; i < half; ++i) out.v[i] = host[i];
    for (int64_t i = half; i < kMaxHalf; ++i) out.v[i] = 0.0f;
    return true;
}

// Tokens per 256-lane workgroup for the one-round kernels: the fewest (1, 2,
// 4 or 8) whose units give every lane at least one, when a token has fewer
// than 256.  Measured across head layouts (28|4, 32|8, 32|32 x 128, 16|8 x
// 256, 32|4 and 8|1 x 64), this matched or beat choosing by the fill of the
// last round of resident workgroups (pick_tokens_per_wg): one token per
// workgroup whenever a token has 256 units or more.
inline int fill_tokens_per_wg(int units_per_token) {
    int tpw = 1;
    while (tpw < 8 && tpw * units_per_token < 256) tpw *= 2;
    return tpw;
}

// Tokens per workgroup for the one-round fused Q/K-norm + RoPE kernel: the
// candidate whose grid leaves the least idle tail in the GPU's last round of
// resident workgroups, with a small charge per extra round (each round
// repeats the load-latency / table / barrier ramp).  (The RoPE kernel used
// this rule until the lane-fill rule above measured as good or better there;
// under the library sincosf's residencies it once took T = 6064 from 58% to
// 68% by avoiding a second round 18% full.)
template <typename K1, typename K2, typename K4, typename K8>
int pick_tokens_per_wg(int64_t T, K1 k1, K2 k2, K4 k4, K8 k8) {
    const void* ks[4] = {reinterpret_cast<const void*>(k1), reinterpret_cast<const void*>(k2),
                         reinterpret_cast<const void*>(k4), reinterpret_cast<const void*>(k8)};
    int best = 1;
    double best_fill = -1.0;
    for (int i = 0, tpw = 1; i < 4; ++i, tpw *= 2) {
        const int64_t groups = ceil_div(T, tpw), cap = resident_workgroups(ks[i], 256);
        const double f = round_fill(groups, cap) -
                         (cap > 0 ? 0.05 * static_cast<double>(ceil_div(groups, cap) - 1) : 0.0);
        if (f > best_fill + 1e-9) {
            best_fill = f;
            best = tpw;
        }
    }
    return best;
}

template <int VEC, bool FROM_POS, bool BIAS = false>
int launch_rope_t(const half_t* q_in, half_t* q_out, int hq, const half_t* k_in, half_t* k_out,
                  int hk, const int64_t* positions, const half_t* cos_t, const half_t* sin_t,
                  int64_t T, int d, const InvFreq& inv, hipStream_t s,
                  const half_t* bq = nullptr, const half_t* bk = nullptr) {
    int tpw = fill_tokens_per_wg((hq + hk) * (d / 2 / VEC));
    // the bias form holds twice the registers per token: 8 tokens of 16-byte
    // units spill (236 bytes of scratch), 4 fit in 122 VGPRs
    if (BIAS && VEC == 8 && tpw > 4) tpw = 4;
    const int64_t grid = ceil_div(T, tpw);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (static_cast<int64_t>(tpw) * (hq + hk) * (d / 2 / VEC) >= (int64_t{1} << 22))
        return MI_ERR_UNSUPPORTED;  // units per workgroup: small_div's exact range
    const dim3 g(static_cast<unsigned>(grid)), b(256);
    switch (tpw) {
#define MI_ROPE_CASE(P)                                                                        \
    case P:                                                                                    \
        rope_kernel<VEC, FROM_POS, P, BIAS><<<g, b, 0, s>>>(q_in, q_out, hq, k_in, k_out, hk,  \
                                                            positions, cos_t, sin_t, T, d, inv, \
                                                            bq, bk);                            \
        break;
        MI_ROPE_CASE(1)
        MI_ROPE_CASE(2)
        MI_ROPE_CASE(4)
        MI_ROPE_CASE(8)
#undef MI_ROPE_CASE
        default: return MI_ERR_UNSUPPORTED;
    }
    return launch_status();
}

int launch_rope(const half_t* q_in, half_t* q_out, int64_t Hq, const half_t* k_in, half_t* k_out,
                int64_t Hkv, const int64_t* positions, const half_t* cos_t, const half_t* sin_t,
                int64_t T, int64_t hd, const InvFreq& inv, hipStream_t s,
                const half_t* bq = nullptr, const half_t* bk = nullptr) {
    const int64_t half = hd / 2;
    bool vec = (half % 8 == 0) && aligned16(q_in) && aligned16(q_out);
    if (Hkv > 0) vec = vec && aligned16(k_in) && aligned16(k_out);
    const int hq = static_cast<int>(Hq), hk = static_cast<int>(Hkv), d = static_cast<int>(hd);
    if (bq) {  // positions, in place, with the projection bias
        vec = vec && aligned16(bq) && (Hkv == 0 || aligned16(bk));
        if (vec)
            return launch_rope_t<8, true, true>(q_in, q_out, hq, k_in, k_out, hk, positions,
                                                nullptr, nullptr, T, d, inv, s, bq, bk);
        return launch_rope_t<1, true, true>(q_in, q_out, hq, k_in, k_out, hk, positions, nullptr,
                                            nullptr, T, d, inv, s, bq, bk);
    }
    if (positions) {
        if (vec)
            return launch_rope_t<8, true>(q_in, q_out, hq, k_in, k_out, hk, positions, nullptr,
                                          nullptr, T, d, inv, s);
        return launch_rope_t<1, true>(q_in, q_out, hq, k_in, k_out, hk, positions, nullptr,
                                      nullptr, T, d, inv, s);
    }
    if (vec)
        return launch_rope_t<8, false>(q_in, q_out, hq, k_in, k_out, hk, nullptr, cos_t, sin_t, T,
                                       d, inv, s);
    return launch_rope_t<1, false>(q_in, q_out, hq, k_in, k_out, hk, nullptr, cos_t, sin_t, T, d,
                                   inv, s);
}

// MI_QKN_PIPE=0 selects the one-round kernel for every shape (measurement).
#ifndef MI_QKN_PIPE
#define MI_QKN_PIPE 1
#endif

// Pipelined launch: P register slots per lane (launched with P = 1, a
// token's units in one slot), G tokens per group (as many as the slots and
// the table hold), and a grid of the resident capacity, so every workgroup stays
// resident and walks ngroups / grid groups.  Measured at T = 6064, Qwen2.5
// heads: 63% of HBM peak against 56% for the one-round kernel; two tokens
// per step (P = 2) and a grid of twice the capacity both measured lower.
template <int CPH, int P>
int launch_qk_norm_rope_pipe(half_t* q, int hq, half_t* k, int hk, const half_t* wq,
                             const half_t* wk, const int64_t* positions, int64_t T, float eps,
                             float w_bias, const InvFreq& inv, hipStream_t s) {
    constexpr int HALF = CPH * 8;
    const int upt = (hq + hk) * CPH;
    int G = (256 * P) / upt;
    if (G > 256 / HALF) G = 256 / HALF;
    const int64_t ngroups = ceil_div(T, G);
    const int64_t cap =
        resident_workgroups(reinterpret_cast<const void*>(qk_norm_rope_pipe_kernel<CPH, P>), 256);
    int64_t grid = cap > 0 ? cap : ngroups;
    if (grid > ngroups) grid = ngroups;
    if (grid > kMaxGridX) grid = kMaxGridX;
    qk_norm_rope_pipe_kernel<CPH, P><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, s>>>(
        q, hq, k, hk, wq, wk, positions, T, G, eps, w_bias, inv);
    return launch_status();
}

template <int CPH>
int launch_qk_norm_rope_t(half_t* q, int hq, half_t* k, int hk, const half_t* wq,
                          const half_t* wk, const int64_t* positions, int64_t T, float eps,
                          float w_bias, const InvFreq& inv, hipStream_t s) {
    // The pipelined kernel when a token's units fit one register slot per
    // lane (<= 256 units).  With 2 or 4 slots (P = 2, 4) its register use
    // (128 / 194 VGPRs) cost more occupancy than the pipelining gained: the
    // one-round kernel below measured 2-11 points faster for 32|8, 32|32,
    // 16|8 x 256 and 64|8 heads, so only P = 1 is launched.
    if (MI_QKN_PIPE && (hq + hk) * CPH <= 256)
        return launch_qk_norm_rope_pipe<CPH, 1>(q, hq, k, hk, wq, wk, positions, T, eps, w_bias,
                                                inv, s);
    // (the lane-fill rule of the RoPE kernel measured 2-3 points lower here)
    const int tpw = pick_tokens_per_wg(T, qk_norm_rope_kernel<CPH, 1>, qk_norm_rope_kernel<CPH, 2>,
                                       qk_norm_rope_kernel<CPH, 4>, qk_norm_rope_kernel<CPH, 8>);
    const int64_t grid = ceil_div(T, tpw);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (static_cast<int64_t>(tpw) * (hq + hk) * CPH >= (int64_t{1} << 22))
        return MI_ERR_UNSUPPORTED;  // units per workgroup: small_div's exact range
    const dim3 g(static_cast<unsigned>(grid)), b(256);
    switch (tpw) {
#define MI_QKN_CASE(P)                                                                          \
    case P:                                                                                     \
        qk_norm_rope_kernel<CPH, P><<<g, b, 0, s>>>(q, hq, k, hk, wq, wk, positions, T, eps,     \
                                                    w_bias, inv);                               \
        break;
        MI_QKN_CASE(1)
        MI_QKN_CASE(2)
        MI_QKN_CASE(4)
        MI_QKN_CASE(8)
#undef MI_QKN_CASE
        default: return MI_ERR_UNSUPPORTED;
    }
    return launch_status();
}

int launch_qk_norm_rope(half_t* q, int64_t Hq, half_t* k, int64_t Hkv, const half_t* wq,
                        const half_t* wk, const int64_t* positions, int64_t T, int64_t hd,
                        float eps, float w_bias, const InvFreq& inv, hipStream_t s) {
    const int hq = static_cast<int>(Hq), hk = static_cast<int>(Hkv);
    switch (hd) {
        case 16: return launch_qk_norm_rope_t<1>(q, hq, k, hk, wq, wk, positions, T, eps, w_bias, inv, s);
        case 32: return launch_qk_norm_rope_t<2>(q, hq, k, hk, wq, wk, positions, T, eps, w_bias, inv, s);
        case 64: return launch_qk_norm_rope_t<4>(q, hq, k, hk, wq, wk, positions, T, eps, w_bias, inv, s);
        case 128: return launch_qk_norm_rope_t<8>(q, hq, k, hk, wq, wk, positions, T, eps, w_bias, inv, s);
        case 256: return launch_qk_norm_rope_t<16>(q, hq, k, hk, wq, wk, positions, T, eps, w_bias, inv, s);
        case 512: return launch_qk_norm_rope_t<32>(q, hq, k, hk, wq, wk, positions, T, eps, w_bias, inv, s);
        default: return MI_ERR_UNSUPPORTED;
    }
}

// ---------------------------------------------------------------------------
// RoPE of Q and K in place, with K's rotated rows and V's rows also written
// into the paged KV cache, one workgroup per token: the attention
// pre-processing of a model without Q/K norm (Qwen2: with the q/k/v_proj
// bias) -- the reference's RoPE pair and two launch_paged_kv_scatter calls
// per sequence group (src/layers/attention.cpp:779-780, :823-846) in one
// launch.  K is not re-read for the scatter.  256 lanes take the (head,
// slice) units of the token as rope_kernel does, and lane j also carries V's
// 16-byte vector j (a 256-lane workgroup keeps rope_kernel's residency of
// 8 workgroups per CU; 64 extra V lanes made it 6: 0.4-0.9 us slower at
// Qwen2.5's shape, T = 6064).  Cache rows are written through to memory ("nt sc1"), as the
// scatter kernel writes them.  The token's cache slot comes from the segment
// holding it (workgroup-uniform scalar lookups issued with the data loads).
// ---------------------------------------------------------------------------
constexpr int kMaxKvSegs = 8;
struct KvSegs {
    int n;
    int64_t off[kMaxKvSegs], B[kMaxKvSegs], S[kMaxKvSegs], mb[kMaxKvSegs];
    const int* bt[kMaxKvSegs];
    const int* sl[kMaxKvSegs];
    const int* sp[kMaxKvSegs];
};

// NORM (Gemma 3): the per-head Q/K RMSNorm of qk_norm_rope_kernel first --
// the CPH = hd/16 lanes of a head sum their squares by DPP, the normalised
// value is rounded to fp16 where the reference stores it, and the rotation
// takes it from registers.  CPH = head_dim / 16 at compile time (shifts for
// the lane -> (head, slice) split: 0.3-0.4 us less than CPH = 0 at Qwen2.5's
// shapes); CPH = 0: head_dim known at run time (no norm).
// SEG = false: RoPE (+ bias or norm) alone -- no cache segment, no V, no
// cache stores (a distinct kernel in traces, with none of that code).
// `inv` is the first parameter: it sits at offset 0 of the kernel-argument
// block, which the SEG = false form reads directly (below).
template <bool BIAS, bool NORM, int CPH, bool SEG = true>
__global__ __launch_bounds__(256) void rope_kv_kernel(InvFreq inv, half_t* q, half_t* k,
                                                       const half_t* v, int Hq, int Hkv, int hd,
                                                       const int64_t* __restrict__ positions,
                                                       const half_t* __restrict__ bq,
                                                       const half_t* __restrict__ bk,
                                                       const half_t* __restrict__ bv,
                                                       const half_t* __restrict__ wq,
                                                       const half_t* __restrict__ wk, float eps,
                                                       float w_bias, half_t* k_cache,
                                                       half_t* v_cache, KvSegs sg, int64_t layer,
                                                       int64_t num_blocks, int64_t bs) {
    static_assert(!(BIAS && NORM), "no model adds a QKV bias before a Q/K norm");
    static_assert(!NORM || (CPH >= 1 && CPH <= 32), "the norm needs head_dim / 16 at compile time");
    __shared__ __attribute__((aligned(16))) float cs[2 * kMaxHalf];
    const int64_t tok = blockIdx.x;
    const int half = CPH ? CPH * 8 : hd >> 1;
    const int cph = CPH ? CPH : half >> 3;  // 16-byte slices per half head
    const int units = (Hq + Hkv) * cph;
    const int tid = threadIdx.x;

    h8 x1 = h8(0), x2 = h8(0), b1 = h8(0), b2 = h8(0);
    half_t* hp = nullptr;
    int h = 0, c = 0;
    // SEG = false: this lane's inverse frequency read from the kernel-argument
    // block ahead of the data, and the data loads straight-line (an idle lane
    // reads head 0's first slice and stores nothing), so the sincos below
    // waits for that one load only -- not, as when the compiler sinks the
    // argument load behind the data (the counter is in order), for every
    // data load first.  Q/K-norm + RoPE at T = 6064: 18.2 -> ... us.
    float inv_l = 0.0f;
    if constexpr (!SEG) {
        const float* ip =
            reinterpret_cast<const float*>(
                reinterpret_cast<uintptr_t>(__builtin_amdgcn_kernarg_segment_ptr())) +
            (tid & (kMaxHalf - 1));  // inv.v[tid] (tid < half <= kMaxHalf uses it)
        asm volatile("global_load_dword %0, %1, off" : "=v"(inv_l) : "v"(ip) : "memory");
        const bool act = tid < units;
        const int u = act ? tid : 0;
        if constexpr (CPH != 0) {
            h = u / CPH;
            c = u & (CPH - 1);
        } else {
            h = small_div(u, 1.0f / static_cast<float>(cph));  // units < 2^22: exact
            c = u - h * cph;
        }
        hp = h < Hq ? q + (tok * Hq + h) * (2 * half) : k + (tok * Hkv + (h - Hq)) * (2 * half);
        x1 = ld8_stream(hp + c * 8);
        x2 = ld8_stream(hp + half + c * 8);
        if constexpr (BIAS) {
            const half_t* bp = h < Hq ? bq + h * (2 * half) : bk + (h - Hq) * (2 * half);
            b1 = ld8(bp + c * 8);
            b2 = ld8(bp + half + c * 8);
        }
        if constexpr (NORM) {
            const half_t* wp = h < Hq ? wq : wk;
            b1 = ld8(wp + c * 8);
            b2 = ld8(wp + half + c * 8);
        }
        // the inverse frequency has landed once only the loads after it remain
        asm volatile("s_waitcnt vmcnt(%0)" : : "n"((BIAS || NORM) ? 4 : 2) : "memory");
        asm volatile("" : "+v"(inv_l));
    } else if (tid < units) {
        if constexpr (CPH != 0) {
            h = tid / CPH;
            c = tid & (CPH - 1);
        } else {
            h = small_div(tid, 1.0f / static_cast<float>(cph));  // units < 2^22: exact
            c = tid - h * cph;
        }
        hp = h < Hq ? q + (tok * Hq + h) * (2 * half) : k + (tok * Hkv + (h - Hq)) * (2 * half);
        x1 = ld8_stream(hp + c * 8);
        x2 = ld8_stream(hp + half + c * 8);
        if constexpr (BIAS) {  // a few KB every token re-reads: plain loads
            const half_t* bp = h < Hq ? bq + h * (2 * half) : bk + (h - Hq) * (2 * half);
            b1 = ld8(bp + c * 8);
            b2 = ld8(bp + half + c * 8);
        }
        if constexpr (NORM) {  // the norm weights [hd], as the biases
            const half_t* wp = h < Hq ? wq : wk;
            b1 = ld8(wp + c * 8);
            b2 = ld8(wp + half + c * 8);
        }
    }
    const int vj = tid;  // V vector of this lane (Hkv * hd / 8 <= 256)
    const bool vlane = SEG && sg.n > 0 && vj < Hkv * (half >> 2);  // no segment: V not read
    h8 vv = h8(0), vb = h8(0);
    if (vlane) {
        vv = ld8_stream(v + tok * Hkv * (2 * half) + vj * 8);
        if constexpr (BIAS) vb = ld8(bv + vj * 8);
    }
    const float fpos = static_cast<float>(positions[tok]);
    // the token's cache row (-1: not scattered), as launch_paged_kv_scatter
    // places it (src/kernels/model_utils_kernel.cu:108-164); looked up after
    // the data loads are issued, so its dependent scalar loads overlap them
    // (token indices and segment sizes fit 32 bits: T <= kMaxGridX)
    int64_t dst_base = -1;
    const int itok = static_cast<int>(tok);
    for (int i = 0; SEG && i < sg.n; ++i) {
        const int r = itok - static_cast<int>(sg.off[i]);
        const int S = static_cast<int>(sg.S[i]);
        if (r < 0 || r >= static_cast<int>(sg.B[i]) * S) continue;
        const int b = static_cast<int>(static_cast<uint32_t>(r) / static_cast<uint32_t>(S));
        const int64_t pos = static_cast<int64_t>(sg.sp[i][b]) + (r - b * S);
        const int len = sg.sl[i][b];
        if (pos < 0 || pos >= len) break;
        // 0 <= pos < len and bs < 2^31: 32-bit division
        const int blk = static_cast<int>(static_cast<uint32_t>(pos) / static_cast<uint32_t>(bs));
        if (blk >= sg.mb[i]) break;
        const int64_t phys = sg.bt[i][b * sg.mb[i] + blk];
        if (phys >= 0 && phys < num_blocks)
            dst_base = ((layer * num_blocks + phys) * Hkv * bs + (pos - blk * bs)) * (2 * half);
        break;
    }
    if (tid < half) {
        half_t hc, hs;
        cos_sin_half(fpos * (SEG ? inv.v[tid] : inv_l), hc, hs);
        const int li = quad_split(tid, half);
        cs[li] = (float)hc;
        cs[kMaxHalf + li] = (float)hs;
    }
    __syncthreads();

    float rrms = 1.0f;
    if constexpr (NORM) {  // every lane takes part in the DPP sum (idle lanes add zeros)
        float ss = pair_sumsq(x1, x2);
        ss = group_sum<CPH ? CPH : 1>(ss);
        rrms = rsqrtf(ss / static_cast<float>(CPH * 16) + eps);
    }
    if (tid < units) {
        // quad_split layout: entries 0-3 of slice c at c*4, 4-7 at half/2 + c*4
        typedef float f4 __attribute__((ext_vector_type(4)));
        const f4 c_lo = *reinterpret_cast<const f4*>(&cs[c * 4]);
        const f4 c_hi = *reinterpret_cast<const f4*>(&cs[(half >> 1) + c * 4]);
        const f4 s_lo = *reinterpret_cast<const f4*>(&cs[kMaxHalf + c * 4]);
        const f4 s_hi = *reinterpret_cast<const f4*>(&cs[kMaxHalf + (half >> 1) + c * 4]);
        h8 y1, y2;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float cv = e < 4 ? c_lo[e & 3] : c_hi[e & 3];
            const float sv = e < 4 ? s_lo[e & 3] : s_hi[e & 3];
            float a = (float)x1[e], bb = (float)x2[e];
            if constexpr (BIAS) {
                a = (float)to_half(a + (float)b1[e]);
                bb = (float)to_half(bb + (float)b2[e]);
            }
            if constexpr (NORM) {  // the normalised value as the reference stores it (fp16)
                a = (float)to_half(a * rrms * ((float)b1[e] + w_bias));
                bb = (float)to_half(bb * rrms * ((float)b2[e] + w_bias));
            }
            y1[e] = to_half(fp32_rounded(a * cv - bb * sv));
            y2[e] = to_half(fp32_rounded(bb * cv + a * sv));
        }
        st8_out<NORM ? MI_WT_QKNR : MI_WT_ROPE>(hp + c * 8, y1);
        st8_out<NORM ? MI_WT_QKNR : MI_WT_ROPE>(hp + half + c * 8, y2);
        if (SEG && h >= Hq && dst_base >= 0) {
            half_t* kd = k_cache + dst_base + static_cast<int64_t>(h - Hq) * bs * (2 * half);
            st8_stream_wt(kd + c * 8, y1);
            st8_stream_wt(kd + half + c * 8, y2);
        }
    }
    if (SEG && vlane && dst_base >= 0) {
        if constexpr (BIAS) {
#pragma unroll
            for (int e = 0; e < 8; ++e) vv[e] = to_half((float)vv[e] + (float)vb[e]);
        }
        const int per_head = half >> 2;
        int vh;
        if constexpr (CPH != 0)
            vh = vj / (CPH * 2);
        else
            vh = small_div(vj, 1.0f / static_cast<float>(per_head));
        const int vd = (vj - vh * per_head) * 8;
        st8_stream_wt(v_cache + dst_base + static_cast<int64_t>(vh) * bs * (2 * half) + vd, vv);
    }
}

// ---------------------------------------------------------------------------
// RoPE of Q and K from positions, in place, TPW tokens per 256-lane
// workgroup with the token rows walked as contiguous 16-byte vectors: lane j
// takes vectors j, j + 256, ... (R of them) of the token's [Q heads | K heads]
// row, so each wave-wide load or store covers 1 KiB of consecutive bytes and
// a workgroup's TPW tokens lie together.  A head's first-half vector s and
// second-half vector s + X (X = head_dim / 16) sit in lanes j and j ^ X of one
// wave; the partner's value comes over DPP (X = 8: row_ror:8) or a lane
// shuffle.  Every load of the workgroup is issued first, then the TPW x
// head_dim/2 cos/sin values are built once in LDS (one barrier), then every
// output is formed, then the stores go out, each waiting for the one before
// it.  On the same access pattern with no arithmetic (floors.hip,
// mi_floor_rope_inplace), 4 tokens per workgroup with paced non-temporal
// stores move 67 MB in place in 11.5 us, one token per workgroup (the
// rope_kv_kernel shape) in 12.3 us.
// The arithmetic is rope_kv_kernel's, operation for operation -- the bias add
// rounded to fp16, the Q/K norm's per-lane sum over (x1[e], x2[e]) pairs and
// its DPP sum over the X lanes of a half head (the first-half and second-half
// lanes each form the same sum), the rotation with one rounding to fp32 -- so
// the outputs equal rope_kv_kernel's bit for bit.  Only plain RoPE takes this
// kernel by default: with the bias (Qwen2's q/k_proj bias) it measured 21.1
// against 18.3 us at T = 6064, with the Q/K norm 19.7-21.0 against 18.0 us
// (MI_ROPE_ROWS_BIAS / MI_ROPE_ROWS_NORM switch them on).
#ifndef MI_ROPE_ROWS
#define MI_ROPE_ROWS 1
#endif
#ifndef MI_ROPE_ROWS_SER
#define MI_ROPE_ROWS_SER 1
#endif
#ifndef MI_ROPE_ROWS_NORM
#define MI_ROPE_ROWS_NORM 0
#endif
#ifndef MI_ROPE_ROWS_BIAS
#define MI_ROPE_ROWS_BIAS 0
#endif

// Lane j's 16-byte vector as seen by lane j ^ X (X = 4, 8, 16).
template <int X>
__device__ __forceinline__ h8 partner_vec(h8 v) {
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    u4v u = __builtin_bit_cast(u4v, v), r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (X == 8)  // row_ror:8 within a 16-lane row: lane i reads lane i ^ 8
            r[i] = static_cast<uint32_t>(
                __builtin_amdgcn_mov_dpp(static_cast<int>(u[i]), 0x128, 0xF, 0xF, false));
        else
            r[i] = static_cast<uint32_t>(__shfl_xor(static_cast<int>(u[i]), X, kWave));
    }
    return __builtin_bit_cast(h8, r);
}

// `inv` is the first kernel parameter, so it sits at offset 0 of the
// kernel-argument block (explicit arguments are laid out in order from 0).
template <bool BIAS, bool NORM, int X, int R, int TPW>
__global__ __launch_bounds__(256) void rope_rows_kernel(
    InvFreq inv, half_t* q, half_t* k, int Hq, int Hkv, int64_t T,
    const int64_t* __restrict__ positions, const half_t* __restrict__ bq, const half_t* __restrict__ bk,
    const half_t* __restrict__ wq, const half_t* __restrict__ wk, float eps, float w_bias) {
    constexpr int HALF = X * 8;  // head_dim / 2
    constexpr int HV = 2 * X;    // 16-byte vectors per head
    constexpr int HD = 2 * HALF;
    __shared__ __attribute__((aligned(16))) float cs[TPW][2][HALF];
    const int tid = threadIdx.x;
    const int qv = Hq * HV, nv = (Hq + Hkv) * HV;
    const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * TPW;

    // this lane's R vectors: Q or K, offset within the token's row, row stride
    // (the tensor picked where each address is formed, so the compiler keeps
    // global rather than flat memory instructions)
    bool inq[R], ok[R];
    int64_t stride[R];
    int col[R], sl[R], head[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int v = tid + 256 * r;
        ok[r] = v < nv;
        inq[r] = v < qv || !ok[r];  // idle lanes point at Q's row and never load or store
        const int vv = v < qv ? v : v - qv;
        stride[r] = static_cast<int64_t>(inq[r] ? Hq : Hkv) * HD;
        col[r] = ok[r] ? vv * 8 : 0;
        sl[r] = vv & (HV - 1);  // slice within the head
        head[r] = vv / HV;
    }
    auto at = [&](int r, int64_t tok) {
        return (inq[r] ? q : k) + (tok * stride[r] + col[r]);
    };
    // The token positions as scalar loads and the bias / norm-weight slices
    // (a few KB every token re-reads: plain loads) ahead of the data loads:
    // vector loads complete in issue order, so a small load issued after the
    // data would wait for all of it.
    int64_t pos[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) pos[t] = positions[tok0 + t < T ? tok0 + t : T - 1];
    h8 b1[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        b1[r] = h8(0);
        if constexpr (BIAS) b1[r] = ld8((inq[r] ? bq : bk) + (ok[r] ? head[r] * HD + sl[r] * 8 : 0));
        if constexpr (NORM) {
            b1[r] = ld8((inq[r] ? wq : wk) + sl[r] * 8);  // the own slice's weights
        }
    }
    // This lane's inverse frequencies for the cos/sin table below, read from
    // the kernel-argument block ahead of the data loads.  Vector loads
    // complete in issue order, so the wait for them below lets the TPW * R
    // data loads issued after them stay in flight.  Written as asm because
    // the compiler sinks an argument-block load to its first use, behind the
    // data loads, where its wait would be a wait for all of them.
    constexpr int NCS = (TPW * HALF + 255) / 256;
    float invv[NCS];
#pragma unroll
    for (int j = 0; j < NCS; ++j) {
        const float* ip =
            reinterpret_cast<const float*>(
                reinterpret_cast<uintptr_t>(__builtin_amdgcn_kernarg_segment_ptr())) +
            ((tid + 256 * j) & (HALF - 1));  // inv.v[...]
        asm volatile("global_load_dword %0, %1, off" : "=v"(invv[j]) : "v"(ip) : "memory");
    }
    // Every load is unconditional (idle lanes read Q's first vector, tokens
    // past T re-read the last token and are never stored), so the loads are
    // straight-line code and each later wait counts exactly the loads it needs.
    h8 x[TPW][R];
    // NORM: the weights as the rotation uses them, w + w_bias in fp32, formed
    // once (a lane's slice of the head is the same in every token)
    float wf[NORM ? R : 1][8];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int64_t tok = tok0 + t < T ? tok0 + t : T - 1;
#pragma unroll
        for (int r = 0; r < R; ++r) x[t][r] = ld8_stream(at(r, tok));
    }
    // the inverse frequencies have landed once at most the data loads issued
    // after them are outstanding
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(TPW * R) : "memory");
#pragma unroll
    for (int j = 0; j < NCS; ++j) asm volatile("" : "+v"(invv[j]));
    // the workgroup's cos/sin rows (quad_split layout)
#pragma unroll
    for (int j = 0; j < NCS; ++j) {
        const int i = tid + 256 * j;
        if (i >= TPW * HALF) break;
        const int t = i / HALF, e = i - t * HALF;
        float fp = 0.0f;
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt)
            if (tt == t) fp = static_cast<float>(pos[tt]);
        half_t hc, hs;
        cos_sin_half(fp * invv[j], hc, hs);
        const int li = quad_split(e, HALF);
        cs[t][0][li] = (float)hc;
        cs[t][1][li] = (float)hs;
    }
    __syncthreads();
    if constexpr (NORM) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int e = 0; e < 8; ++e) wf[r][e] = (float)b1[r][e] + w_bias;
        }
    }

#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int64_t tok = tok0 + t;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            h8 own = x[t][r];
            if constexpr (BIAS) {
#pragma unroll
                for (int e = 0; e < 8; ++e) own[e] = to_half((float)own[e] + (float)b1[r][e]);
            }
            h8 oth = partner_vec<X>(own);  // every lane takes part
            const bool first = (sl[r] & X) == 0;
            const int c = sl[r] & (X - 1);
            float rrms = 1.0f;
            if constexpr (NORM) {  // the sum over (x1[e], x2[e]) pairs, x1 first
                const h8 x1 = first ? own : oth, x2 = first ? oth : own;
                float ss = pair_sumsq(x1, x2);
                ss = group_sum<X>(ss);
                rrms = rsqrtf(ss / static_cast<float>(X * 16) + eps);
                // the normalised value as the reference stores it (fp16); the
                // partner's comes over the same exchange
#pragma unroll
                for (int e = 0; e < 8; ++e) own[e] = to_half((float)own[e] * rrms * wf[r][e]);
                oth = partner_vec<X>(own);
            }
            // entries 0-3 of slice c at c*4, entries 4-7 at HALF/2 + c*4 (quad_split)
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 c_lo = *reinterpret_cast<const f4*>(&cs[t][0][c * 4]);
            const f4 c_hi = *reinterpret_cast<const f4*>(&cs[t][0][(HALF >> 1) + c * 4]);
            const f4 s_lo = *reinterpret_cast<const f4*>(&cs[t][1][c * 4]);
            const f4 s_hi = *reinterpret_cast<const f4*>(&cs[t][1][(HALF >> 1) + c * 4]);
            // y = own * cos + partner * (-sin for a first-half lane, +sin for a
            // second-half one): x1*c - x2*s and x2*c + x1*s, the negation exact
            const float sgn = first ? -1.0f : 1.0f;
            h8 y;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float cv = e < 4 ? c_lo[e & 3] : c_hi[e & 3];
                const float sv = sgn * (e < 4 ? s_lo[e & 3] : s_hi[e & 3]);
                const float a = (float)own[e], bb = (float)oth[e];
                y[e] = to_half(fp32_rounded(a * cv + bb * sv));
            }
            x[t][r] = y;
        }
    }
    // every output formed, then the stores, each waiting for the one before
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
        const int64_t tok = tok0 + t;
        if (tok >= T) break;  // workgroup-uniform
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (ok[r]) {
                st8_stream(at(r, tok), x[t][r]);
                store_gap<MI_ROPE_ROWS_SER != 0>();
            }
        }
    }
}

template <bool BI, bool NO, int XX, int RR>
void rope_rows_go(int tpw, dim3 g, hipStream_t s, const InvFreq& inv, half_t* q, half_t* k,
                  int hq, int hk, int64_t T, const int64_t* positions, const half_t* bq,
                  const half_t* bk, const half_t* wq, const half_t* wk, float eps, float w_bias) {
#define MI_RR_GO(TT)                                                                            \
    rope_rows_kernel<BI, NO, XX, RR, TT><<<g, dim3(256), 0, s>>>(inv, q, k, hq, hk, T, positions, \
                                                                 bq, bk, wq, wk, eps, w_bias)
    switch (tpw) {
        case 1: MI_RR_GO(1); break;
        case 2: MI_RR_GO(2); break;
        case 4: MI_RR_GO(4); break;
        case 6: if constexpr (RR <= 2) MI_RR_GO(6); break;
        default: if constexpr (RR <= 2) MI_RR_GO(8); break;
    }
#undef MI_RR_GO
}

// Tokens per workgroup: the fewest of {1, 2, 4, 6, 8} (R <= 2; {1, 2, 4}
// for R = 3, 4) whose grid fits 4 workgroups per CU -- one resident round
// with every CU equally loaded -- else the most.  Measured at Qwen2.5's
// 28 + 4 heads of 128 (R = 2): T = 4096, 4 tokens (1024 workgroups) 11.7 us
// against 12.6 us for rope_kv_kernel's one token per workgroup; T = 6064,
// 6 tokens (1011 workgroups) 17.5 us against 17.8 us, while 4 tokens
// (1516 workgroups, an uneven round) took 20.1 us.
int rope_rows_tpw(int64_t T, int R) {
    const int64_t target = 4 * static_cast<int64_t>(device_cus() > 0 ? device_cus() : 256);
    static const int kCands[] = {1, 2, 4, 6, 8};
    const int n = R <= 2 ? 5 : 3;
    for (int i = 0; i < n; ++i)
        if (ceil_div(T, kCands[i]) <= target) return kCands[i];
    return kCands[n - 1];
}

// rope_rows_kernel for head_dim 64 / 128 / 256 and up to 1024 vectors per
// token; MI_ERR_UNSUPPORTED otherwise (the caller takes rope_kv_kernel).
int rope_qk_rows(half_t* q, half_t* k, const half_t* bq, const half_t* bk,
                 const int64_t* positions, const InvFreq& inv, int64_t T, int64_t Hq,
                 int64_t Hkv, int64_t head_dim, hipStream_t s, const half_t* wq,
                 const half_t* wk, float eps, float w_bias) {
    const bool norm = wq != nullptr;
    if (!MI_ROPE_ROWS || (norm && !MI_ROPE_ROWS_NORM) || (bq && !MI_ROPE_ROWS_BIAS))
        return MI_ERR_UNSUPPORTED;
    const int64_t nv = (Hq + Hkv) * head_dim / 8;
    if ((head_dim != 64 && head_dim != 128 && head_dim != 256) || nv > 1024 || nv < 1 ||
        !aligned16(q) || (Hkv > 0 && !aligned16(k)) || (bq && !aligned16(bq)) ||
        (bk && Hkv > 0 && !aligned16(bk)) ||
        (norm && (!aligned16(wq) || (Hkv > 0 && !aligned16(wk)))))
        return MI_ERR_UNSUPPORTED;
    const int R = static_cast<int>((nv + 255) / 256);
    const int tpw = rope_rows_tpw(T, R);
    const int64_t grid = ceil_div(T, tpw);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    const dim3 g(static_cast<unsigned>(grid));
    const int hq = static_cast<int>(Hq), hk = static_cast<int>(Hkv);
#define MI_RR_ARGS tpw, g, s, inv, q, k, hq, hk, T, positions, bq, bk, wq, wk, eps, w_bias
#define MI_RR_R(BI, NO, XX)                                    \
    switch (R) {                                               \
        case 1: rope_rows_go<BI, NO, XX, 1>(MI_RR_ARGS); break; \
        case 2: rope_rows_go<BI, NO, XX, 2>(MI_RR_ARGS); break; \
        case 3: rope_rows_go<BI, NO, XX, 3>(MI_RR_ARGS); break; \
        default: rope_rows_go<BI, NO, XX, 4>(MI_RR_ARGS);      \
    }
#define MI_RR_X(BI, NO)                     \
    switch (head_dim) {                     \
        case 64: MI_RR_R(BI, NO, 4) break;  \
        case 128: MI_RR_R(BI, NO, 8) break; \
        default: MI_RR_R(BI, NO, 16)        \
    }
    if (norm) {
#if MI_ROPE_ROWS_NORM
        MI_RR_X(false, true)
#endif
    } else if (bq) {
#if MI_ROPE_ROWS_BIAS
        MI_RR_X(true, false)
#endif
    } else {
        MI_RR_X(false, false)
    }
#undef MI_RR_X
#undef MI_RR_R
#undef MI_RR_ARGS
    return launch_status();
}

// RoPE of Q and K from positions (+ the Q/K bias, or the Q/K norm) through rope_kv_kernel
// with no segment: one token per 256-lane workgroup, head_dim's lane split at
// compile time.  Against rope_kernel at T = 6064 (plain / with the bias):
// 256 (head, slice) units per token 17.9 -> 17.6 / 19.2 -> 18.7 us (at T =
// 4096: 12.8 -> 12.5 us), 192 units 15.1 -> 13.7 / 16.2 -> 14.5, 144 units
// 13.3 -> 12.1 / 15.4 -> 13.7, 96 units 9.4 -> 9.1; below that plain RoPE is
// faster in rope_kernel, which packs several tokens per workgroup (64 units
// 7.3 against 7.6 us), while the bias form there is not (40 units 17.0
// against 7.4 us).  MI_ERR_UNSUPPORTED: the caller runs rope_kernel.
// With the Q/K norm (against qk_norm_rope_pipe_kernel, T = 6064): 256 units
// 19.5 -> 17.9 us (T = 4096: 13.8 -> 12.8, T = 64: 4.2 -> 3.1), 192 units
// 15.5 -> 14.1, 144 units 14.6 -> 13.0; 96 units 9.5 against 10.1 us, so the
// norm form takes tokens of 120 units and more.
#ifndef MI_RKV_MIN_UNITS
#define MI_RKV_MIN_UNITS 80
#endif
constexpr int64_t kRkvMinUnitsNorm = 120;
int rope_qk_one_token(half_t* q, half_t* k, const half_t* bq, const half_t* bk,
                      const int64_t* positions, const InvFreq& inv, int64_t T, int64_t Hq,
                      int64_t Hkv, int64_t head_dim, hipStream_t s,
                      const half_t* wq = nullptr, const half_t* wk = nullptr, float eps = 0.0f,
                      float w_bias = 0.0f) {
    {
        const int st = rope_qk_rows(q, k, bq, bk, positions, inv, T, Hq, Hkv, head_dim, s, wq, wk,
                                    eps, w_bias);
        if (st != MI_ERR_UNSUPPORTED) return st;
    }
    const int64_t units = (Hq + Hkv) * (head_dim / 16);
    const bool norm = wq != nullptr;
    const int64_t min_units = norm ? kRkvMinUnitsNorm : (bq ? 1 : MI_RKV_MIN_UNITS);
    if (head_dim % 16 != 0 || head_dim / 2 > kMaxHalf || units > 256 || units < min_units ||
        T > kMaxGridX || !aligned16(q) || (Hkv > 0 && !aligned16(k)) ||
        (bq && !aligned16(bq)) || (bk && Hkv > 0 && !aligned16(bk)) ||
        (norm && (!aligned16(wq) || (Hkv > 0 && !aligned16(wk)))))
        return MI_ERR_UNSUPPORTED;
    KvSegs sg{};
    sg.n = 0;
    const dim3 g(static_cast<unsigned>(T)), b(256);
    const int hq = static_cast<int>(Hq), hk = static_cast<int>(Hkv), d = static_cast<int>(head_dim);
#define MI_RQ_ARGS                                                                          \
    inv, q, k, k, hq, hk, d, positions, bq, bk, nullptr, wq, wk, eps, w_bias, nullptr, nullptr, \
        sg, 0, 0, 1
#define MI_RQ_CPH(BIAS)                                                                     \
    switch (head_dim / 16) {                                                                \
        case 1: rope_kv_kernel<BIAS, false, 1, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;   \
        case 2: rope_kv_kernel<BIAS, false, 2, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;   \
        case 4: rope_kv_kernel<BIAS, false, 4, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;   \
        case 8: rope_kv_kernel<BIAS, false, 8, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;   \
        case 16: rope_kv_kernel<BIAS, false, 16, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break; \
        case 32: rope_kv_kernel<BIAS, false, 32, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break; \
        default: rope_kv_kernel<BIAS, false, 0, false><<<g, b, 0, s>>>(MI_RQ_ARGS);         \
    }
    if (norm) {
        switch (head_dim / 16) {
            case 1: rope_kv_kernel<false, true, 1, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;
            case 2: rope_kv_kernel<false, true, 2, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;
            case 4: rope_kv_kernel<false, true, 4, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;
            case 8: rope_kv_kernel<false, true, 8, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;
            case 16: rope_kv_kernel<false, true, 16, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;
            case 32: rope_kv_kernel<false, true, 32, false><<<g, b, 0, s>>>(MI_RQ_ARGS); break;
            default: return MI_ERR_UNSUPPORTED;
        }
    } else if (bq) {
        MI_RQ_CPH(true)
    } else {
        MI_RQ_CPH(false)
    }
#undef MI_RQ_CPH
#undef MI_RQ_ARGS
    return launch_status();
}

// (Hq + Hkv) * hd/2 must fit the int lane arithmetic of rope_kernel.
bool heads_ok(int64_t Hq, int64_t Hkv, int64_t hd) {
    return Hq >= 0 && Hkv >= 0 && hd > 0 && hd % 2 == 0 && hd / 2 <= kMaxHalf &&
           (Hq + Hkv) * hd < (int64_t{1} << 30);
}

}  // namespace
}  // namespace mi

using mi::half_t;

extern "C" int mi_rope_neox_f16(const void* x, const void* cos_t, const void* sin_t, void* y,
                                int64_t B, int64_t S, int64_t H, int64_t D, void* stream) {
    if (B < 0 || S < 0 || H < 0 || D < 0) return MI_ERR_INVALID_ARGUMENT;
    if (!mi::product_fits({B, S, H, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t T = B * S;
    if (T == 0 || H == 0) return MI_OK;
    if (!x || !y || !cos_t || !sin_t) return MI_ERR_INVALID_ARGUMENT;
    if (!mi::heads_ok(H, 0, D)) return MI_ERR_UNSUPPORTED;
    const int64_t bytes = T * H * D * 2;
    if (x != y && mi::overlaps(x, bytes, y, bytes)) return MI_ERR_ALIASING;
    mi::InvFreq unused{};
    return mi::launch_rope(static_cast<const half_t*>(x), static_cast<half_t*>(y), H, nullptr,
                           nullptr, 0, nullptr, static_cast<const half_t*>(cos_t),
                           static_cast<const half_t*>(sin_t), T, D, unused,
                           mi::as_stream(stream));
}

extern "C" int mi_rope_tables_f16(const float* inv_freq_host, const int64_t* positions,
                                  void* cos_t, void* sin_t, int64_t N, int64_t half,
                                  void* stream) {
    if (N < 0 || half < 0) return MI_ERR_INVALID_ARGUMENT;
    if (N == 0 || half == 0) return MI_OK;
    if (!positions || !cos_t || !sin_t) return MI_ERR_INVALID_ARGUMENT;
    mi::InvFreq inv;
    if (!mi::load_inv_freq(inv_freq_host, half, inv)) return MI_ERR_INVALID_ARGUMENT;
    if (!mi::product_fits({N, half, 4})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t total = N * half;
    const int64_t grid = mi::ceil_div(total, 256);
    if (grid > mi::kMaxGridX) return MI_ERR_UNSUPPORTED;
    const int64_t bytes = total * 2;
    if (mi::overlaps(cos_t, bytes, sin_t, bytes)) return MI_ERR_ALIASING;
    mi::rope_table_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                            mi::as_stream(stream)>>>(positions, static_cast<half_t*>(cos_t),
                                                     static_cast<half_t*>(sin_t), N,
                                                     static_cast<int>(half), inv);
    return mi::launch_status();
}

extern "C" int mi_rope_neox_qk_f16(void* q, void* k, const int64_t* positions,
                                   const float* inv_freq_host, int64_t T, int64_t Hq,
                                   int64_t Hkv, int64_t head_dim, void* stream) {
    if (T < 0 || Hq < 0 || Hkv < 0 || head_dim < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || Hq + Hkv == 0) return MI_OK;
    if (!positions || (Hq > 0 && !q) || (Hkv > 0 && !k)) return MI_ERR_INVALID_ARGUMENT;
    if (!mi::heads_ok(Hq, Hkv, head_dim)) return MI_ERR_UNSUPPORTED;
    if (!mi::product_fits({T, Hq + Hkv, head_dim, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (Hq > 0 && Hkv > 0 &&
        mi::overlaps(q, T * Hq * head_dim * 2, k, T * Hkv * head_dim * 2))
        return MI_ERR_ALIASING;
    mi::InvFreq inv;
    if (!mi::load_inv_freq(inv_freq_host, head_dim / 2, inv)) return MI_ERR_INVALID_ARGUMENT;
    // With no Q heads, run K through the Q slot (the kernel has one code path).
    if (Hq == 0) {
        q = k;
        Hq = Hkv;
        k = nullptr;
        Hkv = 0;
    }
    const int st = mi::rope_qk_one_token(static_cast<half_t*>(q), static_cast<half_t*>(k),
                                         nullptr, nullptr, positions, inv, T, Hq, Hkv, head_dim,
                                         mi::as_stream(stream));
    if (st != MI_ERR_UNSUPPORTED) return st;
    return mi::launch_rope(static_cast<const half_t*>(q), static_cast<half_t*>(q), Hq,
                           static_cast<const half_t*>(k), static_cast<half_t*>(k), Hkv,
                           positions, nullptr, nullptr, T, head_dim, inv,
                           mi::as_stream(stream));
}

extern "C" int mi_bias_rope_neox_qk_f16(void* q, void* k, const void* q_bias, const void* k_bias,
                                        const int64_t* positions, const float* inv_freq_host,
                                        int64_t T, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                        void* stream) {
    if (T < 0 || Hq < 0 || Hkv < 0 || head_dim < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || Hq + Hkv == 0) return MI_OK;
    if (!positions || (Hq > 0 && (!q || !q_bias)) || (Hkv > 0 && (!k || !k_bias)))
        return MI_ERR_INVALID_ARGUMENT;
    if (!mi::heads_ok(Hq, Hkv, head_dim)) return MI_ERR_UNSUPPORTED;
    if (!mi::product_fits({T, Hq + Hkv, head_dim, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t qb = T * Hq * head_dim * 2, kb = T * Hkv * head_dim * 2;
    if (Hq > 0 && Hkv > 0 && mi::overlaps(q, qb, k, kb)) return MI_ERR_ALIASING;
    if ((Hq > 0 && (mi::overlaps(q_bias, Hq * head_dim * 2, q, qb) ||
                    (Hkv > 0 && mi::overlaps(q_bias, Hq * head_dim * 2, k, kb)))) ||
        (Hkv > 0 && (mi::overlaps(k_bias, Hkv * head_dim * 2, k, kb) ||
                     (Hq > 0 && mi::overlaps(k_bias, Hkv * head_dim * 2, q, qb)))))
        return MI_ERR_ALIASING;
    mi::InvFreq inv;
    if (!mi::load_inv_freq(inv_freq_host, head_dim / 2, inv)) return MI_ERR_INVALID_ARGUMENT;
    // With no Q heads, run K through the Q slot (the kernel has one code path).
    if (Hq == 0) {
        q = k;
        q_bias = k_bias;
        Hq = Hkv;
        k = nullptr;
        k_bias = nullptr;
        Hkv = 0;
    }
    const int st = mi::rope_qk_one_token(
        static_cast<half_t*>(q), static_cast<half_t*>(k), static_cast<const half_t*>(q_bias),
        static_cast<const half_t*>(k_bias), positions, inv, T, Hq, Hkv, head_dim,
        mi::as_stream(stream));
    if (st != MI_ERR_UNSUPPORTED) return st;
    return mi::launch_rope(static_cast<const half_t*>(q), static_cast<half_t*>(q), Hq,
                           static_cast<const half_t*>(k), static_cast<half_t*>(k), Hkv,
                           positions, nullptr, nullptr, T, head_dim, inv, mi::as_stream(stream),
                           static_cast<const half_t*>(q_bias), static_cast<const half_t*>(k_bias));
}

namespace mi {
namespace {

// Shared checks and launch of rope_kv_kernel.  q_bias / k_bias / v_bias (all
// or none) and q_weight / k_weight (NORM) exclude each other.
int rope_kv_launch(void* q, void* k, const void* v, const void* q_bias, const void* k_bias,
                   const void* v_bias, const void* q_weight, const void* k_weight, float eps,
                   int add_one, const int64_t* positions, const float* inv_freq_host, int64_t T,
                   int64_t Hq, int64_t Hkv, int64_t head_dim, void* k_cache, void* v_cache,
                   int64_t layer, int64_t num_blocks, int64_t block_size,
                   const mi_kv_segment* segments, int num_segments, void* stream) {
    if (T < 0 || Hq < 0 || Hkv < 0 || head_dim < 0 || layer < 0 || layer >= (int64_t{1} << 62) ||
        num_blocks < 0 || block_size <= 0 || num_segments < 0)
        return MI_ERR_INVALID_ARGUMENT;
    if (T == 0) return MI_OK;
    const bool bias = q_bias || k_bias || v_bias;
    const bool norm = q_weight || k_weight;
    if (!q || !k || !v || !positions || !k_cache || !v_cache || Hq < 1 || Hkv < 1 ||
        (num_segments > 0 && !segments) || (bias && (!q_bias || !k_bias || !v_bias)) ||
        (norm && (!q_weight || !k_weight)) || (bias && norm))
        return MI_ERR_INVALID_ARGUMENT;
    // one 256-lane workgroup per token: its Q/K slices and V's vectors one
    // per lane (both <= 256), 16-byte vectors, few segments
    if (head_dim % 16 != 0 || head_dim / 2 > kMaxHalf || (Hq + Hkv) * (head_dim / 16) > 256 ||
        Hkv * head_dim / 8 > 256 || num_segments > kMaxKvSegs || T > kMaxGridX ||
        block_size > INT32_MAX)
        return MI_ERR_UNSUPPORTED;
    for (const void* p : {static_cast<const void*>(q), static_cast<const void*>(k), v,
                          static_cast<const void*>(k_cache), static_cast<const void*>(v_cache)})
        if (!aligned16(p)) return MI_ERR_UNSUPPORTED;
    if (bias && !(aligned16(q_bias) && aligned16(k_bias) && aligned16(v_bias)))
        return MI_ERR_UNSUPPORTED;
    if (norm && !(aligned16(q_weight) && aligned16(k_weight))) return MI_ERR_UNSUPPORTED;
    if (!product_fits({layer + 1, num_blocks, Hkv, block_size, head_dim, 2}))
        return MI_ERR_INVALID_ARGUMENT;
    const int64_t qb = T * Hq * head_dim * 2, kb = T * Hkv * head_dim * 2;
    const int64_t cb = (layer + 1) * num_blocks * Hkv * block_size * head_dim * 2;
    const void* bufs[5] = {q, k, v, k_cache, v_cache};
    const int64_t lens[5] = {qb, kb, kb, cb, cb};
    for (int i = 0; i < 5; ++i)
        for (int j = i + 1; j < 5; ++j)
            if (overlaps(bufs[i], lens[i], bufs[j], lens[j])) return MI_ERR_ALIASING;
    KvSegs sg{};
    sg.n = num_segments;
    for (int i = 0; i < num_segments; ++i) {
        const mi_kv_segment& g = segments[i];
        // B and S bounded before their product is formed
        if (g.token_offset < 0 || g.token_offset > T || g.B < 0 || g.S < 0 ||
            (g.B > 0 && g.S > 0 && (g.B > T || g.S > T || g.B * g.S > T - g.token_offset)))
            return MI_ERR_INVALID_ARGUMENT;
        if (g.B * g.S > 0 && (!g.block_table || !g.seq_len || !g.start_pos ||
                              g.max_blocks_per_seq <= 0))
            return MI_ERR_INVALID_ARGUMENT;
        // disjoint token ranges: the kernel scatters a token through the first
        // segment holding it, where separate scatters would write it once per
        // segment
        for (int j = 0; j < i && g.B * g.S > 0; ++j) {
            const mi_kv_segment& o = segments[j];
            if (o.B * o.S > 0 && g.token_offset < o.token_offset + o.B * o.S &&
                o.token_offset < g.token_offset + g.B * g.S)
                return MI_ERR_UNSUPPORTED;
        }
        sg.off[i] = g.token_offset;
        sg.B[i] = g.B;
        sg.S[i] = g.S;
        sg.mb[i] = g.max_blocks_per_seq;
        sg.bt[i] = g.block_table;
        sg.sl[i] = g.seq_len;
        sg.sp[i] = g.start_pos;
    }
    InvFreq inv;
    if (!load_inv_freq(inv_freq_host, head_dim / 2, inv)) return MI_ERR_INVALID_ARGUMENT;
    const dim3 g(static_cast<unsigned>(T)), b(256);
    auto* qh = static_cast<half_t*>(q);
    auto* kh = static_cast<half_t*>(k);
    const auto* vh = static_cast<const half_t*>(v);
    const auto* bqh = static_cast<const half_t*>(q_bias);
    const auto* bkh = static_cast<const half_t*>(k_bias);
    const auto* bvh = static_cast<const half_t*>(v_bias);
    const auto* wqh = static_cast<const half_t*>(q_weight);
    const auto* wkh = static_cast<const half_t*>(k_weight);
    auto* kc = static_cast<half_t*>(k_cache);
    auto* vc = static_cast<half_t*>(v_cache);
    const hipStream_t s = as_stream(stream);
    const int hq = static_cast<int>(Hq), hk = static_cast<int>(Hkv), d = static_cast<int>(head_dim);
    const float wb = add_one ? 1.0f : -0.0f;  // w + (-0) == w, also for w = -0
#define MI_RKV_ARGS                                                                           \
    inv, qh, kh, vh, hq, hk, d, positions, bqh, bkh, bvh, wqh, wkh, eps, wb, kc, vc, sg, layer, \
        num_blocks, block_size
#define MI_RKV_CPH(BIAS, NORM)                                                            \
    switch (head_dim / 16) {                                                              \
        case 1: rope_kv_kernel<BIAS, NORM, 1><<<g, b, 0, s>>>(MI_RKV_ARGS); break;       \
        case 2: rope_kv_kernel<BIAS, NORM, 2><<<g, b, 0, s>>>(MI_RKV_ARGS); break;       \
        case 4: rope_kv_kernel<BIAS, NORM, 4><<<g, b, 0, s>>>(MI_RKV_ARGS); break;       \
        case 8: rope_kv_kernel<BIAS, NORM, 8><<<g, b, 0, s>>>(MI_RKV_ARGS); break;       \
        case 16: rope_kv_kernel<BIAS, NORM, 16><<<g, b, 0, s>>>(MI_RKV_ARGS); break;     \
        case 32: rope_kv_kernel<BIAS, NORM, 32><<<g, b, 0, s>>>(MI_RKV_ARGS); break;     \
        default:                                                                          \
            if (NORM) return MI_ERR_UNSUPPORTED; /* head_dim not 16 * 2^k */             \
            rope_kv_kernel<BIAS, false, 0><<<g, b, 0, s>>>(MI_RKV_ARGS);                 \
    }
    if (norm) {
        MI_RKV_CPH(false, true)
    } else if (bias) {
        MI_RKV_CPH(true, false)
    } else {
        MI_RKV_CPH(false, false)
    }
#undef MI_RKV_CPH
#undef MI_RKV_ARGS
    return launch_status();
}

}  // namespace
}  // namespace mi

extern "C" int mi_rope_kv_scatter_f16(void* q, void* k, const void* v, const void* q_bias,
                                      const void* k_bias, const void* v_bias,
                                      const int64_t* positions, const float* inv_freq_host,
                                      int64_t T, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                      void* k_cache, void* v_cache, int64_t layer,
                                      int64_t num_blocks, int64_t block_size,
                                      const mi_kv_segment* segments, int num_segments,
                                      void* stream) {
    return mi::rope_kv_launch(q, k, v, q_bias, k_bias, v_bias, nullptr, nullptr, 0.0f, 0,
                              positions, inv_freq_host, T, Hq, Hkv, head_dim, k_cache, v_cache,
                              layer, num_blocks, block_size, segments, num_segments, stream);
}

extern "C" int mi_qk_norm_rope_kv_scatter_f16(void* q, void* k, const void* v,
                                              const void* q_weight, const void* k_weight,
                                              const int64_t* positions,
                                              const float* inv_freq_host, int64_t T, int64_t Hq,
                                              int64_t Hkv, int64_t head_dim, float eps,
                                              int add_one, void* k_cache, void* v_cache,
                                              int64_t layer, int64_t num_blocks,
                                              int64_t block_size, const mi_kv_segment* segments,
                                              int num_segments, void* stream) {
    if (!q_weight || !k_weight) return MI_ERR_INVALID_ARGUMENT;
    return mi::rope_kv_launch(q, k, v, nullptr, nullptr, nullptr, q_weight, k_weight, eps,
                              add_one, positions, inv_freq_host, T, Hq, Hkv, head_dim, k_cache,
                              v_cache, layer, num_blocks, block_size, segments, num_segments,
                              stream);
}

extern "C" int mi_qk_norm_rope_f16(void* q, void* k, const void* q_weight, const void* k_weight,
                                   const int64_t* positions, const float* inv_freq_host,
                                   int64_t T, int64_t Hq, int64_t Hkv, int64_t head_dim,
                                   float eps, int add_one, void* stream) {
    if (T < 0 || Hq < 0 || Hkv < 0 || head_dim < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || Hq + Hkv == 0) return MI_OK;
    if (!positions || (Hq > 0 && (!q || !q_weight)) || (Hkv > 0 && (!k || !k_weight)))
        return MI_ERR_INVALID_ARGUMENT;
    if (!mi::heads_ok(Hq, Hkv, head_dim)) return MI_ERR_UNSUPPORTED;
    if (!mi::product_fits({T, Hq + Hkv, head_dim, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (Hq > 0 && Hkv > 0 &&
        mi::overlaps(q, T * Hq * head_dim * 2, k, T * Hkv * head_dim * 2))
        return MI_ERR_ALIASING;
    mi::InvFreq inv;
    if (!mi::load_inv_freq(inv_freq_host, head_dim / 2, inv)) return MI_ERR_INVALID_ARGUMENT;
    const bool aligned = (Hq == 0 || (mi::aligned16(q) && mi::aligned16(q_weight))) &&
                         (Hkv == 0 || (mi::aligned16(k) && mi::aligned16(k_weight)));
    if (!aligned) return MI_ERR_UNSUPPORTED;
    // With no Q heads, run K through the Q slot (the kernel has one code path).
    if (Hq == 0) {
        q = k;
        q_weight = k_weight;
        Hq = Hkv;
        k = nullptr;
        k_weight = nullptr;
        Hkv = 0;
    }
    {
        const int st = mi::rope_qk_one_token(
            static_cast<half_t*>(q), static_cast<half_t*>(k), nullptr, nullptr, positions, inv,
            T, Hq, Hkv, head_dim, mi::as_stream(stream), static_cast<const half_t*>(q_weight),
            static_cast<const half_t*>(k_weight), eps, add_one ? 1.0f : -0.0f);
        if (st != MI_ERR_UNSUPPORTED) return st;
    }
    return mi::launch_qk_norm_rope(static_cast<half_t*>(q), Hq, static_cast<half_t*>(k), Hkv,
                                   static_cast<const half_t*>(q_weight),
                                   static_cast<const half_t*>(k_weight), positions, T, head_dim,
                                   eps, add_one ? 1.0f : -0.0f, inv, mi::as_stream(stream));
}
