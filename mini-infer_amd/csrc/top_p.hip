// top_p.hip -- nucleus (top-p) sampling with the reference's semantics
// (src/kernels/sampling_kernel.cu:86-221, launch_top_p_sample):
//   * a row longer than 30000 logits is sampled greedily: the argmax of
//     mi_greedy_argmax_f16, with the reference's tie order (its launcher
//     falls back to launch_greedy_sample there, :214-218) -- Qwen2.5's 152064
//     logits take this path;
//   * otherwise, with probabilities q_i = exp(x_i / T - max) / sum over the
//     row, the candidates are the logits at indices 0, 128, 256, ... (the
//     reference selects its top-K slots from the strided share of its first
//     thread, :130-145), ordered by q descending (equal q: lower index
//     first).  Walking them in that order, at the first position i whose
//     running fp32 sum of q reaches p, a slot in [0, i] is drawn from a 64-bit
//     finaliser of seed ^ (index << 32) and that slot's index is returned
//     (:171-186).  If the sum never reaches p the result is -1 (the
//     reference returns its last top-K slot, which is empty: fewer than 256
//     candidates exist below 30001 logits).
// The batched form applies the single-row rule to every row, row b with seed
// + b; the reference's batched launcher is an empty stub (:223-227) that
// writes nothing.
//
// One 1024-lane workgroup per row (<= 30000 logits, read once into
// registers; latency-bound).  Finite logits and temperature > 0
// are assumed, as in the reference.
#include <math.h>

#include "mi_device.h"
#include "mi_host.h"

namespace mi {
namespace {

constexpr int64_t kTopPMaxVocab = 30000;  // above: greedy
constexpr int kTopPStride = 128;          // candidate indices are multiples of 128
constexpr int kTopPMaxCand = static_cast<int>((kTopPMaxVocab + kTopPStride - 1) / kTopPStride);
static_assert(kTopPMaxCand <= 256, "candidate slots");

// MurmurHash3's 64-bit finaliser (fmix64), the reference's slot hash.
__device__ __forceinline__ uint64_t fmix64(uint64_t s) {
    s ^= s >> 33;
    s *= 0xff51afd7ed558ccdull;
    s ^= s >> 33;
    s *= 0xc4ceb9fe1a85ec53ull;
    s ^= s >> 33;
    return s;
}

// One workgroup of 1024 lanes per row; lane t loads the 16-byte vectors t,
// t + 1024, ... of the row's 16-byte-aligned window (4 per lane cover 30000
// logits at any 2-byte alignment), all issued at once and kept in registers.
// The window's bytes outside the row share 16-byte granules with the row's
// own, so they never reach another page; they are masked to -inf.
constexpr int kTopPLanes = 1024;
constexpr int kTopPVecs = 4;  // vectors per lane
static_assert(kTopPLanes * kTopPVecs * 8 >= kTopPMaxVocab + 7, "a row must fit the registers");
constexpr int kTopPRankParts = kTopPLanes / 256;  // lanes that rank one candidate
constexpr int kTopPKeys = 256;                    // key slots (>= candidates)
static_assert(kTopPKeys / kTopPRankParts % 2 == 0, "rank slices are whole 16-byte reads");
constexpr int kTopPBatch = 32;  // walk: values per batch of LDS reads
// From this many candidates on, the walk's answer comes from a parallel
// prefix where it can (~0.45 us, against ~5 ns per candidate for the walk).
constexpr int kTopPPrefixMin = 96;

// The reference's running fp32 sum over q (walk order, zero past the nc
// candidates), in order: the first position whose sum reaches p, or -1.
// q >= 0, so the sum never decreases: only a batch's last sum is tested, and
// in the batch that reaches p the first position that does is the count of
// its sums that do not (a test per value costs a vector-to-scalar round trip
// each).  The zeros past the candidates leave the sum as it is, so the sum of
// the whole walk decides whether p is reached.
__device__ __forceinline__ int walk_fp32(const float* sorted_q, int nc, float p) {
    int hit = -1;
    float cum = 0.0f;
    const float4* q4 = reinterpret_cast<const float4*>(sorted_q);
    for (int base = 0; base < nc; base += kTopPBatch) {
        float4 t[kTopPBatch / 4];
#pragma unroll
        for (int k = 0; k < kTopPBatch / 4; ++k) t[k] = q4[base / 4 + k];
        float c[kTopPBatch];
#pragma unroll
        for (int k = 0; k < kTopPBatch / 4; ++k) {
            c[4 * k] = cum += t[k].x;
            c[4 * k + 1] = cum += t[k].y;
            c[4 * k + 2] = cum += t[k].z;
            c[4 * k + 3] = cum += t[k].w;
        }
        if (cum >= p) {
            int below = 0;
#pragma unroll
            for (int k = 0; k < kTopPBatch; ++k) below += c[k] >= p ? 0 : 1;
            hit = base + below < nc ? base + below : -1;
            break;
        }
    }
    return hit;
}

// The slot draw at walk position `hit` (>= 0): a slot in [0, hit] from fmix64
// of (seed + row) ^ (index << 32), its index to out[row]; -1 when hit < 0.
__device__ __forceinline__ void top_p_draw(const int* sorted_i, int hit,
                                           uint64_t seed, int64_t row, int32_t* out) {
    int choice = -1;
    if (hit >= 0) {
        // row b draws with seed + b (a single row: seed itself)
        const uint64_t rs = seed + static_cast<uint64_t>(row);
        const uint64_t h =
            fmix64(rs ^ (static_cast<uint64_t>(static_cast<int64_t>(sorted_i[hit])) << 32));
        const float u = static_cast<float>(h & 0xFFFFFFu) / 16777216.0f;
        int slot = static_cast<int>(u * static_cast<float>(hit + 1));
        slot = slot < 0 ? 0 : (slot > hit ? hit : slot);
        choice = sorted_i[slot];
    }
    out[row] = choice;
}

__global__ __launch_bounds__(kTopPLanes) void top_p_small_kernel(const half_t* __restrict__ logits,
                                                                 int vocab, float p,
                                                                 float temperature, uint64_t seed,
                                                                 int32_t* out) {
    __shared__ float wave_m[kTopPLanes / kWave], wave_s[kTopPLanes / kWave];
    // (q bits << 32) | (255 - c): larger key = earlier in the walk order
    __shared__ __attribute__((aligned(16))) uint64_t keys[kTopPKeys];
    __shared__ int partial[kTopPRankParts][256];
    // q in walk order, zero past the candidates
    __shared__ __attribute__((aligned(16))) float sorted_q[kTopPKeys];
    __shared__ int sorted_i[kTopPKeys];
    const int64_t row = blockIdx.x;
    const half_t* x = logits + row * vocab;
    const int tid = threadIdx.x;
    const int nc = (vocab + kTopPStride - 1) / kTopPStride;
    const float rT = 1.0f / temperature;

    // element e of the row sits at window position e + shift
    const int shift = static_cast<int>((reinterpret_cast<uintptr_t>(x) & 15) >> 1);
    const half_t* xa = x - shift;
    h8 v[kTopPVecs];
#pragma unroll
    for (int j = 0; j < kTopPVecs; ++j) {
        const int e0 = (tid + j * kTopPLanes) * 8 - shift;
        v[j] = e0 < vocab ? ld8_stream(xa + e0 + shift) : h8(-__builtin_huge_valf16());
    }
    // lane c < nc also reads candidate c (index c * 128) itself, with the
    // row's loads: it forms that candidate's probability below
    const float xc = tid < nc ? (float)x[tid * kTopPStride] : 0.0f;
    // elements outside the row (only the vectors at its two ends hold any)
    // become -inf; the lane's maximum over its valid logits in fp16 pairs
    // (exact).  x / T, correctly rounded, is monotone in x, so max(x) / T is
    // the maximum of x / T.
    h2 pm = h2(-__builtin_huge_valf16());
#pragma unroll
    for (int j = 0; j < kTopPVecs; ++j) {
        const int e0 = (tid + j * kTopPLanes) * 8 - shift;
        if (e0 < 0 || e0 + 8 > vocab) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (e0 + k < 0 || e0 + k >= vocab) v[j][k] = -__builtin_huge_valf16();
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            pm = __builtin_elementwise_max(pm, h2{v[j][2 * k], v[j][2 * k + 1]});
    }
    const float m = fmaxf((float)pm[0], (float)pm[1]);
    // the normaliser, merged as (max, sum) pairs: per lane with its own
    // maximum, per wave, then across the 16 waves after one barrier.  Each
    // term is exp2(x (log2(e) / T) - max log2(e)), one fma (within a few ulps
    // of exp(x / T - max) at moderate logits); the candidates' own q below
    // use the division.
    const float ml = m / temperature;  // -inf for a lane past the row
    float s = 0.0f;
    if (ml != -INFINITY) {
        const float c1 = rT * 1.4426950408889634f, c0 = ml * 1.4426950408889634f;
#pragma unroll
        for (int j = 0; j < kTopPVecs; ++j)
#pragma unroll
            for (int k = 0; k < 8; ++k)
                s += __builtin_amdgcn_exp2f(fmaf((float)v[j][k], c1, -c0));  // -inf -> 0
    }
    {
        const float mw = group_max<kWave>(ml);
        float part = ml == -INFINITY ? 0.0f : s * fast_exp(ml - mw);
        part = group_sum<kWave>(part);
        if ((tid & (kWave - 1)) == 0) {
            wave_m[tid / kWave] = mw;
            wave_s[tid / kWave] = part;
        }
    }
    __syncthreads();
    // the first 256 lanes (the candidates' probabilities and keys) fold the
    // wave pairs; the other waves wait at the next barrier
    float qc = 0.0f;
    if (tid < kTopPKeys) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kTopPLanes / kWave; ++w) M = fmaxf(M, wave_m[w]);
        float S = 0.0f;
#pragma unroll
        for (int w = 0; w < kTopPLanes / kWave; ++w)
            S += wave_m[w] == -INFINITY ? 0.0f : wave_s[w] * fast_exp(wave_m[w] - M);
        if (tid < nc) qc = fast_exp(xc / temperature - M) / S;
        // q >= 0: its bits order as unsigned integers
        keys[tid] = (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, qc)) << 32) |
                    static_cast<uint32_t>(kTopPKeys - 1 - tid);
    }
    __syncthreads();
    // rank by (q descending, index ascending), the order the reference's
    // strict-greater selection produces: four lanes per candidate, each
    // counting the larger keys in a quarter of the slots, two keys per read.
    // Slots past the candidates hold q = 0 with a larger index, below every
    // candidate's key.
    {
        const int c = tid & 255, part = tid >> 8;
        int r = 0;
        if (c < nc) {
            const uint64_t kc = keys[c];
            constexpr int kSlice = kTopPKeys / kTopPRankParts;  // 64
            const ulonglong2* k2 = reinterpret_cast<const ulonglong2*>(keys + part * kSlice);
#pragma unroll
            for (int i = 0; i < kSlice / 2; ++i) {
                const ulonglong2 t = k2[i];
                r += (t.x > kc ? 1 : 0) + (t.y > kc ? 1 : 0);
            }
        }
        partial[part][c] = r;
    }
    __syncthreads();
    if (tid < nc) {
        int rank = 0;
#pragma unroll
        for (int k = 0; k < kTopPRankParts; ++k) rank += partial[k][tid];
        sorted_q[rank] = qc;
        sorted_i[rank] = tid * kTopPStride;
    } else if (tid < kTopPKeys) {
        sorted_q[tid] = 0.0f;
    }
    __syncthreads();
    if (nc < kTopPPrefixMin) {  // workgroup-uniform
        if (tid == 0) top_p_draw(sorted_i, walk_fp32(sorted_q, nc, p), seed, row, out);
    } else if (tid < kWave) {
        // The reference's answer is the first position whose running fp32 sum
        // (in walk order) reaches p.  Wave 0 decides it from an exact-order-
        // free double prefix P_i where it can: with every q >= 0, the fp32
        // sum after i + 1 terms is within gamma_i * S_i of the exact S_i
        // (gamma_i = i u / (1 - i u), u = 2^-24; Higham, Accuracy and
        // Stability of Numerical Algorithms, 4.2), and P_i is within ~2^-45
        // S_i of S_i, so B_i = P_i ((i + 1) u 1.004 + 1e-12) bounds their
        // gap.  Positions with P_i + B_i < p certainly stay below p; if the
        // first other one has P_i - B_i >= p it is the answer, otherwise
        // (p within B_i of the sum there) lane 0 runs the fp32 sum in order.
        const int l = tid;
        const float4 t = reinterpret_cast<const float4*>(sorted_q)[l];  // positions 4l..4l+3
        double a[4];
        a[0] = t.x;
        a[1] = a[0] + t.y;
        a[2] = a[1] + t.z;
        a[3] = a[2] + t.w;
        double incl = a[3];
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const double y = __shfl_up(incl, d, kWave);
            if (l >= d) incl += y;
        }
        double base = __shfl_up(incl, 1, kWave);
        if (l == 0) base = 0.0;
        const double pd = p;
        unsigned not_below = 0, above = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = 4 * l + k;
            const double P = base + a[k];
            const double B = P * ((i + 1) * 0x1.01p-24 + 1e-12);
            if (i < nc && !(P + B < pd)) not_below |= 1u << k;
            if (P - B >= pd) above |= 1u << k;
        }
        const uint64_t lanes = __ballot(not_below != 0);
        int hit = -1;
        bool decided = true;
        if (lanes != 0) {
            const int fl = __builtin_ctzll(lanes);
            const unsigned nb = __shfl(not_below, fl, kWave), ab = __shfl(above, fl, kWave);
            const int k = __builtin_ctz(nb);
            hit = 4 * fl + k;
            decided = (ab >> k) & 1u;
        }
        if (tid == 0 && !decided)
            hit = walk_fp32(sorted_q, nc, p);
        if (tid == 0) top_p_draw(sorted_i, hit, seed, row, out);
    }
}

int top_p(const void* logits, int64_t B, int64_t vocab, float p, float temperature,
          uint64_t seed, int32_t* out, void* stream) {
    if (B < 0 || vocab < 0) return MI_ERR_INVALID_ARGUMENT;
    if (B == 0) return MI_OK;
    if (!out || (vocab > 0 && !logits)) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({B, vocab, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(logits) & 1) return MI_ERR_INVALID_ARGUMENT;  // fp16 alignment
    if (vocab > kTopPMaxVocab) return mi_greedy_argmax_f16(logits, B, vocab, out, stream);
    if (B > kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (overlaps(out, B * 4, logits, B * vocab * 2)) return MI_ERR_ALIASING;
    top_p_small_kernel<<<dim3(static_cast<unsigned>(B)), dim3(kTopPLanes), 0,
                         as_stream(stream)>>>(
        static_cast<const half_t*>(logits), static_cast<int>(vocab), p, temperature, seed, out);
    return launch_status();
}

}  // namespace
}  // namespace mi

extern "C" int mi_top_p_sample_f16(const void* logits, int64_t vocab, float p, float temperature,
                                   uint64_t seed, int32_t* out, void* stream) {
    return mi::top_p(logits, 1, vocab, p, temperature, seed, out, stream);
}

extern "C" int mi_top_p_sample_batched_f16(const void* logits, int64_t B, int64_t vocab, float p,
                                           float temperature, uint64_t seed, int32_t* out,
                                           void* stream) {
    return mi::top_p(logits, B, vocab, p, temperature, seed, out, stream);
}
