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
constexpr int kTopPWalk = (kTopPMaxCand + 15) / 16 * 16;  // 240

// MurmurHash3's 64-bit finaliser (fmix64), the reference's slot hash.
__device__ __forceinline__ uint64_t fmix64(uint64_t s) {
    s ^= s >> 33;
    s *= 0xff51afd7ed558ccdull;
    s ^= s >> 33;
    s *= 0xc4ceb9fe1a85ec53ull;
    s ^= s >> 33;
    return s;
}

// Lanes per row and logits per lane: 1024 x 32 >= 30000, so each lane issues
// all of its loads at once and keeps its logits in registers (a strided
// loop, one load at a time, took 63 us at [64, 30000]).
constexpr int kTopPLanes = 1024;
constexpr int kTopPPerLane = 32;
static_assert(kTopPLanes * kTopPPerLane >= kTopPMaxVocab, "a row must fit the registers");
constexpr int kTopPRankParts = kTopPLanes / 256;  // lanes that rank one candidate
static_assert(kTopPWalk / kTopPRankParts % 4 == 0, "rank slices are whole float4s");

__global__ __launch_bounds__(kTopPLanes) void top_p_small_kernel(const half_t* __restrict__ logits,
                                                                 int vocab, float p,
                                                                 float temperature, uint64_t seed,
                                                                 int32_t* out) {
    __shared__ float slots[kTopPLanes / kWave];
    // x, then q, of candidate c (index c * 128); zero past the candidates
    __shared__ __attribute__((aligned(16))) float cand[kTopPWalk];
    __shared__ int partial[kTopPRankParts][256];
    // q in walk order, zero past the candidates, read 16 at a time
    __shared__ __attribute__((aligned(16))) float sorted_q[kTopPWalk];
    __shared__ int sorted_i[kTopPMaxCand];
    const int64_t row = blockIdx.x;
    const half_t* x = logits + row * vocab;
    const int tid = threadIdx.x;
    const int nc = (vocab + kTopPStride - 1) / kTopPStride;

    float xv[kTopPPerLane];
#pragma unroll
    for (int j = 0; j < kTopPPerLane; ++j) {
        const int i = tid + j * kTopPLanes;
        xv[j] = i < vocab ? (float)x[i] : -INFINITY;
    }
    // max of x / T = (max of x) / T: division by T > 0, correctly rounded,
    // is monotone
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kTopPPerLane; ++j) m = fmaxf(m, xv[j]);
    const float M = block_max(m, slots) / temperature;
    __syncthreads();  // slots reused by the sum
    // the normaliser: x / T as x * (1 / T) (within an ulp; the candidates'
    // own probabilities below use the division)
    const float rT = 1.0f / temperature;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kTopPPerLane; ++j) s += fast_exp(xv[j] * rT - M);  // -inf -> 0
    // candidate c sits in lane (c % 8) * 128, register c / 8: those lanes
    // stage x, then lane c forms q_c
    if ((tid & (kTopPStride - 1)) == 0) {
#pragma unroll
        for (int j = 0; j < kTopPPerLane; ++j) {
            const int c = j * (kTopPLanes / kTopPStride) + tid / kTopPStride;
            if (c < nc) cand[c] = xv[j];
        }
    }
    const float S = block_sum(s, slots);  // its barrier also publishes cand
    float qc = 0.0f;
    if (tid < nc) qc = fast_exp(cand[tid] / temperature - M) / S;
    __syncthreads();  // every lane has read its x
    if (tid < kTopPWalk) cand[tid] = qc;  // zero past the candidates
    __syncthreads();
    // rank by (q descending, index ascending), the order the reference's
    // strict-greater selection produces: four lanes per candidate, each
    // comparing a quarter of the candidates, 16 bytes per LDS read
    {
        const int c = tid & 255, part = tid >> 8;
        int r = 0;
        if (c < nc) {
            const float v = cand[c];
            constexpr int kSlice = kTopPWalk / kTopPRankParts;  // 60
            const int lo = part * kSlice;
            const float4* c4 = reinterpret_cast<const float4*>(cand + lo);
#pragma unroll
            for (int k4 = 0; k4 < kSlice / 4; ++k4) {
                const float4 t = c4[k4];
                const float u[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int o = lo + 4 * k4 + e;
                    r += (o < nc && (u[e] > v || (u[e] == v && o < c))) ? 1 : 0;
                }
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
    } else if (tid < kTopPWalk) {
        sorted_q[tid] = 0.0f;
    }
    __syncthreads();
    if (tid == 0) {
        // the reference's running fp32 sum, in order: 16 values per batch of
        // vector reads; only the additions are chained, the threshold tests
        // follow them
        int hit = -1;
        float cum = 0.0f;
        const float4* q4 = reinterpret_cast<const float4*>(sorted_q);
        for (int base = 0; base < nc && hit < 0; base += 16) {
            float v[16], c[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 t = q4[base / 4 + k];
                v[4 * k] = t.x;
                v[4 * k + 1] = t.y;
                v[4 * k + 2] = t.z;
                v[4 * k + 3] = t.w;
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                cum += v[k];
                c[k] = cum;
            }
#pragma unroll
            for (int k = 15; k >= 0; --k)
                if (base + k < nc && c[k] >= p) hit = base + k;
        }
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
}

int top_p(const void* logits, int64_t B, int64_t vocab, float p, float temperature,
          uint64_t seed, int32_t* out, void* stream) {
    if (B < 0 || vocab < 0) return MI_ERR_INVALID_ARGUMENT;
    if (B == 0) return MI_OK;
    if (!out || (vocab > 0 && !logits)) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({B, vocab, 2})) return MI_ERR_INVALID_ARGUMENT;
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
