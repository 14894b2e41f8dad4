// softmax.hip -- row softmax for gfx950, fp16 in/out, fp32 math.
//
// Arithmetic follows the reference (src/kernels/softmax_kernel.cu:26-58):
// m = max(x), S = sum(exp(x - m)), y = half(exp(x - m) * (1 / S)).
//
// Design (HBM-bound: 4 bytes/element):
//   * Each lane keeps an online (max, sum) pair over its 16-byte vectors,
//     rescaling the sum when the max grows, so statistics need ONE read of x
//     (the reference makes separate max and sum passes, then a third to write).
//   * Many rows (N >= 512; N >= 256 up to 65536): whole rows, in registers
//     where they fit (softmax_reg_kernel), else one workgroup per row whose
//     write pass re-reads the row through L2.
//   * Few long rows (the LM-head case, 64 x 152064), and many rows longer
//     than 32768 (N >= 512, or N >= 256 up to 65536): one workgroup per row
//     would light up few CUs or re-read the row, so each row is cut into
//     8192-element chunks.  With row records -- a caller workspace, or on
//     stream 0 a region the library holds -- and y != x, one launch
//     (softmax_stream_kernel, below): a resident grid of chunk workgroups
//     holds the chunks in registers and exchanges their (max, sum) through
//     tagged per-row records, walking the rows in rounds when they are more
//     than the grid holds, with the next row's loads in flight during each
//     exchange.  Otherwise many rows take a workgroup per row, and few rows
//     two launches with `splits` chunks:
//     Kernel 1 writes a (max, sum) pair per chunk to a small stream-ordered
//     workspace (8 bytes per chunk), from tiles whose loads are all issued
//     first (one HBM wait per tile), a packed fp16 lane maximum and one exp
//     per element;
//     kernel 2, on the same grid, merges the row's pairs (each lane folds
//     every 64th chunk, then wave reductions, no barrier) and writes its
//     chunk.  Its re-read of the chunk misses L2, which does not carry
//     data across kernel launches on this multi-XCD GPU (FETCH_SIZE counts
//     the full 2 bytes/element again); it is served from the 256 MB
//     Infinity Cache when the logits are still resident there, else HBM.
#include <atomic>
#include <map>
#include <mutex>

#include "argmax_key.h"
#include "mi_device.h"
#include "mi_host.h"
#include "row_exchange.h"

// Softmax stores: plain non-temporal (1 = write-through "nt sc1"; measured neutral).
#ifndef MI_WT_SM
#define MI_WT_SM 0
#endif

namespace mi {
namespace {

constexpr int kSplitMaxRows = 512;  // below this many rows, split each row
#ifndef MI_SOFTMAX_REG_ROWS
#define MI_SOFTMAX_REG_ROWS 256
#endif
constexpr int kMaxSplits = 1024;    // chunk pairs of a row, folded by one wave
#ifndef MI_SOFTMAX_TARGET_WGS
#define MI_SOFTMAX_TARGET_WGS 2048
#endif
constexpr int64_t kSplitTargetWgs = MI_SOFTMAX_TARGET_WGS;

// exp(x - m) for every element of a row against one m, with m * log2(e)
// formed once: one fma and the exp per element instead of a subtract, a
// multiply and the exp (the VALU work sits on the critical path before and
// after a one-launch row's exchange: 9.5 -> 8.9 us at [64, 152064]).
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float exp_shifted(float x, float m_log2e) {
    return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -m_log2e));
}

// Fold one loaded value group into the lane's online (m, s).
template <int VEC>
__device__ __forceinline__ void fold(const float (&v)[VEC], float& m, float& s) {
    float vm = v[0];
#pragma unroll
    for (int k = 1; k < VEC; ++k) vm = fmaxf(vm, v[k]);
    const float mn = fmaxf(m, vm);
    if (mn == -INFINITY) return;  // nothing but -inf so far
    float acc = s * fast_exp(m - mn);
    const float mnl = mn * kLog2e;
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc += exp_shifted(v[k], mnl);
    s = acc;
    m = mn;
}

// Accumulate elements [begin, end) of a row into this lane's (m, s).  Loads
// are issued kStatUnroll groups at a time, before the math that consumes them.
constexpr int kStatUnroll = 4;
template <int VEC>
__device__ __forceinline__ void lane_stats(const half_t* xr, int64_t begin, int64_t end, float& m,
                                           float& s) {
    const int64_t step = static_cast<int64_t>(blockDim.x) * VEC;
    for (int64_t i0 = begin + static_cast<int64_t>(threadIdx.x) * VEC; i0 < end;
         i0 += step * kStatUnroll) {
        float v[kStatUnroll][VEC];
#pragma unroll
        for (int j = 0; j < kStatUnroll; ++j) {
            const int64_t i = i0 + j * step;
            if (i < end) {
                if constexpr (VEC == 8) {
                    const h8 h = ld8(xr + i);
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[j][k] = (float)h[k];
                } else {
                    v[j][0] = (float)xr[i];
                }
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) v[j][k] = -INFINITY;
            }
        }
#pragma unroll
        for (int j = 0; j < kStatUnroll; ++j) fold<VEC>(v[j], m, s);
    }
}

// Vector form for split rows: [begin, end) is walked in tiles of 2048 * U
// elements (U vectors per lane), all loads of a tile issued first.  The
// tile's lane maximum comes from packed fp16 max (which passes over NaN, as
// fmaxf does), then one exp per element against it, and one online merge
// per tile -- not a rescale per vector.  Out-of-range slots hold -inf, whose
// exp is 0.
template <int U>
__device__ __forceinline__ void tile_stats(const half_t* xr, int64_t begin, int64_t end, float& m,
                                           float& s) {
    constexpr int64_t kTile = 256 * 8 * U;
    for (int64_t t0 = begin; t0 < end; t0 += kTile) {
        h8 a[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const int64_t i = t0 + (threadIdx.x + j * 256) * 8;
            a[j] = i < end ? ld8(xr + i) : h8(-__builtin_huge_valf16());
        }
        h2 m2 = h2(-__builtin_huge_valf16());
#pragma unroll
        for (int j = 0; j < U; ++j) {
#pragma unroll
            for (int k = 0; k < 8; k += 2) m2 = __builtin_elementwise_max(m2, h2{a[j][k], a[j][k + 1]});
        }
        const float mt = (float)__builtin_elementwise_max(m2.x, m2.y);
        if (!(mt > -INFINITY)) continue;  // nothing but -inf (or NaN) in this lane's tile
        float st = 0.0f;
        const float mtl = mt * kLog2e;
#pragma unroll
        for (int j = 0; j < U; ++j) {
#pragma unroll
            for (int k = 0; k < 8; ++k) st += exp_shifted((float)a[j][k], mtl);
        }
        const float mn = fmaxf(m, mt);
        s = s * fast_exp(m - mn) + st * fast_exp(mt - mn);
        m = mn;
    }
}

// y = exp(x - m) * inv over [begin, end): the last use of x and the only
// write of y, both streamed.
template <int VEC>
__device__ __forceinline__ void write_range(const half_t* xr, half_t* yr, int64_t begin,
                                            int64_t end, float m, float inv) {
    const int64_t step = static_cast<int64_t>(blockDim.x) * VEC;
    for (int64_t i0 = begin + static_cast<int64_t>(threadIdx.x) * VEC; i0 < end;
         i0 += step * kStatUnroll) {
        if constexpr (VEC == 8) {
            h8 h[kStatUnroll];
#pragma unroll
            for (int j = 0; j < kStatUnroll; ++j) {
                const int64_t i = i0 + j * step;
                if (i < end) h[j] = ld8_stream(xr + i);
            }
#pragma unroll
            for (int j = 0; j < kStatUnroll; ++j) {
                const int64_t i = i0 + j * step;
                if (i < end) {
                    h8 o;
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        o[k] = to_half(exp_shifted((float)h[j][k], m * kLog2e) * inv);
                    st8_out<MI_WT_SM>(yr + i, o);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < kStatUnroll; ++j) {
                const int64_t i = i0 + j * step;
                if (i < end) yr[i] = to_half(exp_shifted((float)xr[i], m * kLog2e) * inv);
            }
        }
    }
}

// Workgroup-wide merge of per-lane (m, s): max first, then rescaled sums.
// (A one-barrier form -- wave (max, sum) pairs folded after a single barrier
// -- measured no faster at [64, 152064].)  `slots` needs one float per wave.
__device__ __forceinline__ void block_merge(float& m, float& s, float* slots) {
    const float M = block_max(m, slots);
    const float part = (m == -INFINITY) ? 0.0f : s * fast_exp(m - M);
    __syncthreads();  // slots are reused by the sum
    s = block_sum(part, slots);
    m = M;
}

// Register-resident rows (16-byte vectors, D <= G * VPT * 8): G lanes per
// row -- G <= 64: 256 / G rows per workgroup and DPP-only reductions;
// G = 256 or 1024: one row per workgroup and one LDS exchange per
// reduction -- with VPT vectors per lane.  x is read once: a packed fp16
// lane maximum, the row maximum, one exp per element (kept in registers when
// VPT <= 4, recomputed at the write otherwise), the row sum, then the scaled
// write.  Lanes past the row hold -inf, whose exp is 0.  No lane returns
// early, so every group reduction sees all of its lanes.
template <int G, int VPT>
__global__ __launch_bounds__(G > 256 ? G : 256) void softmax_reg_kernel(const half_t* x,
                                                                        half_t* y, int64_t N,
                                                                        int64_t D) {
    constexpr int kThreads = G > 256 ? G : 256;
    constexpr int kRows = kThreads / G;
    constexpr bool kKeepExp = VPT <= 4;
    __shared__ float smax[kThreads / kWave], ssum[kThreads / kWave];
    const int gl = threadIdx.x & (G - 1);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRows + threadIdx.x / G;
    const bool live = row < N;
    const int64_t nv = D >> 3;
    const half_t* xr = x + row * D;
    h8 a[VPT];
    // vector j of this lane: a uniform base per j (xr + j * G * 8) plus the
    // lane's 32-bit byte offset (with the forced recompute below, 8-vector
    // rows went from 90-115 to 78-88 VGPRs)
    const uint32_t lo = static_cast<uint32_t>(gl) * 16u;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t v = gl + j * G;
        const char* base = reinterpret_cast<const char*>(xr + static_cast<int64_t>(j) * G * 8);
        a[j] = live && v < nv ? ld8_stream(reinterpret_cast<const half_t*>(base + lo))
                              : h8(-__builtin_huge_valf16());
    }
    h2 m2 = h2(-__builtin_huge_valf16());
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
#pragma unroll
        for (int k = 0; k < 8; k += 2) m2 = __builtin_elementwise_max(m2, h2{a[j][k], a[j][k + 1]});
    }
    float m = (float)__builtin_elementwise_max(m2.x, m2.y);
    if constexpr (G <= 64)
        m = group_max<G>(m);
    else
        m = block_max(m, smax);
    float e[kKeepExp ? VPT : 1][8];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float t = exp_shifted((float)a[j][k], m * kLog2e);
            if constexpr (kKeepExp) e[j][k] = t;
            s += t;
        }
    }
    if constexpr (G <= 64)
        s = group_sum<G>(s);
    else
        s = block_sum(s, ssum);
    const float inv = 1.0f / s;
    // Recomputing the exps (VPT > 4): an opaque copy of m keeps the compiler
    // from reusing the sum loop's exps, which would hold 8 * VPT fp32 values
    // live instead of the 4 * VPT registers of fp16 data.
    float mw = m;
    if constexpr (!kKeepExp) asm volatile("" : "+v"(mw));
    half_t* yr = y + row * D;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t v = gl + j * G;
        if (live && v < nv) {
            h8 o;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float t =
                    kKeepExp ? e[kKeepExp ? j : 0][k] : exp_shifted((float)a[j][k], mw * kLog2e);
                o[k] = to_half(t * inv);
            }
            st8_out<MI_WT_SM>(
                reinterpret_cast<half_t*>(
                    reinterpret_cast<char*>(yr + static_cast<int64_t>(j) * G * 8) + lo),
                o);
        }
    }
}

// Launch shape for softmax_reg_kernel: the fewest lanes per row (8, 16, 32,
// 64, then 256 or 1024 as whole workgroups) that hold the row in at most
// kRegVpt vectors each, else 1024 lanes with up to 8.  Returns false when
// the row needs more than 1024 x 8 vectors.
#ifndef MI_SOFTMAX_REG_VPT
#define MI_SOFTMAX_REG_VPT 4
#endif
constexpr int kRegVpt = MI_SOFTMAX_REG_VPT;
// At most 8 vectors per lane (rows <= 1024 x 8 x 8 = 65536).  12 fit in
// 110 VGPRs but measured mixed: [256, 98304] 51% -> 57%, [300, 70000]
// 45% -> 36% (idle lanes and a 17%-full second round); 16 or more spill.
constexpr int kRegVptMax = 8;
bool reg_shape(int64_t nv, int& G, int& VPT) {
    static const int kG[] = {8, 16, 32, 64, 256, 1024};
    G = 0;
    for (int g : kG)
        if (nv <= static_cast<int64_t>(kRegVpt) * g) {
            G = g;
            break;
        }
    if (G == 0) {
        if (nv > 1024 * kRegVptMax) return false;
        G = 1024;
    }
    const int64_t v = ceil_div(nv, G);
    VPT = v <= 1 ? 1 : v <= 2 ? 2 : v <= 4 ? 4 : 8;
    if (G < 64 && VPT > 4) return false;  // not instantiated (kRegVpt > 4 only)
    return true;
}

template <int G>
void launch_reg(const half_t* x, half_t* y, int64_t N, int64_t D, int VPT, hipStream_t s) {
    constexpr int kThreads = G > 256 ? G : 256;
    const dim3 g(static_cast<unsigned>(ceil_div(N, kThreads / G))), b(kThreads);
    if (VPT == 1)
        softmax_reg_kernel<G, 1><<<g, b, 0, s>>>(x, y, N, D);
    else if (VPT == 2)
        softmax_reg_kernel<G, 2><<<g, b, 0, s>>>(x, y, N, D);
    else if (VPT == 4 || G < 64)  // reg_shape gives fewer than 64 lanes at most 4 vectors
        softmax_reg_kernel<G, 4><<<g, b, 0, s>>>(x, y, N, D);
    else if constexpr (G >= 64)
        softmax_reg_kernel<G, 8><<<g, b, 0, s>>>(x, y, N, D);
}

template <int VEC>
__global__ __launch_bounds__(1024) void softmax_row_kernel(const half_t* x, half_t* y, int64_t D) {
    __shared__ float slots[1024 / kWave];
    const int64_t row = blockIdx.x;
    const half_t* xr = x + row * D;
    half_t* yr = y + row * D;
    float m = -INFINITY, s = 0.0f;
    lane_stats<VEC>(xr, 0, D, m, s);
    block_merge(m, s, slots);
    write_range<VEC>(xr, yr, 0, D, m, 1.0f / s);
}

// VEC = 8: U vectors per lane per tile (tile_stats); VEC = 1: lane_stats.
template <int VEC, int U>
__global__ __launch_bounds__(256) void softmax_partial_kernel(const half_t* x, float* ws,
                                                              int64_t D, int64_t chunk) {
    __shared__ float slots[256 / kWave];
    const int split = blockIdx.x, splits = gridDim.x;
    const int64_t row = blockIdx.y;
    const int64_t b = split * chunk;
    const int64_t e = b + chunk < D ? b + chunk : D;
    float m = -INFINITY, s = 0.0f;
    if constexpr (VEC == 8)
        tile_stats<U>(x + row * D, b, e, m, s);
    else
        lane_stats<VEC>(x + row * D, b, e, m, s);
    block_merge(m, s, slots);
    if (threadIdx.x == 0) {
        float* p = ws + (row * splits + split) * 2;
        p[0] = m;
        p[1] = s;
    }
}

template <int VEC>
__global__ __launch_bounds__(256) void softmax_finish_kernel(const half_t* x, half_t* y,
                                                             const float* __restrict__ ws,
                                                             int64_t D, int64_t chunk) {
    const int split = blockIdx.x, splits = gridDim.x;
    const int64_t row = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1);
    // Every wave merges the row's pairs itself: lane j folds chunks j, j + 64, ...
    float m = -INFINITY, s = 0.0f;
    for (int j = lane; j < splits; j += kWave) {
        const float* p = ws + (row * splits + j) * 2;
        const float mj = p[0], sj = p[1];
        if (mj == -INFINITY) continue;
        const float mn = fmaxf(m, mj);
        s = s * fast_exp(m - mn) + sj * fast_exp(mj - mn);
        m = mn;
    }
    const float M = group_max<kWave>(m);
    const float S = group_sum<kWave>(m == -INFINITY ? 0.0f : s * fast_exp(m - M));
    const int64_t b = split * chunk;
    const int64_t e = b + chunk < D ? b + chunk : D;
    write_range<VEC>(x + row * D, y + row * D, b, e, M, 1.0f / S);
}

// ---------------------------------------------------------------------------
// One-launch split rows (row records: mi_softmax_ws_f16, or stream 0; x != y):
// each workgroup holds an 8192-element chunk of a row in registers, publishes
// the chunk's (max, sum), and reads every chunk's pair of its row to finish --
// one launch, one read of x, no atomics on a contended address.  The grid is
// `chunks per row` x R row slots, all resident; slot r handles rows r, r + R,
// ... in rounds (one round when every row fits), and issues its next row's
// loads before it polls for the current row's statistics.
//
// Workspace (zero before first use; every call leaves it valid for the
// next): row slot r owns a fixed record at r * kRowRecordBytes -- a 64-bit
// epoch word (128-byte header), then two sets of kOnePassMaxSplits slots of
// two 64-bit words {tag << 32 | bits(max)}, {tag << 32 | bits(sum)}, and a
// mirror of both sets (row_exchange.h: each word is published into the XCD's
// L2 and through to memory; polls read the L2 copy first).  A call
// reads the slot's epoch E; round k publishes into set k & 1 with tag = the
// low 32 bits of E + 1 + k and polls the set until every chunk's pair carries
// that tag.  Because slots are fixed per (row slot, chunk) whatever the
// call's shape, and an epoch only grows (64 bits: it cannot wrap), a slot
// left by an earlier call never carries the tag a later call waits for --
// short of a slot left unwritten for 2^32 of its epochs and read again at
// exactly a multiple of 2^32 later:
//   * the chunk-0 workgroup raises the epoch to E + K (atomic max) after the
//     last (K-th) round, when every workgroup of the slot has published it --
//     so every one of them has already read E;
//   * a workgroup whose polling runs out (kPollLimit polls or kPollTicks of
//     the 100 MHz constant clock, whichever comes first; not expected when
//     the grid fits the GPU) computes that row's statistics itself from x and
//     raises the epoch to E + K + 1 at once, past every tag the launch writes
//     for the slot.  A workgroup that starts after that reads the higher
//     epoch, its tags match nobody's, and it takes the same fallback for its
//     rows: slower, still correct.  A workgroup that has fallen back once
//     stops polling for its remaining rounds (its row-mates may be out of
//     step with it for good), so a late start costs at most one poll bound
//     per workgroup, not one per round.  Polling is bounded: no workgroup
//     can wait forever.
// A workgroup publishes round k + 2 into a set only after it has seen every
// chunk's round k + 1 pair, which its row-mates publish after they have read
// round k: no pair is overwritten before it is read.  Each 64-bit word is
// stored and loaded whole, so a tag always travels with its value.
// The grid is 1-D and places every chunk of a row slot on one XCD
// (chunk_of), so the L2 copy normally serves the polls.
// ---------------------------------------------------------------------------
constexpr int kOnePassMaxSplits = 64;
#ifndef MI_SOFTMAX_ONEPASS_U
#define MI_SOFTMAX_ONEPASS_U 4
#endif
constexpr int kOnePassU = MI_SOFTMAX_ONEPASS_U;     // vectors per lane
constexpr int64_t kOnePassChunk = 2048 * kOnePassU;  // elements per workgroup
// header, then two sets of slots (alternated by round) and their mirror; a
// slot is the chunk's tagged (max, sum) pair, plus its tagged argmax key (two
// words) in the fused softmax + argmax pass
constexpr int64_t kRowRecordBytes = kRecordHeaderBytes + 4 * kOnePassMaxSplits * 16;
constexpr int64_t kRowRecordBytesAM = kRecordHeaderBytes + 4 * kOnePassMaxSplits * 32;
template <bool AM>
constexpr int64_t record_bytes() { return AM ? kRowRecordBytesAM : kRowRecordBytes; }
constexpr int kPollLimit = 1 << 16;
std::atomic<int> g_poll_limit{kPollLimit};  // mi_softmax_test_poll_limit

__device__ __forceinline__ uint64_t tagged(uint32_t tag, float v) {
    return (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, v);
}

// The pieces of a one-launch chunk workgroup.
// The lane's (max, sum) over its vectors: packed fp16 maximum, one exp per
// element.
template <int U>
__device__ __forceinline__ void chunk_lane_stats(const h8 (&a)[U], float& m, float& s) {
    h2 m2 = h2(-__builtin_huge_valf16());
#pragma unroll
    for (int j = 0; j < U; ++j) {
#pragma unroll
        for (int k = 0; k < 8; k += 2) m2 = __builtin_elementwise_max(m2, h2{a[j][k], a[j][k + 1]});
    }
    m = (float)__builtin_elementwise_max(m2.x, m2.y);
    s = 0.0f;
    if (m > -INFINITY) {
        const float ml = m * kLog2e;
#pragma unroll
        for (int j = 0; j < U; ++j) {
#pragma unroll
            for (int k = 0; k < 8; ++k)
                s += exp_shifted((float)a[j][k], ml);
        }
    } else {
        m = -INFINITY;  // NaN-free lane maximum of an all -inf (or NaN) lane
    }
}
// Thread 0 publishes the chunk's pair (and, AM, its argmax key) into slot
// `split` of `slots` (SW = 2 or 4 words per slot) and of its mirror
// (`mirror` words on).
template <bool AM>
__device__ __forceinline__ void chunk_publish(uint64_t* slots, int64_t mirror, int split,
                                              uint32_t tag, float m, float s, uint64_t key) {
    constexpr int SW = AM ? 4 : 2;
    if (threadIdx.x == 0) {
        uint64_t w[SW];
        w[0] = tagged(tag, m);
        w[1] = tagged(tag, s);
        if constexpr (AM) {
            const uint64_t t = static_cast<uint64_t>(tag) << 32;
            w[2] = t | (key >> 32);
            w[3] = t | (key & 0xffffffffu);
        }
        uint64_t* p = slots + SW * split;
#pragma unroll
        for (int i = 0; i < SW; ++i) local_store(&p[i], w[i]);
#pragma unroll
        for (int i = 0; i < SW; ++i) device_store(&p[mirror + i], w[i]);
    }
}
// Wave 0 (the caller calls it there) polls the row's `splits` slots (lane j
// reads chunk j) until all carry `tag`, at most poll_limit rounds -- the L2
// copy (local) for up to kLocalPollTicks, then the mirror `mirror` words on
// at device scope (row_exchange.h) -- and leaves
// the row's (M, S) in row_stats[0..1] (AM with want_key: its best key in
// *row_key, the key words polled too; without, only the pair words, half
// the bytes per poll: 12.9 -> 12.0 us at [64, 152064]) and row_stats[2] = 0,
// or row_stats[2] = 1 when polling ran out.  The caller's barrier publishes
// them.
// Polls of one phase (LOCAL: the L2 copy, else the device-scope mirror) of
// `set` (workgroup-uniform) until every chunk's slot carries `tag`, `it`
// reaches poll_limit or the clock passes t0 + ticks; lane j < splits reads
// slot j.  Returns whether every slot was seen.
template <bool AM, bool LOCAL>
__device__ __forceinline__ bool poll_phase(const uint64_t* set, int splits, uint32_t tag,
                                           bool want_key, int& it, int poll_limit, uint64_t t0,
                                           uint64_t ticks, float& mj, float& sj, uint64_t& kj) {
    constexpr int SW = AM ? 4 : 2;
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t off = static_cast<uint32_t>(lane) * (SW * 8);
    for (; it < poll_limit; ++it) {
        if (it > 0 && __builtin_amdgcn_s_memrealtime() - t0 > ticks) return false;
        bool mine = true;
        if (lane < splits) {
            // chunk 0 alone writes the index, so only it reads the key words
            uint64_t w[SW];
            if (AM && want_key)
                load_slot<LOCAL, SW>(set, off, w);
            else
                load_slot<LOCAL, 2>(set, off, reinterpret_cast<uint64_t(&)[2]>(w));
            mine = static_cast<uint32_t>(w[0] >> 32) == tag && static_cast<uint32_t>(w[1] >> 32) == tag;
            mj = __builtin_bit_cast(float, static_cast<uint32_t>(w[0]));
            sj = __builtin_bit_cast(float, static_cast<uint32_t>(w[1]));
            if constexpr (AM) {
                if (want_key) {
                    mine = mine && static_cast<uint32_t>(w[2] >> 32) == tag &&
                           static_cast<uint32_t>(w[3] >> 32) == tag;
                    kj = (w[2] << 32) | (w[3] & 0xffffffffu);
                }
            }
        }
        if (__all(mine)) return true;
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

template <bool AM>
__device__ __forceinline__ void row_poll(const uint64_t* slots, int64_t mirror, bool local,
                                         int splits, uint32_t tag, int poll_limit,
                                         float* row_stats, uint64_t* row_key, bool want_key) {
    const int lane = threadIdx.x & (kWave - 1);
    float mj = -INFINITY, sj = 0.0f;
    uint64_t kj = 0;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    int it = 0;
    bool all = local && poll_phase<AM, true>(slots, splits, tag, want_key, it, poll_limit, t0,
                                             kLocalPollTicks, mj, sj, kj);
    if (!all)
        all = poll_phase<AM, false>(slots + mirror, splits, tag, want_key, it, poll_limit, t0,
                                    kPollTicks, mj, sj, kj);
    if (all) {
        if (lane >= splits) {
            mj = -INFINITY;
            sj = 0.0f;
            kj = 0;
        }
        const float M = group_max<kWave>(mj);
        const float S = group_sum<kWave>(mj == -INFINITY ? 0.0f : sj * fast_exp(mj - M));
        if (AM && want_key) kj = wave_max_u64(kj);
        if (lane == 0) {
            row_stats[0] = M;
            row_stats[1] = S;
            row_stats[2] = 0.0f;
            if (AM && want_key) *row_key = kj;
        }
    } else if (lane == 0) {
        row_stats[2] = 1.0f;
    }
}
// The row's statistics from x itself (the fallback when polling runs out; x
// is not written: y != x).  Barriers: called by the whole workgroup.
__device__ __forceinline__ void row_stats_from_x(const half_t* xr, int64_t D, float& M, float& S,
                                                 float* slots) {
    float fm = -INFINITY, fs = 0.0f;
    tile_stats<2>(xr, 0, D, fm, fs);
    __syncthreads();  // slots reused
    block_merge(fm, fs, slots);
    __syncthreads();  // every wave has read slots before a later round writes them
    M = fm;
    S = fs;
}
// The persistent kernel's per-lane view of its chunk: the same in every
// round, so one 32-bit byte offset (rows are < 2^31 bytes) and a valid flag
// per vector, against a row base that is uniform across the workgroup.
template <int U>
__device__ __forceinline__ void lane_load(const half_t* row, uint32_t lo, const bool (&ok)[U],
                                          h8 (&a)[U]) {
    const char* base = reinterpret_cast<const char*>(row) + lo;
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const half_t* p = reinterpret_cast<const half_t*>(base + j * 256 * 16);
        a[j] = ok[j] ? ld8_stream(p) : h8(-__builtin_huge_valf16());
    }
}
template <int U>
__device__ __forceinline__ void lane_store(const h8 (&a)[U], half_t* row, uint32_t lo,
                                           const bool (&ok)[U], float M, float inv) {
    // y = exp(x - M) / S = exp2(x log2(e) - (M log2(e) + log2(S))): the division folded into
    // the exponent's constant c, one fma and the exp per element ([512, 131072] 46.4 -> 46.0
    // us; c carries the same rounding as M log2(e) alone, well under an fp16 ulp of y)
    const float c = M * kLog2e - __builtin_amdgcn_logf(inv);
    char* base = reinterpret_cast<char*>(row) + lo;
#pragma unroll
    for (int j = 0; j < U; ++j) {
        if (ok[j]) {
            h8 o;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                o[k] = to_half(__builtin_amdgcn_exp2f(fmaf((float)a[j][k], kLog2e, -c)));
            st8_out<MI_WT_SM>(reinterpret_cast<half_t*>(base + j * 256 * 16), o);
        }
    }
}

// 64 VGPRs, so 8 workgroups per CU (per-lane 32-bit offsets, not 64-bit
// indices: 68 VGPRs and 7 workgroups per CU with them measured 5-10 points
// lower; amdgpu_waves_per_eu(8) also measured ~8 points lower at the same
// 64 VGPRs); wave 0 publishes and polls.
// U vectors per lane: chunks of 2048 * U elements.  AM: the fused softmax +
// greedy argmax pass -- each chunk also forms its best argmax key from the
// registers it already holds, publishes it with its (max, sum), and chunk 0
// writes the row's index to `out` (the fallback scans the row from x).
// (AM: held to 5 waves per SIMD, <= 96 VGPRs, so that 1216 chunk workgroups
// of [64, 152064] stay resident at once; the compiler otherwise settles at
// 98 and the grid needs a second round.)
template <int U, bool AM>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(AM ? 5 : 1))) void softmax_stream_kernel(const half_t* x, half_t* y,
                                                             unsigned char* ws, int64_t N,
                                                             int64_t D, int poll_limit,
                                                             int32_t* out, int splits, int R,
                                                             int local) {
    constexpr int64_t kChunk = 2048 * U;
    constexpr int SW = AM ? 4 : 2;
    __shared__ float slots[256 / kWave];
    __shared__ float row_stats[3];  // M, S, fallback flag
    __shared__ uint64_t epoch_sh;
    __shared__ uint64_t kslots[AM ? 256 / kWave : 1];  // per-wave keys (AM)
    __shared__ uint64_t row_key;                        // the row's best key (AM)
    // 1-D grid of splits x R (R a multiple of kXcds): a row slot's chunks
    // share one XCD (row_exchange.h); slots past N-1 have no rows
    int split, slot;
    chunk_of(blockIdx.x, splits, split, slot);
    const int64_t r0 = slot;
    if (r0 >= N) return;  // workgroup-uniform, before any barrier
    unsigned char* rec = ws + r0 * record_bytes<AM>();
    uint64_t* epoch = reinterpret_cast<uint64_t*>(rec);
    uint64_t* sets = reinterpret_cast<uint64_t*>(rec + kRecordHeaderBytes);
    constexpr int64_t kMirror = 2 * SW * kOnePassMaxSplits;  // words from a set to its mirror
    const int64_t K = (N - r0 + R - 1) / R;  // rounds of this row slot (>= 1)
    const int64_t b = split * kChunk;
    const int64_t e = b + kChunk < D ? b + kChunk : D;
    const uint32_t lo = static_cast<uint32_t>(b + threadIdx.x * 8) * 2;
    bool ok[U];
#pragma unroll
    for (int j = 0; j < U; ++j) ok[j] = b + (threadIdx.x + j * 256) * 8 < e;

    if (threadIdx.x == 0)
        epoch_sh = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    h8 a[U], n[U];
    lane_load<U>(x + r0 * D, lo, ok, a);
    bool gave_up = false;  // workgroup-uniform: set after the first fallback
    for (int64_t k = 0; k < K; ++k) {
        const int64_t row = r0 + k * R;
        // The guard is always true (256 lanes); written out, it keeps the
        // statistics in a block of their own, which measured 64 VGPRs with
        // no spill against 80 without it.
        float m = -INFINITY, s = 0.0f;
        if (threadIdx.x < 256) chunk_lane_stats<U>(a, m, s);
        if constexpr (AM) {
            // vectors past the row hold -inf (lane_load), whose key is 0
            const uint64_t kw = wave_max_u64(lane_best_key<U>(a, b));
            if ((threadIdx.x & (kWave - 1)) == 0) kslots[threadIdx.x / kWave] = kw;
        }
        block_merge(m, s, slots);  // barriers: epoch_sh (first round) and kslots visible after
        uint64_t key = 0;
        if constexpr (AM) {
#pragma unroll
            for (int w = 0; w < 256 / kWave; ++w) key = max_u64(key, kslots[w]);
        }
        const uint64_t E = epoch_sh;
        const uint32_t tag = static_cast<uint32_t>(E + 1 + k);
        uint64_t* set = sets + (k & 1) * (SW * kOnePassMaxSplits);
        chunk_publish<AM>(set, kMirror, split, tag, m, s, key);
        if (k + 1 < K) lane_load<U>(x + (row + R) * D, lo, ok, n);
        if (gave_up) {
            if (threadIdx.x == 0) row_stats[2] = 1.0f;
        } else if (threadIdx.x < kWave) {
            // only chunk 0 writes the index, so only it polls the key words
            row_poll<AM>(set, kMirror, local != 0, splits, tag, poll_limit, row_stats, &row_key,
                         split == 0);
        }
        __syncthreads();
        float M = row_stats[0], S = row_stats[1];
        const bool fallback = row_stats[2] != 0.0f;
        gave_up = gave_up || fallback;
        if (fallback) row_stats_from_x(x + row * D, D, M, S, slots);
        if constexpr (AM) {
            if (split == 0) {  // workgroup-uniform: chunk_best has barriers
                uint64_t rk = row_key;
                if (fallback) {
                    rk = chunk_best<8, 4>(x + row * D, 0, D, kslots);
                    __syncthreads();  // kslots are written again by the next round
                }
                if (threadIdx.x == 0) out[row] = key_index(rk);
            }
        }
        if (threadIdx.x == 0 && (fallback || (split == 0 && k + 1 == K)))
            __hip_atomic_fetch_max(epoch, fallback ? E + K + 1 : E + K, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        lane_store<U>(a, y + row * D, lo, ok, M, 1.0f / S);
        if (k + 1 < K) {
#pragma unroll
            for (int j = 0; j < U; ++j) a[j] = n[j];
        }
    }
}

// kStream: many rows long enough that chunking them beats a workgroup per
// row; with row records and y != x they run as softmax_stream_kernel,
// otherwise as kRow.
enum class Plan { kRow, kTwoPass, kStream };

#ifndef MI_SOFTMAX_STREAM
#define MI_SOFTMAX_STREAM 1
#endif
#ifndef MI_SOFTMAX_STREAM_MIN_D
#define MI_SOFTMAX_STREAM_MIN_D 32769
#endif
bool stream_shape(int64_t D) {
    return MI_SOFTMAX_STREAM && D >= MI_SOFTMAX_STREAM_MIN_D &&
           D <= kOnePassMaxSplits * kOnePassChunk;
}

// Few long rows are split into chunks: aim at ~2048 workgroups (a 19.5 MB
// read-and-reduce measured flat at 5.0-5.5 us from 1216 to 4800 workgroups)
// with chunks of a whole number of tiles -- 4096 elements (two vectors per
// lane) when that still gives >= 1024 workgroups, else 2048.  (Keeping a
// whole row in one workgroup's registers instead measured 2x slower at
// [64, 152064]: a single CU sustains only ~12 GB/s, so 64 busy CUs cannot
// feed HBM.)
int64_t split_tile(int64_t N, int64_t D) { return N * ceil_div(D, 4096) >= 1024 ? 4096 : 2048; }

Plan plan(int64_t N, int64_t D, int64_t& splits, int64_t& chunk) {
    splits = 1;
    chunk = D;
    if (N >= kSplitMaxRows || D < 8192) return stream_shape(D) ? Plan::kStream : Plan::kRow;
    // 256 rows or more that register rows hold (D <= 1024 x 8 x 8): one
    // 1024-lane workgroup per row beat splitting them (measured at [256,
    // 32000] 45% -> 49%, [256, 65536] 49% -> 56%, [384, 16384] 39% -> 47%)
    if (N >= MI_SOFTMAX_REG_ROWS && D <= 1024 * kRegVptMax * 8)
        return stream_shape(D) ? Plan::kStream : Plan::kRow;
    const int64_t tile = split_tile(N, D);
    int64_t sp = ceil_div(kSplitTargetWgs, N);
    if (sp > kMaxSplits) sp = kMaxSplits;
    int64_t tiles = (ceil_div(D, sp) + tile / 2) / tile;  // nearest whole number of tiles
    if (tiles < 1) tiles = 1;
    chunk = tiles * tile;
    splits = ceil_div(D, chunk);
    return Plan::kTwoPass;
}

// Workspace of the two-pass split plan: one (max, sum) pair per chunk.
int64_t twopass_bytes(int64_t N, int64_t D) {
    int64_t splits, chunk;
    if (plan(N, D, splits, chunk) != Plan::kTwoPass) return 0;
    return N * splits * 2 * static_cast<int64_t>(sizeof(float));
}

// mi_softmax_ws_f16's workspace for split rows: the one-pass records of
// every possible row (fixed, so any call shape finds its rows' records in the
// same place), then the two-pass pairs (in-place or unaligned calls).
constexpr int64_t kOnePassRegion = kSplitMaxRows * kRowRecordBytes;
int64_t workspace_bytes(int64_t N, int64_t D) {
    int64_t splits, chunk;
    if (plan(N, D, splits, chunk) == Plan::kStream) return kOnePassRegion;
    const int64_t two = twopass_bytes(N, D);
    return two > 0 ? kOnePassRegion + two : 0;
}

#ifndef MI_SOFTMAX_ONEPASS
#define MI_SOFTMAX_ONEPASS 1
#endif
#ifndef MI_SOFTMAX_REG
#define MI_SOFTMAX_REG 1
#endif

// What a workspace handed to softmax_checked holds.
enum class Ws {
    kPairs,             // the two-pass (max, sum) pairs only (allocating entry point)
    kRecordsThenPairs,  // workspace_bytes() layout (mi_softmax_ws_f16)
    kRecords,           // the one-pass row records only (library-held, stream 0)
};

// Vectors per lane of the one-launch chunks: kOnePassU (8192 elements), or
// half that when the larger chunks would leave fewer than
// MI_SOFTMAX_SMALL_CHUNK_WGS workgroups in the launch (measured +1.4 to +2.2
// points at [200, 32000], [100, 40000], [32, 152064]; 2048 cost [64, 152064]
// 6 points, as its 38 smaller chunks per row no longer fit in one round).
#ifndef MI_SOFTMAX_SMALL_CHUNK_WGS
#define MI_SOFTMAX_SMALL_CHUNK_WGS 1024
#endif
int onelaunch_u(int64_t N, int64_t D) {
    constexpr int kSmall = kOnePassU / 2;
    if (N * ceil_div(D, kOnePassChunk) < MI_SOFTMAX_SMALL_CHUNK_WGS &&
        ceil_div(D, 2048 * kSmall) <= kOnePassMaxSplits)
        return kSmall;
    return kOnePassU;
}
const void* onelaunch_kernel(int u, bool am) {
    if (am)
        return u == kOnePassU
                   ? reinterpret_cast<const void*>(softmax_stream_kernel<kOnePassU, true>)
                   : reinterpret_cast<const void*>(softmax_stream_kernel<kOnePassU / 2, true>);
    return u == kOnePassU ? reinterpret_cast<const void*>(softmax_stream_kernel<kOnePassU, false>)
                          : reinterpret_cast<const void*>(softmax_stream_kernel<kOnePassU / 2, false>);
}

// Rows of the one-launch grid: as many as stay resident next to each other
// with every chunk of a row (at most the record rows).
int64_t onelaunch_rows(int64_t N, int64_t D, bool am = false) {
    const int u = onelaunch_u(N, D);
    const int64_t sp1 = ceil_div(D, 2048 * u);
    int64_t R = resident_workgroups(onelaunch_kernel(u, am), 256) / sp1;
    if (R > N) R = N;
    if (R > kSplitMaxRows) R = kSplitMaxRows;
    return R;
}

// The one-launch grid: `splits` chunks per row, R row slots (a multiple of
// kXcds, so that chunk_of keeps each slot's chunks on one XCD; slots past
// N - 1 exit at once), 1-D.  `local`: whether polls start on the L2 copy.
struct OneLaunchGrid {
    int splits, R, local;
    unsigned blocks() const { return static_cast<unsigned>(splits) * static_cast<unsigned>(R); }
};
OneLaunchGrid onelaunch_grid(int64_t N, int64_t D, bool am) {
    OneLaunchGrid g;
    const int u = onelaunch_u(N, D);
    g.splits = static_cast<int>(ceil_div(D, 2048 * u));
    // row slots that stay resident next to each other (at most the records;
    // at least 20 = 1280 resident workgroups / 64 chunks)
    int64_t cap = resident_workgroups(onelaunch_kernel(u, am), 256) / g.splits;
    if (cap > kSplitMaxRows) cap = kSplitMaxRows;
    // every row in one round when a whole number of groups of that many
    // slots fits (slots past N - 1 idle), else the largest whole number of
    // groups that does (rows in rounds)
    const int64_t up = ceil_div(N < cap ? N : cap, kXcds) * kXcds;
    g.R = static_cast<int>(up <= cap ? up : cap / kXcds * kXcds);
    g.local = exchange_test_mode().load() == 0 ? 1 : 0;
    return g;
}

// Whether [N, D] runs as the one-launch form given row records: a split or
// kStream shape, aligned rows, y != x (the fallback re-reads x), at most 64
// chunks per row.
bool onelaunch_ok(const void* x, const void* y, int64_t N, int64_t D, bool am = false) {
    int64_t splits, chunk;
    if (!MI_SOFTMAX_ONEPASS || plan(N, D, splits, chunk) == Plan::kRow) return false;
    return D % 8 == 0 && aligned16(x) && aligned16(y) && x != y &&
           ceil_div(D, 2048 * onelaunch_u(N, D)) <= kOnePassMaxSplits &&
           onelaunch_rows(N, D, am) >= 1;
}

int softmax_checked(const void* x, void* y, int64_t N, int64_t D, void* ws, int64_t ws_bytes,
                    Ws layout, void* stream) {
    if (N < 0 || D < 0 || ws_bytes < 0) return MI_ERR_INVALID_ARGUMENT;
    if (N == 0 || D == 0) return MI_OK;
    if (!x || !y) return MI_ERR_INVALID_ARGUMENT;
    if (N > kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (!product_fits({N, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t bytes = N * D * 2;
    if (x != y && overlaps(x, bytes, y, bytes)) return MI_ERR_ALIASING;
    int64_t splits, chunk;
    const Plan p = plan(N, D, splits, chunk);
    const bool onelaunch = layout != Ws::kPairs && onelaunch_ok(x, y, N, D);
    if (layout == Ws::kRecords && p == Plan::kTwoPass && !onelaunch)
        return MI_ERR_UNSUPPORTED;  // no pairs to fall back on (callers check onelaunch_ok)
    const int64_t need = p == Plan::kRow ? 0
                         : p == Plan::kStream ? (onelaunch ? kOnePassRegion : 0)
                         : layout == Ws::kPairs ? twopass_bytes(N, D)
                         : layout == Ws::kRecords ? kOnePassRegion
                                                  : workspace_bytes(N, D);
    if (need > 0) {
        if (!ws || ws_bytes < need) return MI_ERR_INVALID_ARGUMENT;
        if (overlaps(ws, need, x, bytes) || overlaps(ws, need, y, bytes)) return MI_ERR_ALIASING;
        if (layout != Ws::kPairs && reinterpret_cast<uintptr_t>(ws) % 16 != 0)
            return MI_ERR_INVALID_ARGUMENT;
    }
    const auto* xh = static_cast<const half_t*>(x);
    auto* yh = static_cast<half_t*>(y);
    const hipStream_t s = as_stream(stream);
    const bool vec = D % 8 == 0 && aligned16(x) && aligned16(y);
    if (p == Plan::kRow || (p == Plan::kStream && !onelaunch)) {
        int G = 0, VPT = 0;
        if (MI_SOFTMAX_REG && vec && reg_shape(D / 8, G, VPT) &&
            ceil_div(N, (G > 256 ? G : 256) / G) <= kMaxGridX) {
            switch (G) {
                case 8: launch_reg<8>(xh, yh, N, D, VPT, s); break;
                case 16: launch_reg<16>(xh, yh, N, D, VPT, s); break;
                case 32: launch_reg<32>(xh, yh, N, D, VPT, s); break;
                case 64: launch_reg<64>(xh, yh, N, D, VPT, s); break;
                case 256: launch_reg<256>(xh, yh, N, D, VPT, s); break;
                default: launch_reg<1024>(xh, yh, N, D, VPT, s); break;
            }
            return launch_status();
        }
        const int64_t want = ceil_div(D, vec ? 8 : 1);
        const int threads = static_cast<int>(ceil_div(want < 1024 ? want : 1024, kWave) * kWave);
        if (vec)
            softmax_row_kernel<8><<<dim3(static_cast<unsigned>(N)), dim3(threads), 0, s>>>(xh, yh, D);
        else
            softmax_row_kernel<1><<<dim3(static_cast<unsigned>(N)), dim3(threads), 0, s>>>(xh, yh, D);
        return launch_status();
    }
    if (onelaunch) {
        const int u = onelaunch_u(N, D);
        const OneLaunchGrid g = onelaunch_grid(N, D, false);
        auto* rec = static_cast<unsigned char*>(ws);
        if (u == kOnePassU)
            softmax_stream_kernel<kOnePassU, false><<<dim3(g.blocks()), dim3(256), 0, s>>>(
                xh, yh, rec, N, D, g_poll_limit.load(), nullptr, g.splits, g.R, g.local);
        else
            softmax_stream_kernel<kOnePassU / 2, false><<<dim3(g.blocks()), dim3(256), 0, s>>>(
                xh, yh, rec, N, D, g_poll_limit.load(), nullptr, g.splits, g.R, g.local);
        return launch_status();
    }
    auto* part = reinterpret_cast<float*>(static_cast<unsigned char*>(ws) +
                                          (layout == Ws::kRecordsThenPairs ? kOnePassRegion : 0));
    const dim3 g(static_cast<unsigned>(splits), static_cast<unsigned>(N));
    if (vec) {
        if (split_tile(N, D) == 4096)
            softmax_partial_kernel<8, 2><<<g, dim3(256), 0, s>>>(xh, part, D, chunk);
        else
            softmax_partial_kernel<8, 1><<<g, dim3(256), 0, s>>>(xh, part, D, chunk);
        softmax_finish_kernel<8><<<g, dim3(256), 0, s>>>(xh, yh, part, D, chunk);
    } else {
        softmax_partial_kernel<1, 1><<<g, dim3(256), 0, s>>>(xh, part, D, chunk);
        softmax_finish_kernel<1><<<g, dim3(256), 0, s>>>(xh, yh, part, D, chunk);
    }
    return launch_status();
}

// ---------------------------------------------------------------------------
// Allocation-free entry (mi_softmax_noalloc_f16): the same plans and kernels
// as mi_softmax_ws_f16, with the workspace taken from a file-scope device
// array (`scratch`, below) instead of the caller or the runtime.  Its host
// address comes from hipGetSymbolAddress once per device; it is zero from
// the library's load (the row records must start at zero) and then left to
// each call, which leaves it valid for the next.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocPairBytes = 256 * 1024;  // two-pass (max, sum) pairs
constexpr int64_t kScratchBytes = kOnePassRegion + kNoAllocPairBytes;

}  // namespace
}  // namespace mi

// 2,424,832 bytes per GPU, held from the library's load until the process
// ends.  Host code never passes this name to a kernel or a copy: it is a
// host-side stand-in; the device address comes from hipGetSymbolAddress.
// It starts at zero, as the row records must: an object of static storage
// with no initializer is zero-initialized, and in the code object it is
// .bss, which the loader zero-fills on each device when it loads the code.
static __device__ __align__(256) unsigned char scratch[mi::kScratchBytes];

namespace mi {
namespace {

// This device's address of `scratch` (nullptr with *err set when the
// runtime cannot give it), looked up on the device's first call.  Nothing
// is launched here (the array is zero from load; each call leaves it valid
// for the next), so a first call under graph capture records only the
// softmax itself.
void* scratch_for_current_device(int* err) {
    static std::mutex mu;
    static std::map<int, void*> ptrs;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *err = static_cast<int>(e);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    auto it = ptrs.find(dev);
    if (it != ptrs.end()) return it->second;
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
        *err = static_cast<int>(e != hipSuccess ? e : hipErrorInvalidSymbol);
        (void)hipGetLastError();
        return nullptr;
    }
    ptrs[dev] = ptr;
    return ptr;
}

}  // namespace
}  // namespace mi

extern "C" int mi_softmax_noalloc_f16(const void* x, void* y, int64_t N, int64_t D,
                                      void* stream) {
    if (N < 0 || D < 0) return MI_ERR_INVALID_ARGUMENT;
    if (N == 0 || D == 0) return MI_OK;
    if (!x || !y) return MI_ERR_INVALID_ARGUMENT;
    const int64_t need = mi::workspace_bytes(N, D);
    if (need > mi::kScratchBytes) return MI_ERR_UNSUPPORTED;  // beyond the array
    if (need == 0)
        return mi::softmax_checked(x, y, N, D, nullptr, 0, mi::Ws::kRecordsThenPairs, stream);
    int err = MI_OK;
    void* ptr = mi::scratch_for_current_device(&err);
    if (!ptr) return err;
    return mi::softmax_checked(x, y, N, D, ptr, mi::kScratchBytes, mi::Ws::kRecordsThenPairs,
                               stream);
}

extern "C" int64_t mi_softmax_workspace_bytes(int64_t N, int64_t D) {
    if (N <= 0 || D <= 0) return 0;
    return mi::workspace_bytes(N, D);
}

extern "C" int mi_softmax_ws_f16(const void* x, void* y, int64_t N, int64_t D, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
    return mi::softmax_checked(x, y, N, D, workspace, workspace_bytes,
                               mi::Ws::kRecordsThenPairs, stream);
}

// Fused softmax + greedy argmax: [fused row records | softmax workspace |
// argmax workspace]; the one-launch fused kernel when the shape takes the
// one-launch softmax, else the two entry points in turn on their parts.
namespace {
constexpr int64_t kFusedRegion = mi::kSplitMaxRows * mi::kRowRecordBytesAM;
}

extern "C" int64_t mi_softmax_argmax_workspace_bytes(int64_t N, int64_t V) {
    if (N <= 0 || V <= 0) return 0;
    return kFusedRegion + mi::workspace_bytes(N, V) + mi_greedy_argmax_workspace_bytes(N, V);
}

extern "C" int mi_softmax_argmax_ws_f16(const void* logits, void* probs, int32_t* out, int64_t N,
                                        int64_t V, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
    if (N < 0 || V < 0 || workspace_bytes < 0) return MI_ERR_INVALID_ARGUMENT;
    if (N == 0 || V == 0) return MI_OK;
    if (!logits || !probs || !out || !workspace) return MI_ERR_INVALID_ARGUMENT;
    if (N > 65535) return MI_ERR_UNSUPPORTED;  // the argmax grid's rows
    if (!mi::product_fits({N, V, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t need = mi_softmax_argmax_workspace_bytes(N, V);
    if (workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
        return MI_ERR_INVALID_ARGUMENT;
    const int64_t bytes = N * V * 2;
    if (logits != probs && mi::overlaps(logits, bytes, probs, bytes)) return MI_ERR_ALIASING;
    if (mi::overlaps(workspace, need, logits, bytes) || mi::overlaps(workspace, need, probs, bytes) ||
        mi::overlaps(out, N * 4, logits, bytes) || mi::overlaps(out, N * 4, probs, bytes) ||
        mi::overlaps(out, N * 4, workspace, need))
        return MI_ERR_ALIASING;
    auto* ws = static_cast<unsigned char*>(workspace);
    const hipStream_t s = mi::as_stream(stream);
    if (mi::onelaunch_ok(logits, probs, N, V, true)) {
        const int u = mi::onelaunch_u(N, V);
        const mi::OneLaunchGrid g = mi::onelaunch_grid(N, V, true);
        const auto* xh = static_cast<const mi::half_t*>(logits);
        auto* yh = static_cast<mi::half_t*>(probs);
        if (u == mi::kOnePassU)
            mi::softmax_stream_kernel<mi::kOnePassU, true><<<dim3(g.blocks()), dim3(256), 0, s>>>(
                xh, yh, ws, N, V, mi::g_poll_limit.load(), out, g.splits, g.R, g.local);
        else
            mi::softmax_stream_kernel<mi::kOnePassU / 2, true>
                <<<dim3(g.blocks()), dim3(256), 0, s>>>(xh, yh, ws, N, V, mi::g_poll_limit.load(),
                                                        out, g.splits, g.R, g.local);
        return mi::launch_status();
    }
    // separately: argmax first (in place, softmax would overwrite the logits)
    const int64_t sw = mi::workspace_bytes(N, V);
    unsigned char* aw = ws + kFusedRegion + sw;
    const int st = mi_greedy_argmax_ws_f16(logits, N, V, out, aw,
                                           mi_greedy_argmax_workspace_bytes(N, V), stream);
    if (st != MI_OK) return st;
    return mi_softmax_ws_f16(logits, probs, N, V, sw > 0 ? ws + kFusedRegion : nullptr, sw,
                             stream);
}

extern "C" int mi_softmax_f16(const void* x, void* y, int64_t N, int64_t D, void* stream) {
    const int64_t need = (N > 0 && D > 0) ? mi::twopass_bytes(N, D) : 0;
    const hipStream_t s = mi::as_stream(stream);
    // Long split rows on the default stream (every caller in the reference
    // passes 0): one launch, with row records the library holds for stream 0.
    if (x && y && N > 0 && D > 0 && N <= mi::kMaxGridX && mi::onelaunch_ok(x, y, N, D)) {
        void* rec = mi::default_stream_region(mi::kRegionSoftmax, mi::kOnePassRegion, s);
        if (rec)
            return mi::softmax_checked(x, y, N, D, rec, mi::kOnePassRegion, mi::Ws::kRecords,
                                       stream);
    }
    if (need == 0) return mi::softmax_checked(x, y, N, D, nullptr, 0, mi::Ws::kPairs, stream);
    if (!x || !y) return MI_ERR_INVALID_ARGUMENT;
    // Otherwise two launches with a stream-ordered workspace from the
    // device's default pool (concurrent calls on other streams get their
    // own; a fresh pool allocation is not zeroed, which the two-pass form
    // does not need).
    void* ws = nullptr;
    hipError_t e = hipMallocAsync(&ws, static_cast<size_t>(need), s);
    if (e != hipSuccess) return static_cast<int>(e);
    const int st = mi::softmax_checked(x, y, N, D, ws, need, mi::Ws::kPairs, stream);
    e = hipFreeAsync(ws, s);
    if (st != MI_OK) return st;
    return e == hipSuccess ? MI_OK : static_cast<int>(e);
}

extern "C" int mi_softmax_test_poll_limit(int limit) {
    if (limit < 0) return MI_ERR_INVALID_ARGUMENT;
    return mi::g_poll_limit.exchange(limit);
}
