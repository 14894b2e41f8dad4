// softmax.hip -- row softmax for gfx950, fp16 in/out, fp32 math.
//
// Arithmetic follows the reference (src/kernels/softmax_kernel.cu:26-58):
// m = max(x), S = sum(exp(x - m)), y = half(exp(x - m) * (1 / S)).
//
// Design (HBM-bound: 4 bytes/element):
//   * Each lane keeps an online (max, sum) pair over its 16-byte vectors,
//     rescaling the sum when the max grows, so statistics need ONE read of x
//     (the reference makes separate max and sum passes, then a third to write).
//   * Many rows (N >= 512): one workgroup per row; the write pass re-reads the
//     row, which the workgroup has just streamed through L2.
//   * Few long rows (the LM-head case, 64 x 152064): one workgroup per row
//     would light up 64 of 256 CUs, so each row is cut into `splits` chunks.
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
#include "mi_device.h"
#include "mi_host.h"

namespace mi {
namespace {

constexpr int kSplitMaxRows = 512;  // below this many rows, split each row
constexpr int kMaxSplits = 1024;    // chunk pairs of a row, folded by one wave
#ifndef MI_SOFTMAX_TARGET_WGS
#define MI_SOFTMAX_TARGET_WGS 2048
#endif
constexpr int64_t kSplitTargetWgs = MI_SOFTMAX_TARGET_WGS;

// Fold one loaded value group into the lane's online (m, s).
template <int VEC>
__device__ __forceinline__ void fold(const float (&v)[VEC], float& m, float& s) {
    float vm = v[0];
#pragma unroll
    for (int k = 1; k < VEC; ++k) vm = fmaxf(vm, v[k]);
    const float mn = fmaxf(m, vm);
    if (mn == -INFINITY) return;  // nothing but -inf so far
    float acc = s * fast_exp(m - mn);
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc += fast_exp(v[k] - mn);
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
#pragma unroll
        for (int j = 0; j < U; ++j) {
#pragma unroll
            for (int k = 0; k < 8; ++k) st += fast_exp((float)a[j][k] - mt);
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
                    for (int k = 0; k < 8; ++k) o[k] = to_half(fast_exp((float)h[j][k] - m) * inv);
                    st8_stream(yr + i, o);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < kStatUnroll; ++j) {
                const int64_t i = i0 + j * step;
                if (i < end) yr[i] = to_half(fast_exp((float)xr[i] - m) * inv);
            }
        }
    }
}

// Workgroup-wide merge of per-lane (m, s): max first, then rescaled sums.
__device__ __forceinline__ void block_merge(float& m, float& s, float* slots) {
    const float M = block_max(m, slots);
    const float part = (m == -INFINITY) ? 0.0f : s * fast_exp(m - M);
    __syncthreads();  // slots are reused by the sum
    s = block_sum(part, slots);
    m = M;
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

enum class Plan { kRow, kTwoPass };

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
    if (N >= kSplitMaxRows || D < 8192) return Plan::kRow;
    const int64_t tile = split_tile(N, D);
    int64_t sp = ceil_div(kSplitTargetWgs, N);
    if (sp > kMaxSplits) sp = kMaxSplits;
    int64_t tiles = (ceil_div(D, sp) + tile / 2) / tile;  // nearest whole number of tiles
    if (tiles < 1) tiles = 1;
    chunk = tiles * tile;
    splits = ceil_div(D, chunk);
    return Plan::kTwoPass;
}

// Workspace of a split plan: one (max, sum) pair per chunk.
int64_t workspace_bytes(int64_t N, int64_t D) {
    int64_t splits, chunk;
    if (plan(N, D, splits, chunk) == Plan::kRow) return 0;
    return N * splits * 2 * static_cast<int64_t>(sizeof(float));
}

int softmax_checked(const void* x, void* y, int64_t N, int64_t D, void* ws, int64_t ws_bytes,
                    void* stream) {
    if (N < 0 || D < 0 || ws_bytes < 0) return MI_ERR_INVALID_ARGUMENT;
    if (N == 0 || D == 0) return MI_OK;
    if (!x || !y) return MI_ERR_INVALID_ARGUMENT;
    if (N > kMaxGridX) return MI_ERR_UNSUPPORTED;
    const int64_t bytes = N * D * 2;
    if (x != y && overlaps(x, bytes, y, bytes)) return MI_ERR_ALIASING;
    const int64_t need = workspace_bytes(N, D);
    if (need > 0) {
        if (!ws || ws_bytes < need) return MI_ERR_INVALID_ARGUMENT;
        if (overlaps(ws, need, x, bytes) || overlaps(ws, need, y, bytes)) return MI_ERR_ALIASING;
    }
    const auto* xh = static_cast<const half_t*>(x);
    auto* yh = static_cast<half_t*>(y);
    auto* part = static_cast<float*>(ws);
    const hipStream_t s = as_stream(stream);
    const bool vec = D % 8 == 0 && aligned16(x) && aligned16(y);
    int64_t splits, chunk;
    switch (plan(N, D, splits, chunk)) {
        case Plan::kRow: {
            const int64_t want = ceil_div(D, vec ? 8 : 1);
            const int threads = static_cast<int>(ceil_div(want < 1024 ? want : 1024, kWave) * kWave);
            if (vec)
                softmax_row_kernel<8><<<dim3(static_cast<unsigned>(N)), dim3(threads), 0, s>>>(xh, yh, D);
            else
                softmax_row_kernel<1><<<dim3(static_cast<unsigned>(N)), dim3(threads), 0, s>>>(xh, yh, D);
            break;
        }
        case Plan::kTwoPass: {
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
            break;
        }
    }
    return launch_status();
}

}  // namespace
}  // namespace mi

extern "C" int64_t mi_softmax_workspace_bytes(int64_t N, int64_t D) {
    if (N <= 0 || D <= 0) return 0;
    return mi::workspace_bytes(N, D);
}

extern "C" int mi_softmax_ws_f16(const void* x, void* y, int64_t N, int64_t D, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
    return mi::softmax_checked(x, y, N, D, workspace, workspace_bytes, stream);
}

extern "C" int mi_softmax_f16(const void* x, void* y, int64_t N, int64_t D, void* stream) {
    const int64_t need = (N > 0 && D > 0) ? mi::workspace_bytes(N, D) : 0;
    if (need == 0) return mi::softmax_checked(x, y, N, D, nullptr, 0, stream);
    // Few long rows: a stream-ordered workspace from the device's default
    // pool (concurrent calls on other streams get their own).
    if (!x || !y) return MI_ERR_INVALID_ARGUMENT;
    const hipStream_t s = mi::as_stream(stream);
    void* ws = nullptr;
    hipError_t e = hipMallocAsync(&ws, static_cast<size_t>(need), s);
    if (e != hipSuccess) return static_cast<int>(e);
    const int st = mi::softmax_checked(x, y, N, D, ws, need, stream);
    e = hipFreeAsync(ws, s);
    if (st != MI_OK) return st;
    return e == hipSuccess ? MI_OK : static_cast<int>(e);
}
