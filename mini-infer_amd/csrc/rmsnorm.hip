// rmsnorm.hip -- RMSNorm, Gemma (1 + w) RMSNorm, per-head Q/K RMSNorm and
// residual-add + RMSNorm for gfx950.
//
// Arithmetic follows the reference kernel (src/kernels/rmsnorm_kernel.cu:30-67):
// fp32 sum of squares, rrms = rsqrt(sum / D + eps), y = half(x * rrms * f(w))
// with f(w) = w or 1 + w.  The fused variant first forms
// residual = half(residual + x) exactly as launch_add_inplace does
// (src/kernels/model_utils_kernel.cu:31-35) and normalises that rounded sum.
//
// Design (HBM-bound; 4 bytes/element for the plain norm, 8 for the fused one):
//   * rows stay in registers, so x is read from HBM once (the reference reads
//     it twice) and, fused, residual is read and written once;
//   * 16-byte vector accesses (8 halves per lane per access), non-temporal
//     for the streamed rows, cached for the weight every workgroup re-reads;
//   * long rows (hidden 3584): a workgroup of up to 256 lanes, each holding
//     VPT = ceil(D / 2048) vectors of the row (3584: 2 vectors, 224 busy
//     lanes; rows past 8 vectors per lane widen to 1024 lanes), takes
//     kRowsPerWg rows (1 by default; with more, every row's loads are issued
//     before the first reduction), one wave64 DPP reduction per row and ONE
//     barrier for all of them.  Measured at [8192, 3584]: 256 lanes x 2
//     vectors reach 75% of HBM peak fused and 71% plain, against 72-74% and
//     60-62% for 448 lanes x 1 vector and 74% / 70% for 192 x 3;
//   * short rows (Q/K-norm, head_dim 128): a G-lane slice of a wave owns a
//     row (G = 16 for 128), each slice takes kRowsPerGroup rows, and the
//     reduction is DPP-only: no LDS, no barrier;
//   * shapes the vector path cannot take (D % 8 != 0, unaligned pointers,
//     D > 65536) use a scalar two-pass kernel.
#include "mi_device.h"
#include "mi_host.h"

#ifndef MI_RMS_ROWS_PER_WG
#define MI_RMS_ROWS_PER_WG 1
#endif
#ifndef MI_RMS_ROWS_PER_GROUP
#define MI_RMS_ROWS_PER_GROUP 1
#endif
#ifndef MI_RMS_MAX_THREADS
#define MI_RMS_MAX_THREADS 256
#endif

// Stores of rms_small_kernel (per-head Q/K norm, in place): write-through
// ("nt sc1", st8_stream_wt) measured 1.5 points faster; the row kernels keep
// plain non-temporal stores.
#ifndef MI_WT_RMSS
#define MI_WT_RMSS 1
#endif

namespace mi {
namespace {

constexpr int kRowsPerWg = MI_RMS_ROWS_PER_WG;
constexpr int kRowsPerGroup = MI_RMS_ROWS_PER_GROUP;
constexpr int kMaxThreads = MI_RMS_MAX_THREADS;
#ifndef MI_RMS_PACK_ROWS_MAX
#define MI_RMS_PACK_ROWS_MAX 32
#endif
constexpr int64_t kPackRowsMax = MI_RMS_PACK_ROWS_MAX;

// ---------------------------------------------------------------------------
// Long rows: RPW rows per workgroup, VPT 16-byte vectors per lane per row.
// ---------------------------------------------------------------------------
// xcds > 0 (a few rows, RPW = 1): workgroup i runs on XCD i mod 8 (the
// dispatcher's round robin); only those on the first `xcds` XCDs work, taking
// rows (i / 8) * xcds + i mod 8, so the weight every row re-reads is fetched
// into `xcds` L2s instead of all eight.
template <int VPT, int RPW, bool FUSED>
__global__ __launch_bounds__(1024) void rms_row_kernel(const half_t* x, half_t* residual,
                                                       const half_t* __restrict__ w, half_t* y,
                                                       int64_t N, int64_t D, float eps,
                                                       float w_bias, int xcds) {
    __shared__ float slots[(1024 / kWave) * RPW];
    int64_t row0 = static_cast<int64_t>(blockIdx.x) * RPW;
    if (xcds > 0) {  // workgroup-uniform, before any barrier
        const int xcd = static_cast<int>(blockIdx.x & 7);
        if (xcd >= xcds) return;
        row0 = static_cast<int64_t>(blockIdx.x >> 3) * xcds + xcd;
        if (row0 >= N) return;
    }
    const int64_t chunks = D >> 3;
    const int nthr = blockDim.x;

    h8 v[RPW][VPT];
    h8 r[FUSED ? RPW : 1][VPT];
    // 1. issue every load of every row
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        const int64_t row = row0 + q;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c = threadIdx.x + static_cast<int64_t>(j) * nthr;
            const bool ok = row < N && c < chunks;
            v[q][j] = ok ? ld8_stream(x + row * D + c * 8) : h8(0);
            if constexpr (FUSED) r[q][j] = ok ? ld8_stream(residual + row * D + c * 8) : h8(0);
        }
    }
    h8 wv[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = threadIdx.x + static_cast<int64_t>(j) * nthr;
        wv[j] = c < chunks ? ld8(w + c * 8) : h8(0);
    }
    // 2. residual sums (stored back) and sums of squares
    float ss[RPW];
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        const int64_t row = row0 + q;
        ss[q] = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            if constexpr (FUSED) {
                const int64_t c = threadIdx.x + static_cast<int64_t>(j) * nthr;
#pragma unroll
                for (int k = 0; k < 8; ++k) v[q][j][k] = to_half((float)r[q][j][k] + (float)v[q][j][k]);
                if (row < N && c < chunks) st8_stream(residual + row * D + c * 8, v[q][j]);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float f = (float)v[q][j][k];
                ss[q] = fmaf(f, f, ss[q]);
            }
        }
    }
    // 3. one barrier for all rows
    block_sum_n<RPW>(ss, slots);
    // 4. normalise and write
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        const int64_t row = row0 + q;
        if (row >= N) break;
        const float rrms = rsqrtf(ss[q] / static_cast<float>(D) + eps);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int64_t c = threadIdx.x + static_cast<int64_t>(j) * nthr;
            if (c < chunks) {
                h8 o;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    o[k] = to_half((float)v[q][j][k] * rrms * ((float)wv[j][k] + w_bias));
                st8_stream(y + row * D + c * 8, o);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Short rows: a G-lane group owns a row (one 16-byte vector per lane,
// D <= 8*G); the 256/G groups of a workgroup cover a contiguous block of rows
// and each group takes RPG such blocks, all loads issued first.
// ---------------------------------------------------------------------------
template <int G, int RPG, bool FUSED>
__global__ __launch_bounds__(256) void rms_small_kernel(const half_t* x, half_t* residual,
                                                        const half_t* __restrict__ w, half_t* y,
                                                        int64_t N, int D, float eps, float w_bias) {
    constexpr int kGroups = 256 / G;
    const int lane = threadIdx.x & (G - 1);
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (kGroups * RPG) + threadIdx.x / G;
    const int chunks = D >> 3;
    const bool lane_ok = lane < chunks;

    h8 a[RPG];
    h8 r[FUSED ? RPG : 1];
#pragma unroll
    for (int q = 0; q < RPG; ++q) {
        const int64_t row = base + q * kGroups;
        const bool ok = lane_ok && row < N;
        a[q] = ok ? ld8_stream(x + row * D + lane * 8) : h8(0);
        if constexpr (FUSED) r[q] = ok ? ld8_stream(residual + row * D + lane * 8) : h8(0);
    }
    const h8 wv = lane_ok ? ld8(w + lane * 8) : h8(0);
#pragma unroll
    for (int q = 0; q < RPG; ++q) {
        const int64_t row = base + q * kGroups;
        const bool ok = lane_ok && row < N;
        if constexpr (FUSED) {
#pragma unroll
            for (int k = 0; k < 8; ++k) a[q][k] = to_half((float)r[q][k] + (float)a[q][k]);
            if (ok) st8_out<MI_WT_RMSS>(residual + row * D + lane * 8, a[q]);
        }
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float f = (float)a[q][k];
            ss = fmaf(f, f, ss);
        }
        // every lane takes part in the DPP reduction (no lane has exited)
        ss = group_sum<G>(ss);
        const float rrms = rsqrtf(ss / static_cast<float>(D) + eps);
        if (ok) {
            h8 o;
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = to_half((float)a[q][k] * rrms * ((float)wv[k] + w_bias));
            st8_out<MI_WT_RMSS>(y + row * D + lane * 8, o);
        }
    }
}

// ---------------------------------------------------------------------------
// Q and K heads in one launch (in place): the short-row kernel over the
// Nq + Nk rows of both tensors, row r < Nq from q with wq, the rest from k
// with wk -- the reference's two launch_rmsnorm calls
// (src/layers/attention.cpp:757-768) as one, saving a launch and its ramp.
// ---------------------------------------------------------------------------
template <int G, int RPG>
__global__ __launch_bounds__(256) void rms_pair_kernel(half_t* q, const half_t* __restrict__ wq,
                                                       int64_t Nq, half_t* k,
                                                       const half_t* __restrict__ wk, int64_t Nk,
                                                       int D, float eps, float w_bias) {
    constexpr int kGroups = 256 / G;
    const int lane = threadIdx.x & (G - 1);
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (kGroups * RPG) + threadIdx.x / G;
    const int chunks = D >> 3;
    const bool lane_ok = lane < chunks;
    const int64_t N = Nq + Nk;
    auto row_ptr = [&](int64_t row) { return row < Nq ? q + row * D : k + (row - Nq) * D; };

    h8 a[RPG];
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
        const int64_t row = base + j * kGroups;
        a[j] = (lane_ok && row < N) ? ld8_stream(row_ptr(row) + lane * 8) : h8(0);
    }
    const h8 wqv = lane_ok ? ld8(wq + lane * 8) : h8(0);
    const h8 wkv = lane_ok && Nk > 0 ? ld8(wk + lane * 8) : h8(0);
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
        const int64_t row = base + j * kGroups;
        const bool ok = lane_ok && row < N;
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float f = (float)a[j][e];
            ss = fmaf(f, f, ss);
        }
        ss = group_sum<G>(ss);  // every lane takes part (no lane has exited)
        const float rrms = rsqrtf(ss / static_cast<float>(D) + eps);
        if (ok) {
            const h8 wv = row < Nq ? wqv : wkv;
            h8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = to_half((float)a[j][e] * rrms * ((float)wv[e] + w_bias));
            st8_out<MI_WT_RMSS>(row_ptr(row) + lane * 8, o);
        }
    }
}

// ---------------------------------------------------------------------------
// Scalar fallback: one 256-lane workgroup per row, two passes.  Each lane
// revisits only the elements it produced in pass 1, so in-place use is safe.
// ---------------------------------------------------------------------------
template <bool FUSED>
__global__ __launch_bounds__(256) void rms_scalar_kernel(const half_t* x, half_t* residual,
                                                         const half_t* __restrict__ w, half_t* y,
                                                         int64_t D, float eps, float w_bias) {
    __shared__ float slots[256 / kWave];
    const int64_t row = blockIdx.x;
    const half_t* xr = x + row * D;
    half_t* rr = FUSED ? residual + row * D : nullptr;
    half_t* yr = y + row * D;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < D; i += blockDim.x) {
        float v = (float)xr[i];
        if constexpr (FUSED) {
            const half_t s = to_half((float)rr[i] + v);
            rr[i] = s;
            v = (float)s;
        }
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, slots);
    const float rrms = rsqrtf(ss / static_cast<float>(D) + eps);
    for (int64_t i = threadIdx.x; i < D; i += blockDim.x) {
        const float v = FUSED ? (float)rr[i] : (float)xr[i];
        yr[i] = to_half(v * rrms * ((float)w[i] + w_bias));
    }
}

template <bool FUSED>
int launch_small(const half_t* x, half_t* r, const half_t* w, half_t* y, int64_t N, int D,
                 float eps, float bias, hipStream_t s) {
    const int chunks = D >> 3;
    int G = 1;
    while (G < chunks) G <<= 1;
    const int64_t rows_per_wg = (256 / G) * kRowsPerGroup;
    const int64_t grid = ceil_div(N, rows_per_wg);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    const dim3 g(static_cast<unsigned>(grid)), b(256);
    switch (G) {
#define MI_SMALL_CASE(GG)                                                                       \
    case GG:                                                                                    \
        rms_small_kernel<GG, kRowsPerGroup, FUSED><<<g, b, 0, s>>>(x, r, w, y, N, D, eps, bias); \
        break;
        MI_SMALL_CASE(1)
        MI_SMALL_CASE(2)
        MI_SMALL_CASE(4)
        MI_SMALL_CASE(8)
        MI_SMALL_CASE(16)
        MI_SMALL_CASE(32)
        MI_SMALL_CASE(64)
#undef MI_SMALL_CASE
        default: return MI_ERR_UNSUPPORTED;
    }
    return launch_status();
}

// Vectors per lane for a row of `chunks` 16-byte vectors: kMaxThreads lanes
// while that needs at most 8 per lane, else 1024 lanes (rows <= 65536).
int row_vpt(int64_t chunks) {
    int64_t v = ceil_div(chunks, kMaxThreads);
    if (v > 8) v = ceil_div(chunks, 1024);
    return static_cast<int>(v);
}

template <int RPW, bool FUSED>
int launch_row_rpw(const half_t* x, half_t* r, const half_t* w, half_t* y, int64_t N, int64_t D,
                   float eps, float bias, hipStream_t s, int xcds = 0) {
    const int64_t chunks = D >> 3;
    const int vpt = row_vpt(chunks);
    const int threads = static_cast<int>(ceil_div(ceil_div(chunks, vpt), kWave) * kWave);
    const int64_t grid = xcds > 0 ? 8 * ceil_div(N, xcds) : ceil_div(N, RPW);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    const dim3 g(static_cast<unsigned>(grid)), b(threads);
    switch (vpt) {
#define MI_ROW_CASE(V) \
    case V: rms_row_kernel<V, RPW, FUSED><<<g, b, 0, s>>>(x, r, w, y, N, D, eps, bias, xcds); break;
        MI_ROW_CASE(1)
        MI_ROW_CASE(2)
        MI_ROW_CASE(3)
        MI_ROW_CASE(4)
        MI_ROW_CASE(5)
        MI_ROW_CASE(6)
        MI_ROW_CASE(7)
        MI_ROW_CASE(8)
#undef MI_ROW_CASE
        default: return MI_ERR_UNSUPPORTED;
    }
    return launch_status();
}

template <bool FUSED>
int launch_row(const half_t* x, half_t* r, const half_t* w, half_t* y, int64_t N, int64_t D,
               float eps, float bias, hipStream_t s) {
    // Several rows per workgroup only pay off with enough rows to fill the
    // GPU; large-VPT rows already keep many bytes in flight per lane.
    const int vpt = row_vpt(D >> 3);
    if (kRowsPerWg > 1 && vpt <= 2 && N >= 2048)
        return launch_row_rpw<kRowsPerWg, FUSED>(x, r, w, y, N, D, eps, bias, s);
    // A few rows (a decode batch): on ceil(N / 8) XCDs, eight rows each, so
    // the weight is fetched into that many L2s rather than all eight (the
    // launch is latency-bound; the extra fetches are what a counter sees).
    if (N <= kPackRowsMax)
        return launch_row_rpw<1, FUSED>(x, r, w, y, N, D, eps, bias, s,
                                        static_cast<int>(ceil_div(N, 8)));
    return launch_row_rpw<1, FUSED>(x, r, w, y, N, D, eps, bias, s);
}

template <bool FUSED>
int rmsnorm_dispatch(const void* xv, void* rv, const void* wv, void* yv, int64_t N, int64_t D,
                     float eps, int add_one, void* stream) {
    if (N < 0 || D < 0) return MI_ERR_INVALID_ARGUMENT;
    if (N == 0 || D == 0) return MI_OK;
    if (!xv || !wv || !yv || (FUSED && !rv)) return MI_ERR_INVALID_ARGUMENT;
    if (N > kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (!product_fits({N, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t bytes = N * D * 2;
    if (xv != yv && overlaps(xv, bytes, yv, bytes)) return MI_ERR_ALIASING;
    if (FUSED && (overlaps(rv, bytes, xv, bytes) || overlaps(rv, bytes, yv, bytes)))
        return MI_ERR_ALIASING;

    const half_t* x = static_cast<const half_t*>(xv);
    half_t* r = static_cast<half_t*>(rv);
    const half_t* w = static_cast<const half_t*>(wv);
    half_t* y = static_cast<half_t*>(yv);
    // -0.0f, not +0.0f: w + (-0) == w for every w including -0, so the
    // sign of a zero output follows x * rrms * w as the reference computes it
    const float bias = add_one ? 1.0f : -0.0f;
    const hipStream_t s = as_stream(stream);

    const bool vec = (D % 8 == 0) && aligned16(x) && aligned16(w) && aligned16(y) &&
                     (!FUSED || aligned16(r));
    if (vec && D <= 512) return launch_small<FUSED>(x, r, w, y, N, static_cast<int>(D), eps, bias, s);
    if (vec && D <= int64_t{8} * 1024 * 8)
        return launch_row<FUSED>(x, r, w, y, N, D, eps, bias, s);
    rms_scalar_kernel<FUSED><<<dim3(static_cast<unsigned>(N)), dim3(256), 0, s>>>(x, r, w, y, D, eps,
                                                                                  bias);
    return launch_status();
}

int qk_rmsnorm(void* qv, void* kv, const void* wqv, const void* wkv, int64_t T, int64_t Hq,
               int64_t Hkv, int64_t D, float eps, int add_one, void* stream) {
    if (T < 0 || Hq < 0 || Hkv < 0 || D < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || Hq + Hkv == 0 || D == 0) return MI_OK;
    if ((Hq > 0 && (!qv || !wqv)) || (Hkv > 0 && (!kv || !wkv))) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({T, Hq + Hkv, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t Nq = T * Hq, Nk = T * Hkv;
    if (Hq > 0 && Hkv > 0 && overlaps(qv, Nq * D * 2, kv, Nk * D * 2)) return MI_ERR_ALIASING;
    const bool vec = D % 8 == 0 && D <= 512 && (Hq == 0 || (aligned16(qv) && aligned16(wqv))) &&
                     (Hkv == 0 || (aligned16(kv) && aligned16(wkv)));
    if (!vec) {  // the general kernels, one launch per tensor
        if (Hq > 0) {
            const int st = rmsnorm_dispatch<false>(qv, nullptr, wqv, qv, Nq, D, eps, add_one, stream);
            if (st != MI_OK) return st;
        }
        return Hkv > 0 ? rmsnorm_dispatch<false>(kv, nullptr, wkv, kv, Nk, D, eps, add_one, stream)
                       : MI_OK;
    }
    // with no Q heads, K takes the Q slot
    auto* q = static_cast<half_t*>(Hq > 0 ? qv : kv);
    const auto* wq = static_cast<const half_t*>(Hq > 0 ? wqv : wkv);
    auto* k = static_cast<half_t*>(Hq > 0 ? kv : nullptr);
    const auto* wk = static_cast<const half_t*>(Hq > 0 ? wkv : nullptr);
    const int64_t n1 = Hq > 0 ? Nq : Nk, n2 = Hq > 0 ? Nk : 0;
    const int chunks = static_cast<int>(D >> 3);
    int G = 1;
    while (G < chunks) G <<= 1;
    const int64_t grid = ceil_div(n1 + n2, (256 / G) * kRowsPerGroup);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    const float bias = add_one ? 1.0f : -0.0f;  // -0: w + bias == w, signed zeros kept
    const dim3 g(static_cast<unsigned>(grid)), b(256);
    const hipStream_t s = as_stream(stream);
    const int d = static_cast<int>(D);
    switch (G) {
#define MI_PAIR_CASE(GG)                                                                         \
    case GG:                                                                                     \
        rms_pair_kernel<GG, kRowsPerGroup><<<g, b, 0, s>>>(q, wq, n1, k, wk, n2, d, eps, bias);  \
        break;
        MI_PAIR_CASE(1)
        MI_PAIR_CASE(2)
        MI_PAIR_CASE(4)
        MI_PAIR_CASE(8)
        MI_PAIR_CASE(16)
        MI_PAIR_CASE(32)
        MI_PAIR_CASE(64)
#undef MI_PAIR_CASE
        default: return MI_ERR_UNSUPPORTED;
    }
    return launch_status();
}

}  // namespace
}  // namespace mi

extern "C" int mi_qk_rmsnorm_f16(void* q, void* k, const void* q_weight, const void* k_weight,
                                 int64_t T, int64_t Hq, int64_t Hkv, int64_t head_dim, float eps,
                                 int add_one, void* stream) {
    return mi::qk_rmsnorm(q, k, q_weight, k_weight, T, Hq, Hkv, head_dim, eps, add_one, stream);
}

extern "C" int mi_rmsnorm_f16(const void* x, const void* weight, void* y, int64_t N, int64_t D,
                              float eps, int add_one, void* stream) {
    return mi::rmsnorm_dispatch<false>(x, nullptr, weight, y, N, D, eps, add_one, stream);
}

extern "C" int mi_fused_add_rmsnorm_f16(const void* x, void* residual, const void* weight, void* y,
                                        int64_t N, int64_t D, float eps, int add_one,
                                        void* stream) {
    return mi::rmsnorm_dispatch<true>(x, residual, weight, y, N, D, eps, add_one, stream);
}
