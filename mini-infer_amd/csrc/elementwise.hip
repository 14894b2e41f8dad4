// elementwise.hip -- gated activations (SwiGLU, GeGLU), gelu_tanh and the
// in-place add / mul / scale used by the model chain, for gfx950.
//
// Arithmetic (fp32 math, one fp16 rounding of each output):
//   swiglu : out = half(silu(g) * u),  silu(g) = g / (1 + exp(-g))
//            (src/kernels/swiglu_kernel.cu:16-26)
//   gelu   : y = half(0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))))
//            (src/kernels/gelu_kernel.cu:23-35), evaluated as x / (1 + exp(-2u)),
//            which is the same function since 0.5 (1 + tanh(u)) = sigmoid(2u)
//   geglu  : out = half(half(gelu(g)) * u) -- the reference runs gelu then
//            mul_inplace (src/layers/mlp.cpp:282-291), rounding twice; the
//            fused pass keeps both roundings at one pass's traffic
//   add    : y = half(y + x)   (src/kernels/model_utils_kernel.cu:31-35)
//   mul    : y = half(y * x)   (:82-86)
//   scale  : y = half(y * s)   (:68-72)
//   bias   : y[b, m, n] = half(y[b, m, n] + bias[n])   (:11-20)
//
// Design (HBM-bound; 6 bytes/element for the binary ops, 4 for unary): each
// 256-lane workgroup owns a contiguous tile of kUnroll x 256 16-byte vectors
// per operand; a lane issues all of its loads before any math.  kUnroll = 1
// measured best at [6064, 18944]: 80-81% of HBM peak against 77% at 2 (and
// 74% at 4, 73% at 8 at [4096, 18944]).  Inputs and outputs are touched
// once, so loads and stores carry the non-temporal hint.  A scalar kernel takes
// the n % 8 tail and any unaligned buffer.
#include "mi_device.h"
#include "mi_host.h"

namespace mi {
namespace {

enum Op { kSwiglu = 0, kGelu = 1, kGeglu = 2, kAdd = 3, kMul = 4, kScale = 5 };

template <int OP>
__device__ __forceinline__ float apply(float a, float b, float scale) {
    if constexpr (OP == kSwiglu) return silu_mul(a, b);
    if constexpr (OP == kGelu) return gelu_tanh(a);
    // gelu rounded to fp16 before the multiply, as the reference's
    // launch_gelu_tanh + launch_mul_inplace pair stores it in between
    if constexpr (OP == kGeglu) return (float)to_half(gelu_tanh(a)) * b;
    if constexpr (OP == kAdd) return a + b;
    if constexpr (OP == kMul) return a * b;
    if constexpr (OP == kScale) return a * scale;
    return 0.0f;
}

template <int OP>
constexpr bool binary() {
    return OP == kSwiglu || OP == kGeglu || OP == kAdd || OP == kMul;
}

#ifndef MI_EW_UNROLL
#define MI_EW_UNROLL 1
#endif
constexpr int kUnroll = MI_EW_UNROLL;
constexpr int kThreads = 256;
constexpr int64_t kTileVec = kUnroll * kThreads;  // 16-byte vectors per workgroup

template <int OP>
__global__ __launch_bounds__(kThreads) void ew_vec_kernel(const half_t* a, const half_t* b,
                                                          half_t* out, int64_t nvec, float scale) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kTileVec + threadIdx.x;
    h8 va[kUnroll], vb[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
        const int64_t v = base + j * kThreads;
        if (v < nvec) {
            va[j] = ld8_stream(a + v * 8);
            if constexpr (binary<OP>()) vb[j] = ld8_stream(b + v * 8);
        }
    }
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
        const int64_t v = base + j * kThreads;
        if (v < nvec) {
            h8 o;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float bb = binary<OP>() ? (float)vb[j][k] : 0.0f;
                o[k] = to_half(apply<OP>((float)va[j][k], bb, scale));
            }
            st8_stream(out + v * 8, o);
        }
    }
}

template <int OP>
__global__ __launch_bounds__(kThreads) void ew_scalar_kernel(const half_t* a, const half_t* b,
                                                             half_t* out, int64_t begin,
                                                             int64_t n, float scale) {
    const int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const float bb = binary<OP>() ? (float)b[i] : 0.0f;
    out[i] = to_half(apply<OP>((float)a[i], bb, scale));
}

// Elementwise over n: out[i] = op(a[i], b[i]).  For the in-place ops the
// caller passes out == a.  Each element is read and written by one lane, so
// out may equal a or b.
template <int OP>
int ew_launch(const void* av, const void* bv, void* outv, int64_t n, float scale, void* stream) {
    if (n < 0) return MI_ERR_INVALID_ARGUMENT;
    if (n == 0) return MI_OK;
    if (!av || !outv || (binary<OP>() && !bv)) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({n, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t bytes = n * 2;
    if (outv != av && overlaps(outv, bytes, av, bytes)) return MI_ERR_ALIASING;
    if (binary<OP>() && outv != bv && overlaps(outv, bytes, bv, bytes)) return MI_ERR_ALIASING;

    const half_t* a = static_cast<const half_t*>(av);
    const half_t* b = static_cast<const half_t*>(bv);
    half_t* out = static_cast<half_t*>(outv);
    const hipStream_t s = as_stream(stream);

    const bool vec = aligned16(a) && aligned16(out) && (!binary<OP>() || aligned16(b));
    int64_t done = 0;
    if (vec) {
        const int64_t nvec = n / 8;
        if (nvec > 0) {
            const int64_t grid = ceil_div(nvec, kTileVec);
            if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
            ew_vec_kernel<OP><<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s>>>(
                a, b, out, nvec, scale);
            done = nvec * 8;
        }
    }
    if (done < n) {
        const int64_t grid = ceil_div(n - done, kThreads);
        if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
        ew_scalar_kernel<OP><<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s>>>(
            a, b, out, done, n, scale);
    }
    return launch_status();
}

// Broadcast bias add over rows of N: one 16-byte vector per lane, the
// batch on grid.y; bias vector = (vector index within the batch) mod (N / 8),
// read through the caches (the bias is a few KB that every row re-reads).
__global__ __launch_bounds__(kThreads) void bias_vec_kernel(half_t* y, const half_t* __restrict__ bias,
                                                            uint32_t row_vec, int64_t batch_vec,
                                                            int64_t batch_stride) {
    const int64_t v = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (v >= batch_vec) return;
    half_t* p = y + static_cast<int64_t>(blockIdx.y) * batch_stride + v * 8;
    const h8 a = ld8_stream(p);
    const h8 b = ld8(bias + (static_cast<uint32_t>(v) % row_vec) * 8);
    h8 o;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = to_half((float)a[k] + (float)b[k]);
    st8_stream(p, o);
}

__global__ __launch_bounds__(kThreads) void bias_scalar_kernel(half_t* y, const half_t* bias,
                                                               int64_t N, int64_t batch_elems,
                                                               int64_t batch_stride) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= batch_elems) return;
    half_t* p = y + static_cast<int64_t>(blockIdx.y) * batch_stride + i;
    *p = to_half((float)*p + (float)bias[i % N]);
}

// y [batches, M, N] (batches = batch_stride / (M * N), batch b at
// b * batch_stride) += bias [N], broadcast over rows.
int add_bias(void* yv, const void* biasv, int64_t M, int64_t N, int64_t batch_stride,
             void* stream) {
    if (M < 0 || N < 0 || batch_stride < 0) return MI_ERR_INVALID_ARGUMENT;
    if (M == 0) return MI_OK;  // the reference returns before launching
    if (N == 0 || !yv || !biasv) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({M, N, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({batch_stride, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t per = M * N;
    const int64_t batches = batch_stride / per;
    if (batches < 1) return MI_ERR_INVALID_ARGUMENT;  // a grid with no batch: no launch
    if (batches > 65535) return MI_ERR_UNSUPPORTED;   // grid.y
    const int64_t span = (batches - 1) * batch_stride + per;
    if (overlaps(biasv, N * 2, yv, span * 2)) return MI_ERR_ALIASING;
    auto* y = static_cast<half_t*>(yv);
    const auto* bias = static_cast<const half_t*>(biasv);
    const hipStream_t s = as_stream(stream);
    const bool vec = N % 8 == 0 && batch_stride % 8 == 0 && aligned16(y) && aligned16(bias) &&
                     per / 8 <= 0xffffffffll;
    const int64_t items = vec ? per / 8 : per;
    const int64_t grid = ceil_div(items, kThreads);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    const dim3 g(static_cast<unsigned>(grid), static_cast<unsigned>(batches));
    if (vec)
        bias_vec_kernel<<<g, dim3(kThreads), 0, s>>>(y, bias, static_cast<uint32_t>(N / 8), items,
                                                     batch_stride);
    else
        bias_scalar_kernel<<<g, dim3(kThreads), 0, s>>>(y, bias, N, items, batch_stride);
    return launch_status();
}

}  // namespace
}  // namespace mi

extern "C" int mi_add_bias_f16(void* y, const void* bias, int64_t M, int64_t N,
                               int64_t batch_stride, void* stream) {
    return mi::add_bias(y, bias, M, N, batch_stride, stream);
}

extern "C" int mi_swiglu_f16(const void* gate, const void* up, void* out, int64_t n,
                             void* stream) {
    return mi::ew_launch<mi::kSwiglu>(gate, up, out, n, 0.0f, stream);
}

extern "C" int mi_gelu_tanh_f16(const void* x, void* y, int64_t n, void* stream) {
    return mi::ew_launch<mi::kGelu>(x, nullptr, y, n, 0.0f, stream);
}

extern "C" int mi_geglu_f16(const void* gate, const void* up, void* out, int64_t n,
                            void* stream) {
    return mi::ew_launch<mi::kGeglu>(gate, up, out, n, 0.0f, stream);
}

extern "C" int mi_add_inplace_f16(void* y, const void* x, int64_t n, void* stream) {
    return mi::ew_launch<mi::kAdd>(y, x, y, n, 0.0f, stream);
}

extern "C" int mi_mul_inplace_f16(void* y, const void* x, int64_t n, void* stream) {
    return mi::ew_launch<mi::kMul>(y, x, y, n, 0.0f, stream);
}

extern "C" int mi_scale_inplace_f16(void* y, float scale, int64_t n, void* stream) {
    return mi::ew_launch<mi::kScale>(y, nullptr, y, n, scale, stream);
}
