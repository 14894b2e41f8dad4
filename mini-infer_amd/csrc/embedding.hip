// embedding.hip -- token-embedding gather for gfx950 (bit-exact copy).
//
// out[t, :] = table[ids[t], :] (src/kernels/model_utils_kernel.cu:45-56).
//
// Design (HBM-bound: 2 x H x 2 bytes + 8 bytes of id per token): one wave per
// token row, four rows per 256-lane workgroup.  The id is read once per wave
// into a scalar register; each lane then moves 16-byte vectors, issuing up to
// kBatch loads before the matching stores so a 7 KiB row (H = 3584) is in
// flight at once.  An id outside [0, vocab) (when vocab > 0) produces a zero
// row rather than an out-of-bounds read.
#include "mi_device.h"
#include "mi_host.h"

namespace mi {
namespace {

constexpr int kRowsPerWg = 4;
constexpr int kBatch = 8;

template <int VEC>
__global__ __launch_bounds__(256) void gather_kernel(const int64_t* __restrict__ ids,
                                                     const half_t* __restrict__ table,
                                                     half_t* __restrict__ out, int64_t T,
                                                     int64_t H, int64_t vocab) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kRowsPerWg + wave;
    if (t >= T) return;  // wave-uniform exit; no cross-lane work follows
    const int64_t id = ids[t];
    const bool valid = id >= 0 && (vocab <= 0 || id < vocab);
    const half_t* src = table + (valid ? id : 0) * H;
    half_t* dst = out + t * H;
    const int64_t nv = H / VEC;
    for (int64_t c0 = 0; c0 < nv; c0 += kWave * kBatch) {
        if constexpr (VEC == 8) {
            h8 v[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kWave + lane;
                v[j] = (valid && c < nv) ? ld8_stream(src + c * 8) : h8(0);
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kWave + lane;
                if (c < nv) st8_stream(dst + c * 8, v[j]);
            }
        } else {
            half_t v[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kWave + lane;
                v[j] = (valid && c < nv) ? src[c] : half_t(0);
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kWave + lane;
                if (c < nv) dst[c] = v[j];
            }
        }
    }
}

}  // namespace
}  // namespace mi

extern "C" int mi_embedding_gather_f16(const int64_t* ids, const void* table, void* out, int64_t T,
                                       int64_t H, int64_t vocab, void* stream) {
    if (T < 0 || H < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || H == 0) return MI_OK;
    if (!ids || !table || !out) return MI_ERR_INVALID_ARGUMENT;
    const int64_t grid = mi::ceil_div(T, mi::kRowsPerWg);
    if (grid > mi::kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (vocab > 0 && mi::overlaps(out, T * H * 2, table, vocab * H * 2)) return MI_ERR_ALIASING;
    const auto* tb = static_cast<const mi::half_t*>(table);
    auto* o = static_cast<mi::half_t*>(out);
    const hipStream_t s = mi::as_stream(stream);
    const dim3 g(static_cast<unsigned>(grid)), b(256);
    if (H % 8 == 0 && mi::aligned16(table) && mi::aligned16(out))
        mi::gather_kernel<8><<<g, b, 0, s>>>(ids, tb, o, T, H, vocab);
    else
        mi::gather_kernel<1><<<g, b, 0, s>>>(ids, tb, o, T, H, vocab);
    return mi::launch_status();
}
