// embedding.hip -- token-embedding gather for gfx950 (bit-exact copy).
//
// out[t, :] = table[ids[t], :] (src/kernels/model_utils_kernel.cu:45-56).
//
// Design (HBM-bound: 2 x H x 2 bytes + 8 bytes of id per token): one wave per
// token row (two or four for rows of more than 512 vectors), four rows per
// 256-lane workgroup.  The id is read once per wave into a scalar register;
// each lane then moves 16-byte vectors, issuing up to kBatch loads before the
// matching stores, so a whole row (7 KiB at H = 3584, 16 KiB at H = 8192 over
// two waves) is in flight at once.  An id outside [0, vocab) (when vocab > 0) produces a zero
// row rather than an out-of-bounds read.
#include "mi_device.h"
#include "mi_host.h"

namespace mi {
namespace {

constexpr int kBatch = 8;

// W waves per token row, 4 / W rows per 256-lane workgroup: a row of up to
// W * 64 * kBatch vectors is in flight at once (one batch; a second batch
// would wait for the first one's stores to drain).
template <int VEC, int W>
__global__ __launch_bounds__(256) void gather_kernel(const int64_t* __restrict__ ids,
                                                     const half_t* __restrict__ table,
                                                     half_t* __restrict__ out, int64_t T,
                                                     int64_t H, int64_t vocab) {
    constexpr int kLanes = W * kWave;  // lanes per row
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x & (kLanes - 1);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * (4 / W) + wave / W;
    if (t >= T) return;  // wave-uniform exit; no cross-lane work follows
    const int64_t id = ids[t];
    const bool valid = id >= 0 && (vocab <= 0 || id < vocab);
    const half_t* src = table + (valid ? id : 0) * H;
    half_t* dst = out + t * H;
    const int64_t nv = H / VEC;
    for (int64_t c0 = 0; c0 < nv; c0 += kLanes * kBatch) {
        if constexpr (VEC == 8) {
            h8 v[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kLanes + lane;
                v[j] = (valid && c < nv) ? ld8_stream(src + c * 8) : h8(0);
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kLanes + lane;
                if (c < nv) st8_stream(dst + c * 8, v[j]);
            }
        } else {
            half_t v[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kLanes + lane;
                v[j] = (valid && c < nv) ? src[c] : half_t(0);
            }
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                const int64_t c = c0 + j * kLanes + lane;
                if (c < nv) dst[c] = v[j];
            }
        }
    }
}

// Waves per row: the fewest (1, 2, 4) that hold the row in one batch.
inline int gather_waves(int64_t nv) {
    return nv <= kWave * kBatch ? 1 : nv <= 2 * kWave * kBatch ? 2 : 4;
}

template <int VEC>
void launch_gather(const int64_t* ids, const half_t* tb, half_t* o, int64_t T, int64_t H,
                   int64_t vocab, int W, hipStream_t s) {
    const dim3 b(256);
    if (W == 1)
        gather_kernel<VEC, 1><<<dim3(static_cast<unsigned>(ceil_div(T, 4))), b, 0, s>>>(
            ids, tb, o, T, H, vocab);
    else if (W == 2)
        gather_kernel<VEC, 2><<<dim3(static_cast<unsigned>(ceil_div(T, 2))), b, 0, s>>>(
            ids, tb, o, T, H, vocab);
    else
        gather_kernel<VEC, 4><<<dim3(static_cast<unsigned>(T)), b, 0, s>>>(ids, tb, o, T, H,
                                                                          vocab);
}

}  // namespace
}  // namespace mi

extern "C" int mi_embedding_gather_f16(const int64_t* ids, const void* table, void* out, int64_t T,
                                       int64_t H, int64_t vocab, void* stream) {
    if (T < 0 || H < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || H == 0) return MI_OK;
    if (!ids || !table || !out) return MI_ERR_INVALID_ARGUMENT;
    const bool vec = H % 8 == 0 && mi::aligned16(table) && mi::aligned16(out);
    const int W = mi::gather_waves(vec ? H / 8 : H);
    if (mi::ceil_div(T, 4 / W) > mi::kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (vocab > 0 && mi::overlaps(out, T * H * 2, table, vocab * H * 2)) return MI_ERR_ALIASING;
    const auto* tb = static_cast<const mi::half_t*>(table);
    auto* o = static_cast<mi::half_t*>(out);
    const hipStream_t s = mi::as_stream(stream);
    if (vec)
        mi::launch_gather<8>(ids, tb, o, T, H, vocab, W, s);
    else
        mi::launch_gather<1>(ids, tb, o, T, H, vocab, W, s);
    return mi::launch_status();
}
