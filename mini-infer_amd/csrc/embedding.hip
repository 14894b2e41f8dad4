// embedding.hip -- token-embedding gather for gfx950 (bit-exact copy).
//
// out[t, :] = table[ids[t], :] (src/kernels/model_utils_kernel.cu:45-56).
//
// Design (HBM-bound: 2 x H x 2 bytes + 8 bytes of id per token): 16 to 256
// lanes per token row -- the fewest that hold the row at kBatch 16-byte
// vectors per lane -- so one wave at H = 3584 or 4096, two at H = 8192, and
// two rows per wave at H = 2048.  Each lane issues its loads before the
// matching stores, so a whole row is in flight at once.  An id outside [0, vocab) (when vocab > 0) produces a zero
// row rather than an out-of-bounds read.
#include "mi_device.h"
#include "mi_host.h"

namespace mi {
namespace {

constexpr int kBatch = 8;

// kLanes lanes per token row (16 .. 256), 256 / kLanes rows per workgroup:
// a row of up to kLanes * kBatch vectors is in flight at once (one batch; a
// second batch would wait for the first one's stores to drain), and narrow
// rows share a wave instead of leaving lanes idle.
template <int VEC, int kLanes>
__global__ __launch_bounds__(256) void gather_kernel(const int64_t* __restrict__ ids,
                                                     const half_t* __restrict__ table,
                                                     half_t* __restrict__ out, int64_t T,
                                                     int64_t H, int64_t vocab) {
    int r = threadIdx.x / kLanes;  // row within the workgroup
    if constexpr (kLanes >= kWave) r = __builtin_amdgcn_readfirstlane(r);  // wave-uniform
    const int lane = threadIdx.x & (kLanes - 1);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * (256 / kLanes) + r;
    if (t >= T) return;  // no cross-lane work follows
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
                // plain loads: the rows are scattered over a table far larger than
                // the caches, and the non-temporal hint measured 66% -> 72% of peak
                // slower at T = 6064 of [152064, 3584] (16.4 -> 15.1 us)
                v[j] = (valid && c < nv) ? ld8(src + c * 8) : h8(0);
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

// Lanes per row: the fewest power of two (16 .. 256) that hold the row in
// one batch of kBatch vectors per lane.
inline int gather_lanes(int64_t nv) {
    int l = 16;
    while (l < 256 && static_cast<int64_t>(l) * kBatch < nv) l *= 2;
    return l;
}

template <int VEC>
void launch_gather(const int64_t* ids, const half_t* tb, half_t* o, int64_t T, int64_t H,
                   int64_t vocab, int L, hipStream_t s) {
    const dim3 g(static_cast<unsigned>(ceil_div(T, 256 / L))), b(256);
    switch (L) {
        case 16: gather_kernel<VEC, 16><<<g, b, 0, s>>>(ids, tb, o, T, H, vocab); break;
        case 32: gather_kernel<VEC, 32><<<g, b, 0, s>>>(ids, tb, o, T, H, vocab); break;
        case 64: gather_kernel<VEC, 64><<<g, b, 0, s>>>(ids, tb, o, T, H, vocab); break;
        case 128: gather_kernel<VEC, 128><<<g, b, 0, s>>>(ids, tb, o, T, H, vocab); break;
        default: gather_kernel<VEC, 256><<<g, b, 0, s>>>(ids, tb, o, T, H, vocab); break;
    }
}

}  // namespace
}  // namespace mi

extern "C" int mi_embedding_gather_f16(const int64_t* ids, const void* table, void* out, int64_t T,
                                       int64_t H, int64_t vocab, void* stream) {
    if (T < 0 || H < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || H == 0) return MI_OK;
    if (!ids || !table || !out) return MI_ERR_INVALID_ARGUMENT;
    const bool vec = H % 8 == 0 && mi::aligned16(table) && mi::aligned16(out);
    const int L = mi::gather_lanes(vec ? H / 8 : H);
    if (mi::ceil_div(T, 256 / L) > mi::kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (vocab > 0 && mi::overlaps(out, T * H * 2, table, vocab * H * 2)) return MI_ERR_ALIASING;
    const auto* tb = static_cast<const mi::half_t*>(table);
    auto* o = static_cast<mi::half_t*>(out);
    const hipStream_t s = mi::as_stream(stream);
    if (vec)
        mi::launch_gather<8>(ids, tb, o, T, H, vocab, L, s);
    else
        mi::launch_gather<1>(ids, tb, o, T, H, vocab, L, s);
    return mi::launch_status();
}
