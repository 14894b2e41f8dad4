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

#ifndef MI_EMBED_RMS_WAVE
#define MI_EMBED_RMS_WAVE 1
#endif
// Tokens from which gather + input norm runs one wave per row (four rows per
// workgroup): at T = 6064 of [152064, 3584] 25.4 -> 24.1 us (2 or 8 rows per
// workgroup: 25.6 / 24.3 us); at T = 64 the one-workgroup-per-row kernel
// keeps more CUs busy (2.5 against 3.6 us).
#ifndef MI_EMBED_RMS_WAVE_MIN_T
#define MI_EMBED_RMS_WAVE_MIN_T 2048
#endif


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
                // the caches; plain loads measured 72% of peak against 66% with the
                // non-temporal hint at T = 6064 of [152064, 3584] (15.1 vs 16.4 us).
                // (The stores below each wait for the one before them -- the
                // counter is in order -- and measured faster that way: one
                // explicit wait for all loads instead took 15.3 -> 17.0 us.)
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

// ---------------------------------------------------------------------------
// Gather fused with the first layer's input RMSNorm (and Gemma's embedding
// scale): hidden[t] = half(table[ids[t]] * scale) (the gathered row itself
// when scale == 1), y[t] = rmsnorm(hidden[t]), one workgroup per token row
// held in registers -- the gathered row is written once and normalised
// from registers instead of being read back by a second launch.  The
// arithmetic is the rmsnorm kernels' (fp32 sum of squares, rsqrt,
// half(h * rrms * f(w))) applied to the fp16 hidden value.
// ---------------------------------------------------------------------------
template <int VPT>
__global__ __launch_bounds__(256) void embed_rms_kernel(const int64_t* __restrict__ ids,
                                                        const half_t* __restrict__ table,
                                                        half_t* __restrict__ hidden,
                                                        const half_t* __restrict__ w,
                                                        half_t* __restrict__ y, int64_t D,
                                                        int64_t vocab, float scale, float eps,
                                                        float w_bias) {
    __shared__ float slots[256 / kWave];
    const int64_t t = blockIdx.x;
    const int64_t id = ids[t];
    const bool valid = id >= 0 && (vocab <= 0 || id < vocab);
    const half_t* src = table + (valid ? id : 0) * D;
    const int64_t nv = D >> 3;
    h8 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = threadIdx.x + j * 256;
        // plain loads, as in gather_kernel: the rows are scattered over the table
        v[j] = (valid && c < nv) ? ld8(src + c * 8) : h8(0);
    }
    h8 wv[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = threadIdx.x + j * 256;
        wv[j] = c < nv ? ld8(w + c * 8) : h8(0);
    }
    // Every load is waited for once, here, and every vector scaled and
    // squared before the first store: with a store in flight, any later wait
    // on the (in-order) vector-memory counter would also wait for the store.
    __builtin_amdgcn_s_waitcnt(kDrainVmem);
    if (scale != 1.0f) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[j][k] = to_half((float)v[j][k] * scale);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float f = (float)v[j][k];
            ss = fmaf(f, f, ss);
        }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = threadIdx.x + j * 256;
        if (c < nv) st8_stream(hidden + t * D + c * 8, v[j]);
    }
    ss = block_sum(ss, slots);
    const float rrms = rsqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t c = threadIdx.x + j * 256;
        if (c < nv) {
            h8 o;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                o[k] = to_half((float)v[j][k] * rrms * ((float)wv[j][k] + w_bias));
            st8_stream(y + t * D + c * 8, o);
        }
    }
}

// The same, one wave per token row, RPW rows per workgroup (4).  The
// wave reproduces embed_rms_kernel's reduction bit for bit: its lane j plays
// the 256-lane kernel's lanes j, j + 64, j + 128, j + 192 (one per wave of
// that kernel), holding their vectors, forming each one's sum of squares in
// the same order, reducing each set of 64 with the same DPP pattern, and
// adding the four wave totals in slot order from 0.0f as block_sum does --
// so hidden and the normalised rows equal the one-workgroup-per-row kernel's
// (and the unfused gather + rmsnorm's) exactly.  The weight is staged in LDS
// once per workgroup (its loads issued before the table rows'; reading it from
// the L2 per row instead measured 24.1 -> 24.5 us); no barrier follows the one
// that publishes it, so each wave runs from its loads to its stores on its
// own.  (Store pacing or non-temporal table loads: 0.1-1.5 us slower.)
template <int VPT, int RPW>
__global__ __launch_bounds__(64 * RPW) void embed_rms_wave_kernel(const int64_t* __restrict__ ids,
                                                                  const half_t* __restrict__ table,
                                                                  half_t* __restrict__ hidden,
                                                                  const half_t* __restrict__ w,
                                                                  half_t* __restrict__ y, int64_t T,
                                                                  int64_t D, int64_t vocab,
                                                                  float scale, float eps,
                                                                  float w_bias) {
    constexpr int NV = 4 * VPT;           // vectors per lane: 4 virtual lanes x VPT
    constexpr int NW = 256 * VPT;         // weight vectors staged
    constexpr int PER = (NW + 64 * RPW - 1) / (64 * RPW);  // of them per lane
    __shared__ h8 wl[NW];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int64_t nv = D >> 3;
    // the weight's vectors (vector c at wl[c]), loaded before the table rows
    // Every load below is unconditional (indices clamped into range, values
    // masked afterwards): a load under a branch made the compiler wait for it
    // inside the branch, which serialised the row's loads.
    h8 wv[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int64_t c = tid + j * 64 * RPW;
        wv[j] = ld8(w + (c < nv ? c : nv - 1) * 8);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep them ahead of the table rows' loads
    const int64_t t_raw = static_cast<int64_t>(blockIdx.x) * RPW + (tid >> 6);
    const bool row_ok = t_raw < T;
    const int64_t t = __builtin_amdgcn_readfirstlane(static_cast<int>(row_ok ? t_raw : T - 1));
    const int64_t id = ids[t];
    const bool valid = id >= 0 && (vocab <= 0 || id < vocab);
    const half_t* src = table + (valid ? id : 0) * D;
    // slot (u, j): virtual lane L = lane + 64 u, its vector L + 256 j; plain
    // loads of scattered table rows, as in gather_kernel
    h8 v[NV];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t c = lane + 64 * u + j * 256;
            v[j * 4 + u] = ld8(src + (c < nv ? c : nv - 1) * 8);
        }
    }
#pragma unroll
    for (int j = 0; j < PER; ++j)
        if (NW % (64 * RPW) == 0 || tid + j * 64 * RPW < NW) wl[tid + j * 64 * RPW] = wv[j];
    __syncthreads();
    __builtin_amdgcn_s_waitcnt(kDrainVmem);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t c = lane + 64 * u + j * 256;
            if (!(valid && c < nv)) v[j * 4 + u] = h8(0);
        }
    }
    if (scale != 1.0f) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[i][k] = to_half((float)v[i][k] * scale);
        }
    }
    float ss[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        ss[u] = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float f = (float)v[j * 4 + u][k];
                ss[u] = fmaf(f, f, ss[u]);
            }
        }
    }
    if (row_ok) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t c = lane + 64 * u + j * 256;
                if (c < nv) st8_stream(hidden + t * D + c * 8, v[j * 4 + u]);
            }
        }
    }
    float tot = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) tot += group_sum<kWave>(ss[u]);
    const float rrms = rsqrtf(tot / static_cast<float>(D) + eps);
    if (!row_ok) return;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t c = lane + 64 * u + j * 256;
            if (c < nv) {
                const h8 wc = wl[c];
                h8 o;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    o[k] = to_half((float)v[j * 4 + u][k] * rrms * ((float)wc[k] + w_bias));
                st8_stream(y + t * D + c * 8, o);
            }
        }
    }
}

// Any D or alignment: one workgroup per row, two passes over the row (the
// second re-reads the hidden values this workgroup's own lanes wrote).
__global__ __launch_bounds__(256) void embed_rms_scalar_kernel(
    const int64_t* __restrict__ ids, const half_t* __restrict__ table, half_t* hidden,
    const half_t* __restrict__ w, half_t* __restrict__ y, int64_t D, int64_t vocab, float scale,
    float eps, float w_bias) {
    __shared__ float slots[256 / kWave];
    const int64_t t = blockIdx.x;
    const int64_t id = ids[t];
    const bool valid = id >= 0 && (vocab <= 0 || id < vocab);
    const half_t* src = table + (valid ? id : 0) * D;
    half_t* hr = hidden + t * D;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < D; i += 256) {
        half_t h = valid ? src[i] : half_t(0);
        if (scale != 1.0f) h = to_half((float)h * scale);
        hr[i] = h;
        const float f = (float)h;
        ss = fmaf(f, f, ss);
    }
    ss = block_sum(ss, slots);
    const float rrms = rsqrtf(ss / static_cast<float>(D) + eps);
    for (int64_t i = threadIdx.x; i < D; i += 256)
        y[t * D + i] = to_half((float)hr[i] * rrms * ((float)w[i] + w_bias));
}

}  // namespace
}  // namespace mi

extern "C" int mi_embedding_rmsnorm_f16(const int64_t* ids, const void* table, void* hidden,
                                        const void* weight, void* y, int64_t T, int64_t D,
                                        int64_t vocab, float scale, float eps, int add_one,
                                        void* stream) {
    if (T < 0 || D < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || D == 0) return MI_OK;
    if (!ids || !table || !hidden || !weight || !y) return MI_ERR_INVALID_ARGUMENT;
    if (T > mi::kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (!mi::product_fits({T, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (!mi::product_fits({vocab, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t bytes = T * D * 2;
    if (mi::overlaps(hidden, bytes, y, bytes)) return MI_ERR_ALIASING;
    if (vocab > 0 && (mi::overlaps(hidden, bytes, table, vocab * D * 2) ||
                      mi::overlaps(y, bytes, table, vocab * D * 2)))
        return MI_ERR_ALIASING;
    const auto* tb = static_cast<const mi::half_t*>(table);
    const auto* w = static_cast<const mi::half_t*>(weight);
    auto* h = static_cast<mi::half_t*>(hidden);
    auto* yo = static_cast<mi::half_t*>(y);
    const float bias = add_one ? 1.0f : -0.0f;  // -0: w + bias == w, signed zeros kept
    const hipStream_t s = mi::as_stream(stream);
    const dim3 g(static_cast<unsigned>(T)), b(256);
    const bool vec = D % 8 == 0 && mi::aligned16(table) && mi::aligned16(hidden) &&
                     mi::aligned16(weight) && mi::aligned16(y);
    const int64_t vpt = mi::ceil_div(D / 8, 256);
    if (vec && vpt <= 4 && MI_EMBED_RMS_WAVE && T >= MI_EMBED_RMS_WAVE_MIN_T) {
        constexpr int kR = 4;
        const dim3 gw(static_cast<unsigned>(mi::ceil_div(T, kR))), bw(64 * kR);
        switch (vpt) {
            case 1: mi::embed_rms_wave_kernel<1, kR><<<gw, bw, 0, s>>>(ids, tb, h, w, yo, T, D, vocab, scale, eps, bias); break;
            case 2: mi::embed_rms_wave_kernel<2, kR><<<gw, bw, 0, s>>>(ids, tb, h, w, yo, T, D, vocab, scale, eps, bias); break;
            case 3: mi::embed_rms_wave_kernel<3, kR><<<gw, bw, 0, s>>>(ids, tb, h, w, yo, T, D, vocab, scale, eps, bias); break;
            default: mi::embed_rms_wave_kernel<4, kR><<<gw, bw, 0, s>>>(ids, tb, h, w, yo, T, D, vocab, scale, eps, bias); break;
        }
    } else if (vec && vpt <= 4) {
        switch (vpt) {
            case 1: mi::embed_rms_kernel<1><<<g, b, 0, s>>>(ids, tb, h, w, yo, D, vocab, scale, eps, bias); break;
            case 2: mi::embed_rms_kernel<2><<<g, b, 0, s>>>(ids, tb, h, w, yo, D, vocab, scale, eps, bias); break;
            case 3: mi::embed_rms_kernel<3><<<g, b, 0, s>>>(ids, tb, h, w, yo, D, vocab, scale, eps, bias); break;
            default: mi::embed_rms_kernel<4><<<g, b, 0, s>>>(ids, tb, h, w, yo, D, vocab, scale, eps, bias); break;
        }
    } else {
        mi::embed_rms_scalar_kernel<<<g, b, 0, s>>>(ids, tb, h, w, yo, D, vocab, scale, eps, bias);
    }
    return mi::launch_status();
}

extern "C" int mi_embedding_gather_f16(const int64_t* ids, const void* table, void* out, int64_t T,
                                       int64_t H, int64_t vocab, void* stream) {
    if (T < 0 || H < 0) return MI_ERR_INVALID_ARGUMENT;
    if (T == 0 || H == 0) return MI_OK;
    if (!ids || !table || !out) return MI_ERR_INVALID_ARGUMENT;
    if (!mi::product_fits({T, H, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (!mi::product_fits({vocab, H, 2})) return MI_ERR_INVALID_ARGUMENT;
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
