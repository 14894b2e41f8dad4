// floors.hip -- calibration streams for the benchmark (libmi_floors.so).
//
// Kernels that move bytes and do nothing else, so a layer kernel's time can
// be set beside the time the same bytes take with no arithmetic, no
// reduction and no exchange:
//   * copy     : dst[i] = src[i]            (read n, write n, out of place)
//   * inplace  : buf[i] = buf[i] ^ pattern  (read n, write n, same address;
//                the XOR keeps the write from being a no-op store of the value
//                just read, and each call flips the buffer back and forth)
//   * read     : every word folded into a per-lane value that guards a store
//                which never fires (read n, write nothing)
//   * empty    : a one-workgroup kernel that returns at once (launch floor)
// Each stream kernel moves 16-byte vectors, VPL of them per lane per step,
// all loads of a step issued before its stores, with non-temporal stores and
// non-temporal or plain loads; a `form` also selects one workgroup per tile
// or a grid of the resident capacity walking the buffer with a grid stride,
// and stores issued back to back or each waiting for the one before it.  The
// benchmark takes the fastest of a few (VPL, persistent) forms as the floor.
// Not part of the layer-kernel library: nothing here is reached from
// include/mi_kernels.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mi_device.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ u4 ld(const u4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p); else return *p;
}
__device__ __forceinline__ void st(u4* p, u4 v) { __builtin_nontemporal_store(v, p); }

constexpr int kThreads = 256;

enum Kind { kCopy = 0, kInplace = 1, kRead = 2 };

template <int KIND, int VPL, bool NT, bool SER = false>
__global__ __launch_bounds__(kThreads) void stream_kernel(const u4* src, u4* dst, int64_t nvec,
                                                          uint32_t pattern, uint32_t* sink) {
    const int64_t tile = static_cast<int64_t>(kThreads) * VPL;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * tile;
    uint32_t acc = 0;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * tile + threadIdx.x; base < nvec;
         base += stride) {
        u4 v[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t i = base + static_cast<int64_t>(j) * kThreads;
            if (i < nvec) v[j] = ld<NT>(src + i);
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int64_t i = base + static_cast<int64_t>(j) * kThreads;
            if (i < nvec) {
                if constexpr (KIND == kCopy) st(dst + i, v[j]);
                if constexpr (SER && KIND == kCopy) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if constexpr (KIND == kInplace) st(dst + i, v[j] ^ pattern);
                if constexpr (SER && KIND == kInplace) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if constexpr (KIND == kRead) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
            }
        }
    }
    // The loaded values feed a store that a fixed pattern never triggers
    // (the buffers hold 0x01 bytes), so no load can be dropped and no lane
    // pays for a reduction.
    if constexpr (KIND == kRead)
        if (acc == pattern) sink[blockIdx.x] = acc;
}

__global__ void empty_kernel() {}

// The in-place RoPE kernels' exact grid and access pattern with no
// arithmetic: a 256-lane workgroup per token, lane j < (Hq + Hkv) * hd/16
// taking head j / (hd/16), 16-byte slice j % (hd/16), loading x[i..i+8) and
// x[h + i .. h + i + 8) of that head (h = hd/2), XOR-ing both and storing
// them back in place.  WT: write-through stores ("nt sc1") as the RoPE
// kernels use, else non-temporal stores.  SER: each store waits for the one
// before it.  PERS: a resident grid walking tokens with a stride, the next
// token's loads issued before this token's stores.
template <bool WT>
__device__ __forceinline__ void rope_shape_store(_Float16* p, u4 v) {
    if constexpr (WT) mi::st8_stream_wt(p, __builtin_bit_cast(mi::h8, v));
    else st(reinterpret_cast<u4*>(p), v);
}
template <bool WT, bool SER, bool PERS, int TPW, int CONTIG = 0>
__global__ __launch_bounds__(256) void rope_shape_kernel(_Float16* q, _Float16* k, int64_t T,
                                                         int Hq, int Hkv, int hd) {
    const int half = hd >> 1, cph = hd >> 4;
    const int tid = threadIdx.x;
    if (tid >= (Hq + Hkv) * cph) return;
    const int h = tid / cph, c = tid - h * cph;
    auto addr = [&](int64_t tok) {
        return h < Hq ? q + (tok * Hq + h) * hd + c * 8 : k + (tok * Hkv + (h - Hq)) * hd + c * 8;
    };
    if constexpr (TPW > 1 || CONTIG) {  // TPW tokens per workgroup, every load issued first
        u4 a[TPW], b[TPW];
        _Float16 *pa[TPW], *pb[TPW];
        const int qv = Hq * cph * 2;  // 16-byte vectors of a token's Q row
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            int64_t tok = static_cast<int64_t>(blockIdx.x) * TPW + t;
            tok = tok < T ? tok : T - 1;
            if (CONTIG == 2) {
                // lane j: vectors j + 256 i of the workgroup's TPW Q rows as one
                // block, then of its TPW K rows as one block
                const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TPW;
                const int nq = TPW * qv;
                const int i0 = tid + 256 * (2 * t), i1 = i0 + 256;
                pa[t] = i0 < nq ? q + t0 * Hq * hd + i0 * 8 : k + t0 * Hkv * hd + (i0 - nq) * 8;
                pb[t] = i1 < nq ? q + t0 * Hq * hd + i1 * 8 : k + t0 * Hkv * hd + (i1 - nq) * 8;
            } else if (CONTIG) {  // lane j: vectors j and j + 256 of the token's [Q | K] rows
                pa[t] = q + (tok * Hq * hd) + tid * 8;
                const int j2 = tid + 256;
                pb[t] = j2 < qv ? q + (tok * Hq * hd) + j2 * 8 : k + tok * Hkv * hd + (j2 - qv) * 8;
            } else {
                pa[t] = addr(tok);
                pb[t] = pa[t] + half;
            }
            a[t] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(pa[t]));
            b[t] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(pb[t]));
        }
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            if (static_cast<int64_t>(blockIdx.x) * TPW + t >= T) break;
            rope_shape_store<WT>(pa[t], a[t] ^ 0x3c003c00u);
            mi::store_gap<SER>();
            rope_shape_store<WT>(pb[t], b[t] ^ 0x3c003c00u);
            mi::store_gap<SER>();
        }
        return;
    }
    int64_t tok = blockIdx.x;
    _Float16* hp = addr(tok);
    u4 a = __builtin_nontemporal_load(reinterpret_cast<const u4*>(hp));
    u4 b = __builtin_nontemporal_load(reinterpret_cast<const u4*>(hp + half));
    while (true) {
        const int64_t nt = tok + gridDim.x;
        const bool more = PERS && nt < T;
        _Float16* np = hp;
        u4 na = a, nb = b;
        if (more) {
            np = addr(nt);
            na = __builtin_nontemporal_load(reinterpret_cast<const u4*>(np));
            nb = __builtin_nontemporal_load(reinterpret_cast<const u4*>(np + half));
        }
        rope_shape_store<WT>(hp, a ^ 0x3c003c00u);
        mi::store_gap<SER>();
        rope_shape_store<WT>(hp + half, b ^ 0x3c003c00u);
        mi::store_gap<SER>();
        if (!more) break;
        tok = nt;
        hp = np;
        a = na;
        b = nb;
    }
}

// RoPE-shaped in-place stream over Q [T, Hq, hd] and K [T, Hkv, hd] (fp16,
// 16-byte aligned, hd a multiple of 16, (Hq + Hkv) * hd / 16 <= 256).
// form bit 0: write-through stores (else non-temporal); bit 1: each store
// waits for the one before; bit 2: a resident grid of `form >> 8` workgroups
// per CU (0: the occupancy limit) walking the tokens; bit 3 / 4 / 6: 2 / 4 / 8
// tokens per workgroup; bit 5: the contiguous-row kernel's pattern (below).
template <bool WT, bool SER, bool PERS, int TPW = 1, int CONTIG = 0>
int rope_shape_launch(_Float16* q, _Float16* k, int64_t T, int Hq, int Hkv, int hd, int per_cu_req,
                      hipStream_t s) {
    const auto kf = rope_shape_kernel<WT, SER, PERS, TPW, CONTIG>;
    int64_t grid = (T + TPW - 1) / TPW;
    if (PERS) {
        int per_cu = 0, cus = 0, dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kf, 256, 0) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return -2;
        if (per_cu_req > 0 && per_cu_req < per_cu) per_cu = per_cu_req;
        const int64_t cap = static_cast<int64_t>(per_cu) * cus;
        if (cap > 0 && cap < grid) grid = cap;
    }
    kf<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, s>>>(q, k, T, Hq, Hkv, hd);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

template <int KIND, int VPL, bool NT, bool SER>
int launch_vpl(const void* src, void* dst, int64_t nvec, int persistent, uint32_t* sink,
               int64_t sink_words, hipStream_t s) {
    const auto k = stream_kernel<KIND, VPL, NT, SER>;
    const int64_t tiles = (nvec + kThreads * VPL - 1) / (kThreads * VPL);
    int64_t grid = tiles;
    if (persistent) {
        int per_cu = 0, cus = 0, dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kThreads, 0) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return -2;
        const int64_t cap = static_cast<int64_t>(per_cu) * cus;
        if (cap > 0 && cap < grid) grid = cap;
    }
    if (grid < 1) grid = 1;
    if (grid > 2147483647) return -2;
    if (KIND == kRead && grid > sink_words) return -1;
    k<<<dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s>>>(
        static_cast<const u4*>(src), static_cast<u4*>(dst), nvec, 0x3c003c00u, sink);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

template <int KIND, bool NT, bool SER>
int launch_nt(const void* src, void* dst, int64_t nvec, int vpl, int persistent, uint32_t* sink,
              int64_t sink_words, hipStream_t s) {
    switch (vpl) {
        case 1: return launch_vpl<KIND, 1, NT, SER>(src, dst, nvec, persistent, sink, sink_words, s);
        case 2: return launch_vpl<KIND, 2, NT, SER>(src, dst, nvec, persistent, sink, sink_words, s);
        case 4: return launch_vpl<KIND, 4, NT, SER>(src, dst, nvec, persistent, sink, sink_words, s);
        case 8: return launch_vpl<KIND, 8, NT, SER>(src, dst, nvec, persistent, sink, sink_words, s);
        default: return -1;
    }
}

// form: vpl (1, 2, 4, 8) | 16 (resident grid-stride grid) | 32 (plain loads
// instead of non-temporal ones) | 64 (each store waits for the one before)
template <int KIND>
int launch(const void* src, void* dst, int64_t bytes, int form, uint32_t* sink,
           int64_t sink_words, void* stream) {
    const int vpl = form & 15, persistent = (form >> 4) & 1, plain = (form >> 5) & 1,
              ser = (form >> 6) & 1;
    if (bytes <= 0 || bytes % 16 != 0 || !src || (KIND != kRead && !dst) ||
        (KIND == kRead && !sink))
        return -1;
    if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) return -1;
    const int64_t nvec = bytes / 16;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (ser)
        return plain ? launch_nt<KIND, false, true>(src, dst, nvec, vpl, persistent, sink, sink_words, s)
                     : launch_nt<KIND, true, true>(src, dst, nvec, vpl, persistent, sink, sink_words, s);
    return plain ? launch_nt<KIND, false, false>(src, dst, nvec, vpl, persistent, sink, sink_words, s)
                 : launch_nt<KIND, true, false>(src, dst, nvec, vpl, persistent, sink, sink_words, s);
}

}  // namespace

// Out-of-place copy of `bytes` (a multiple of 16, 16-byte aligned buffers).
extern "C" int mi_floor_copy(const void* src, void* dst, int64_t bytes, int form, void* stream) {
    return launch<kCopy>(src, dst, bytes, form, nullptr, 0, stream);
}

// In-place read-then-write of `bytes` of buf (each 32-bit word XOR-ed with
// a fixed pattern, so two calls restore it).
extern "C" int mi_floor_inplace(void* buf, int64_t bytes, int form, void* stream) {
    return launch<kInplace>(buf, buf, bytes, form, nullptr, 0, stream);
}

// Read of `bytes` of src; sink (sink_words words, at least the grid) is only
// written if the XOR of a lane's words equals the fixed pattern, which the
// benchmark's 0x01-filled buffers never give.
extern "C" int mi_floor_read(const void* src, int64_t bytes, int form, uint32_t* sink,
                             int64_t sink_words, void* stream) {
    return launch<kRead>(src, nullptr, bytes, form, sink, sink_words, stream);
}

extern "C" int mi_floor_rope_inplace(void* q, void* k, int64_t T, int64_t Hq, int64_t Hkv,
                                     int64_t hd, int form, void* stream) {
    if (T <= 0 || T > 2147483647 || Hq < 0 || Hkv < 0 || hd <= 0 || hd % 16 != 0 ||
        (Hq + Hkv) * (hd / 16) > 256 || (Hq + Hkv) * (hd / 16) < 1 || !q || (Hkv > 0 && !k))
        return -1;
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k)) & 15u) return -1;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    auto* qh = static_cast<_Float16*>(q);
    auto* kh = static_cast<_Float16*>(k);
    const int a = static_cast<int>(Hq), b = static_cast<int>(Hkv), d = static_cast<int>(hd);
    const int pc = form >> 8;
    if (form & 8) {  // bit 3: 2 tokens per workgroup; bit 4: 4 tokens (no persistence)
        switch (form & 3) {
            case 0: return rope_shape_launch<false, false, false, 2>(qh, kh, T, a, b, d, 0, s);
            case 1: return rope_shape_launch<true, false, false, 2>(qh, kh, T, a, b, d, 0, s);
            case 2: return rope_shape_launch<false, true, false, 2>(qh, kh, T, a, b, d, 0, s);
            default: return rope_shape_launch<true, true, false, 2>(qh, kh, T, a, b, d, 0, s);
        }
    }
    if (form & 32) {
        // bit 5: the contiguous-row RoPE kernel's pattern -- lane j on vectors j
        // and j + 256 of a token's [Q | K] row (512 vectors a token), paced
        // non-temporal stores, its tokens per workgroup: the fewest of 1, 2, 4,
        // 6, 8 that keep the grid within 4 workgroups per CU
        if (Hq * hd / 8 < 256 || (Hq + Hkv) * hd / 8 != 512) return -1;
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return -2;
        const int64_t target = 4 * static_cast<int64_t>(cus);
        int tpw = 8;
        for (int c : {1, 2, 4, 6, 8})
            if ((T + c - 1) / c <= target) {
                tpw = c;
                break;
            }
        switch (tpw) {
            case 1: return rope_shape_launch<false, true, false, 1, 1>(qh, kh, T, a, b, d, 0, s);
            case 2: return rope_shape_launch<false, true, false, 2, 1>(qh, kh, T, a, b, d, 0, s);
            case 4: return rope_shape_launch<false, true, false, 4, 1>(qh, kh, T, a, b, d, 0, s);
            case 6: return rope_shape_launch<false, true, false, 6, 1>(qh, kh, T, a, b, d, 0, s);
            default: return rope_shape_launch<false, true, false, 8, 1>(qh, kh, T, a, b, d, 0, s);
        }
    }
    if (form & 128) {  // bit 7: 4 tokens, flat over the workgroup's Q block, then its K block
        if (T % 4 != 0 || (Hq + Hkv) * hd / 8 != 512) return -1;
        if (form & 2)
            return rope_shape_launch<false, true, false, 4, 2>(qh, kh, T, a, b, d, 0, s);
        return rope_shape_launch<false, false, false, 4, 2>(qh, kh, T, a, b, d, 0, s);
    }
    if (form & 64) {  // bit 6: 8 tokens per workgroup
        switch (form & 3) {
            case 0: return rope_shape_launch<false, false, false, 8>(qh, kh, T, a, b, d, 0, s);
            case 1: return rope_shape_launch<true, false, false, 8>(qh, kh, T, a, b, d, 0, s);
            case 2: return rope_shape_launch<false, true, false, 8>(qh, kh, T, a, b, d, 0, s);
            default: return rope_shape_launch<true, true, false, 8>(qh, kh, T, a, b, d, 0, s);
        }
    }
    if (form & 16) {
        switch (form & 3) {
            case 0: return rope_shape_launch<false, false, false, 4>(qh, kh, T, a, b, d, 0, s);
            case 1: return rope_shape_launch<true, false, false, 4>(qh, kh, T, a, b, d, 0, s);
            case 2: return rope_shape_launch<false, true, false, 4>(qh, kh, T, a, b, d, 0, s);
            default: return rope_shape_launch<true, true, false, 4>(qh, kh, T, a, b, d, 0, s);
        }
    }
    switch (form & 7) {
        case 0: return rope_shape_launch<false, false, false>(qh, kh, T, a, b, d, pc, s);
        case 1: return rope_shape_launch<true, false, false>(qh, kh, T, a, b, d, pc, s);
        case 2: return rope_shape_launch<false, true, false>(qh, kh, T, a, b, d, pc, s);
        case 3: return rope_shape_launch<true, true, false>(qh, kh, T, a, b, d, pc, s);
        case 4: return rope_shape_launch<false, false, true>(qh, kh, T, a, b, d, pc, s);
        case 5: return rope_shape_launch<true, false, true>(qh, kh, T, a, b, d, pc, s);
        case 6: return rope_shape_launch<false, true, true>(qh, kh, T, a, b, d, pc, s);
        default: return rope_shape_launch<true, true, true>(qh, kh, T, a, b, d, pc, s);
    }
}

// The gather + input-norm pattern with no arithmetic: one wave per token
// row, four rows per 256-lane workgroup; the wave reads table row ids[t]
// (plain loads, H / 8 vectors, up to 16 per lane) and writes it to out1[t]
// and, XOR-ed, to out2[t].  H a multiple of 8, at most 8192; 16-byte
// aligned buffers.
__global__ __launch_bounds__(256) void gather2_kernel(const int64_t* __restrict__ ids,
                                                      const u4* __restrict__ table, u4* out1,
                                                      u4* out2, int64_t T, int nv) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const int64_t id = ids[t];
    u4 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (lane + 64 * i < nv) v[i] = table[id * nv + lane + 64 * i];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (lane + 64 * i < nv) st(out1 + t * nv + lane + 64 * i, v[i]);
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (lane + 64 * i < nv) st(out2 + t * nv + lane + 64 * i, v[i] ^ 0x3c003c00u);
}

extern "C" int mi_floor_gather2(const int64_t* ids, const void* table, void* out1, void* out2,
                                int64_t T, int64_t H, void* stream) {
    if (T <= 0 || H <= 0 || H % 8 != 0 || H > 8192 || !ids || !table || !out1 || !out2) return -1;
    if ((reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out1) |
         reinterpret_cast<uintptr_t>(out2)) & 15u)
        return -1;
    gather2_kernel<<<dim3(static_cast<unsigned>((T + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream)>>>(
        ids, static_cast<const u4*>(table), static_cast<u4*>(out1), static_cast<u4*>(out2), T,
        static_cast<int>(H / 8));
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// The one-launch argmax's read pattern with no arithmetic: rows of V fp16
// (V a multiple of 8192), one 256-lane workgroup per 8192-element chunk (4
// vectors per lane), the workgroups of a row either on one XCD (grouped: the
// row_exchange.h order, chunk c of row 8g + q at index g * 8 * splits + 8c +
// q) or row-major (chunk c of row r at r * splits + c).  Every word feeds a
// store that the 0x01-filled buffers never trigger.
__global__ __launch_bounds__(256) void read_rows_kernel(const u4* __restrict__ x, int64_t B,
                                                        int splits, int64_t V, int grouped,
                                                        uint32_t* sink) {
    int split, row;
    if (grouped) {
        const int per = 8 * splits;
        const int g = blockIdx.x / per, j = blockIdx.x - g * per;
        split = j / 8;
        row = g * 8 + (j - split * 8);
    } else {
        row = blockIdx.x / splits;
        split = blockIdx.x - row * splits;
    }
    if (row >= B) return;
    const u4* p = x + (row * V + static_cast<int64_t>(split) * 8192) / 8 + threadIdx.x;
    u4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = __builtin_nontemporal_load(p + j * 256);
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    if (acc == 0x3c003c00u) sink[blockIdx.x] = acc;
}

extern "C" int mi_floor_read_rows(const void* x, int64_t B, int64_t V, int grouped,
                                  uint32_t* sink, int64_t sink_words, void* stream) {
    if (B <= 0 || V <= 0 || V % 8192 != 0 || !x || !sink) return -1;
    const int64_t splits = V / 8192;
    const int64_t rows = grouped ? (B + 7) / 8 * 8 : B;
    if (splits * rows > sink_words) return -1;
    read_rows_kernel<<<dim3(static_cast<unsigned>(splits * rows)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<const u4*>(x), B, static_cast<int>(splits), V, grouped, sink);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// An empty one-workgroup launch.
extern "C" int mi_floor_empty(void* stream) {
    empty_kernel<<<dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream)>>>();
    return hipGetLastError() == hipSuccess ? 0 : 1;
}
