// kv_argmax.hip -- the two steps either side of the layer chain: scattering
// the rotated K / V into the paged KV cache, and greedy (argmax) sampling
// over the LM-head logits.  Both are HBM-bound with no arithmetic to speak of.
//
// Paged KV scatter (src/kernels/model_utils_kernel.cu:108-164): token (b, s)
// of src [B, S, H_kv, D] sits at global position p = start_pos[b] + s and,
// if p < seq_len[b], is copied to block block_table[b, p / BS], slot p % BS
// of the cache laid out [L, num_blocks, H_kv, BS, D].  Bit-exact copy.  One
// wave per token moves its H_kv * D halves as 16-byte vectors (H_kv = 4,
// D = 128: 64 vectors = one per lane; a token of 32 or fewer vectors shares
// its wave with others, e.g. 4 tokens per wave for one KV head of 128).  The
// source loads are issued first:
// they depend only on the token, while the destination takes two dependent
// lookups (start_pos / seq_len, then the block table; wave-uniform).
// Entries that would leave the cache (block index past max_blocks_per_seq,
// physical block outside [0, num_blocks)) are skipped, where the reference
// would write out of bounds.  A K+V form moves both tensors in one launch.
//
// Greedy argmax (src/kernels/sampling_kernel.cu:14-38, :52-76): the reference
// lets each of 256 threads keep its first strict maximum over a stride-256
// slice (thread u = i mod 256), then tree-reduces pairs (t, t + offset) for
// offset = 128 .. 1, keeping the lower slot on ties.  Slot t at offset o holds
// the best of the threads congruent to t mod 2o, so among tied threads the
// one whose index has the smallest 8-bit bit reversal wins (low bits decide
// first).  NaN is never chosen (comparisons are false); only values above
// -inf are (the result is -1 when none is); -0 and +0 compare equal.  Here
// that order is one 64-bit key per element --
//   [ordered fp16 value : 16 | 255 - bitrev8(i mod 256) : 16 | ~i : 32]
// -- larger is better, 0 = not eligible, so any reduction order gives the
// reference's answer.  Few long rows are split into chunks.  With row records
// (a caller workspace, or on stream 0 a region the library holds) one launch:
// every chunk publishes its best key to its row's record and chunk 0 combines
// them.  Otherwise two: kernel 1 writes each chunk's best key, kernel 2
// reduces a row's keys in one wave.
#include <atomic>

#include "argmax_key.h"
#include "mi_device.h"
#include "mi_host.h"
#include "row_exchange.h"

// KV stores: plain non-temporal (1 = write-through "nt sc1"; measured neutral).
#ifndef MI_WT_KV
#define MI_WT_KV 0
#endif

namespace mi {
namespace {

// ---------------------------------------------------------------------------
// Paged KV scatter
// ---------------------------------------------------------------------------

struct KvGeometry {
    int64_t B, S;
    int64_t layer, num_blocks, H_kv, D, block_size, max_blocks_per_seq;
};

// 16-byte vectors (streamed) or single elements.
template <int VEC>
struct HVecKv;
// MI_SER_KV: each store waits for the one before it (measured 6.05 ->
// 5.68 us for K + V at T = 6064, [4, 128] heads: the writes trickle behind
// the reads instead of queueing with them).
#ifndef MI_SER_KV
#define MI_SER_KV 1
#endif
template <>
struct HVecKv<8> {
    typedef h8 T;
    __device__ static T load(const half_t* p) { return ld8_stream(p); }
    __device__ static void store(half_t* p, T v) {
        st8_out<MI_WT_KV>(p, v);
        store_gap<MI_SER_KV>();
    }
};
template <>
struct HVecKv<1> {
    typedef half_t T;
    __device__ static T load(const half_t* p) { return *p; }
    __device__ static void store(half_t* p, T v) { *p = v; }
};

// half(x + b) per element; the bias is a few KB every token re-reads, so
// plain loads.
template <int VEC>
__device__ __forceinline__ typename HVecKv<VEC>::T add_bias_vec(typename HVecKv<VEC>::T x,
                                                              const half_t* b) {
    if constexpr (VEC == 8) {
        const h8 bv = ld8(b);
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = to_half((float)x[k] + (float)bv[k]);
        return x;
    } else {
        return to_half((float)x + (float)*b);
    }
}

// L lanes per token (64, or 32 / 16 / 8 when a token has that few vectors,
// so a wave moves 2 / 4 / 8 tokens: one KV head of 128 is 16 vectors),
// 256 / L tokens per workgroup.  bias0 / bias1 ([H_kv * D], or null): a
// projection bias added to each source element, rounded to fp16 as the
// reference's launch_add_bias stores it (model_utils_kernel.cu:19).
template <int VEC, int L>
__global__ __launch_bounds__(256) void kv_scatter_kernel(const half_t* __restrict__ src0,
                                                         half_t* __restrict__ cache0,
                                                         const half_t* __restrict__ src1,
                                                         half_t* __restrict__ cache1,
                                                         const int* __restrict__ block_table,
                                                         const int* __restrict__ seq_len,
                                                         const int* __restrict__ start_pos,
                                                         KvGeometry g,
                                                         const half_t* __restrict__ bias0,
                                                         const half_t* __restrict__ bias1) {
    int tl = threadIdx.x / L;  // token within the workgroup
    if constexpr (L == kWave) tl = __builtin_amdgcn_readfirstlane(tl);  // wave-uniform
    const int lane = threadIdx.x & (L - 1);
    const int64_t tok = static_cast<int64_t>(blockIdx.x) * (256 / L) + tl;
    if (tok >= g.B * g.S) return;  // no cross-lane work follows
    const int64_t row = g.H_kv * g.D;               // halves per token
    const int64_t nv = row / VEC;                   // vectors per token
    const half_t* s0 = src0 + tok * row;
    const half_t* s1 = src1 ? src1 + tok * row : nullptr;
    // The source row depends only on the token: its first vectors are in
    // flight while the destination is resolved (two dependent lookups:
    // start_pos / seq_len, then the block table).  Loads of a token that
    // turns out to be skipped read valid source memory and are dropped.
    typename HVecKv<VEC>::T a0{}, c0{};
    if (lane < nv) {
        a0 = HVecKv<VEC>::load(s0 + lane * VEC);
        if (s1) c0 = HVecKv<VEC>::load(s1 + lane * VEC);
    }
    const int64_t b = tok / g.S;
    const int64_t s = tok - b * g.S;
    const int64_t pos = static_cast<int64_t>(start_pos[b]) + s;
    if (pos >= seq_len[b] || pos < 0) return;
    const int64_t blk = pos / g.block_size;
    if (blk >= g.max_blocks_per_seq) return;
    const int64_t phys = block_table[b * g.max_blocks_per_seq + blk];
    if (phys < 0 || phys >= g.num_blocks) return;
    const int64_t slot = pos - blk * g.block_size;

    const int64_t per_head = g.D / VEC;             // vectors per head
    const int64_t head_stride = g.block_size * g.D; // halves between heads in a block
    const int64_t dst_base =
        ((g.layer * g.num_blocks + phys) * g.H_kv) * head_stride + slot * g.D;
    const float inv_per_head = 1.0f / static_cast<float>(per_head);
    for (int64_t v = lane; v < nv; v += L) {
        // nv < 2^22 (checked at launch): small_div is exact
        const int64_t h = small_div(static_cast<int>(v), inv_per_head);
        const int64_t d = (v - h * per_head) * VEC;
        const int64_t dst = dst_base + h * head_stride + d;
        if (v != lane) {
            a0 = HVecKv<VEC>::load(s0 + v * VEC);
            if (s1) c0 = HVecKv<VEC>::load(s1 + v * VEC);
        }
        if (bias0) a0 = add_bias_vec<VEC>(a0, bias0 + v * VEC);
        if (bias1) c0 = add_bias_vec<VEC>(c0, bias1 + v * VEC);
        HVecKv<VEC>::store(cache0 + dst, a0);
        if (s1) HVecKv<VEC>::store(cache1 + dst, c0);
    }
}

int kv_scatter(const void* src0, void* cache0, const void* src1, void* cache1,
               const int* block_table, const int* seq_len, const int* start_pos, int64_t B,
               int64_t S, int64_t layer, int64_t num_blocks, int64_t H_kv, int64_t D,
               int64_t block_size, int64_t max_blocks_per_seq, void* stream,
               const void* bias0v = nullptr, const void* bias1v = nullptr) {
    if (B < 0 || S < 0 || layer < 0 || layer >= (int64_t{1} << 62) || num_blocks < 0 ||
        H_kv < 0 || D < 0 || block_size <= 0 || max_blocks_per_seq < 0)
        return MI_ERR_INVALID_ARGUMENT;
    if (B == 0 || S == 0 || H_kv == 0 || D == 0 || num_blocks == 0 || max_blocks_per_seq == 0)
        return MI_OK;
    if (!src0 || !cache0 || !block_table || !seq_len || !start_pos) return MI_ERR_INVALID_ARGUMENT;
    if ((src1 == nullptr) != (cache1 == nullptr)) return MI_ERR_INVALID_ARGUMENT;
    if (bias1v && !src1) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({B, S, H_kv, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({layer + 1, num_blocks, H_kv, block_size, D, 2})) return MI_ERR_INVALID_ARGUMENT;
    if (!product_fits({B, max_blocks_per_seq, 4})) return MI_ERR_INVALID_ARGUMENT;
    const int64_t tokens = B * S;
    const bool vec = D % 8 == 0 && aligned16(src0) && aligned16(cache0) &&
                     (!src1 || (aligned16(src1) && aligned16(cache1))) &&
                     (!bias0v || aligned16(bias0v)) && (!bias1v || aligned16(bias1v));
    const int64_t nv = H_kv * D / (vec ? 8 : 1);  // vectors per token
    const int L = nv > 32 ? 64 : nv > 16 ? 32 : nv > 8 ? 16 : 8;
    const int64_t grid = ceil_div(tokens, 256 / L);
    if (grid > kMaxGridX) return MI_ERR_UNSUPPORTED;
    if (H_kv * D >= (int64_t{1} << 22)) return MI_ERR_UNSUPPORTED;  // elements per token
    const int64_t src_bytes = tokens * H_kv * D * 2;
    const int64_t cache_bytes = (layer + 1) * num_blocks * H_kv * block_size * D * 2;
    if (overlaps(src0, src_bytes, cache0, cache_bytes)) return MI_ERR_ALIASING;
    if (src1 && (overlaps(src1, src_bytes, cache1, cache_bytes) ||
                 overlaps(cache0, cache_bytes, cache1, cache_bytes)))
        return MI_ERR_ALIASING;
    const int64_t bias_bytes = H_kv * D * 2;
    for (const void* bz : {bias0v, bias1v})
        if (bz && (overlaps(bz, bias_bytes, cache0, cache_bytes) ||
                   (cache1 && overlaps(bz, bias_bytes, cache1, cache_bytes))))
            return MI_ERR_ALIASING;
    const auto* bias0 = static_cast<const half_t*>(bias0v);
    const auto* bias1 = static_cast<const half_t*>(bias1v);
    const KvGeometry g{B, S, layer, num_blocks, H_kv, D, block_size, max_blocks_per_seq};
    const hipStream_t st = as_stream(stream);
    const auto* s0 = static_cast<const half_t*>(src0);
    const auto* s1 = static_cast<const half_t*>(src1);
    auto* c0 = static_cast<half_t*>(cache0);
    auto* c1 = static_cast<half_t*>(cache1);
    const dim3 gr(static_cast<unsigned>(grid)), b(256);
#define MI_KV_CASE(V, LL)                                                                      \
    kv_scatter_kernel<V, LL><<<gr, b, 0, st>>>(s0, c0, s1, c1, block_table, seq_len, start_pos, g, \
                                               bias0, bias1)
    if (vec) {
        if (L == 64) MI_KV_CASE(8, 64);
        else if (L == 32) MI_KV_CASE(8, 32);
        else if (L == 16) MI_KV_CASE(8, 16);
        else MI_KV_CASE(8, 8);
    } else {
        if (L == 64) MI_KV_CASE(1, 64);
        else if (L == 32) MI_KV_CASE(1, 32);
        else if (L == 16) MI_KV_CASE(1, 16);
        else MI_KV_CASE(1, 8);
    }
#undef MI_KV_CASE
    return launch_status();
}

// ---------------------------------------------------------------------------
// Greedy argmax
// ---------------------------------------------------------------------------
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kArgmaxSplitMaxRows = 512;
constexpr int kArgmaxMaxSplits = 1024;

// grid (splits, B).  With one split the index goes straight to `out`;
// otherwise each chunk's key goes to ws[row * splits + split].
template <int VEC, int U>
__global__ __launch_bounds__(256) void argmax_partial_kernel(const half_t* __restrict__ x,
                                                             int64_t V, int64_t chunk,
                                                             uint64_t* __restrict__ ws,
                                                             int32_t* __restrict__ out) {
    __shared__ uint64_t slots[256 / kWave];
    const int split = blockIdx.x, splits = gridDim.x;
    const int64_t row = blockIdx.y;
    const int64_t b = split * chunk;
    const int64_t e = b + chunk < V ? b + chunk : V;
    const uint64_t best = chunk_best<VEC, U>(x + row * V, b, e, slots);
    if (threadIdx.x == 0) {
        if (splits == 1)
            out[row] = key_index(best);
        else
            ws[row * splits + split] = best;
    }
}

// One wave per row: lane j folds chunks j, j + 64, ...
__global__ __launch_bounds__(256) void argmax_final_kernel(const uint64_t* __restrict__ ws,
                                                           int splits, int64_t B,
                                                           int32_t* __restrict__ out) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (row >= B) return;  // wave-uniform
    uint64_t k = 0;
    for (int j = lane; j < splits; j += kWave) k = max_u64(k, ws[row * splits + j]);
    k = wave_max_u64(k);
    if (lane == 0) out[row] = key_index(k);
}

// Few long rows are cut into chunks of whole tiles: aim at ~2048 workgroups
// (a 19.5 MB read-and-reduce measured flat at 5.0-5.5 us for 1216 to 4800
// workgroups and slower below), chunk = the nearest whole number of tiles.
// Tiles of 4096 elements (two vectors per lane) when that still gives >= 1024
// workgroups, else 2048.
int argmax_tile(int64_t B, int64_t V) {
    return B * ceil_div(V, 4096) >= 1024 ? 4096 : 2048;
}

int64_t argmax_splits(int64_t B, int64_t V, int64_t& chunk) {
    chunk = V;
    if (B >= kArgmaxSplitMaxRows || V < 8192) return 1;
    const int64_t tile = argmax_tile(B, V);
    int64_t sp = ceil_div(2048, B);
    if (sp > kArgmaxMaxSplits) sp = kArgmaxMaxSplits;
    int64_t tiles = (ceil_div(V, sp) + tile / 2) / tile;  // nearest whole number of tiles
    if (tiles < 1) tiles = 1;
    chunk = tiles * tile;
    return ceil_div(V, chunk);
}

// ---------------------------------------------------------------------------
// One-launch split rows (mi_greedy_argmax_ws_f16): every chunk workgroup
// publishes its best key to a fixed per-row record and exits; only chunk 0
// of each row waits, polls the row's records, and writes the index.  The
// record scheme is the one-launch softmax's with a single round and a single
// slot set (64-bit epoch E, slots tagged with the low 32 bits of E + 1;
// chunk 0 raises the epoch to E + 1 once it has seen every slot; a poll that
// runs out makes chunk 0 scan the whole row itself and raise it to E + 2).  A key
// travels as two 64-bit words {tag << 32 | key >> 32}, {tag << 32 | key
// & 0xffffffff}, each stored and loaded whole, into the row's slots in the
// XCD's L2 and into their device-scope mirror (row_exchange.h; the 1-D grid
// keeps a row's chunks on one XCD).  The workspace must be zero before its
// first use.
// ---------------------------------------------------------------------------
constexpr int kArgmaxOnePassMaxSplits = 64;
#ifndef MI_ARGMAX_ONEPASS_U
#define MI_ARGMAX_ONEPASS_U 4
#endif
constexpr int kArgmaxOnePassU = MI_ARGMAX_ONEPASS_U;             // vectors per lane
constexpr int64_t kArgmaxOnePassChunk = 2048 * kArgmaxOnePassU;  // elements per workgroup
// 128-byte epoch header, the slots, their mirror
constexpr int64_t kArgmaxRecordBytes = kRecordHeaderBytes + 2 * kArgmaxOnePassMaxSplits * 16;
constexpr int64_t kArgmaxMirror = 2 * kArgmaxOnePassMaxSplits;  // words from a slot to its mirror
constexpr int64_t kArgmaxRecordRegion = kArgmaxSplitMaxRows * kArgmaxRecordBytes;
constexpr int kArgmaxPollLimit = 1 << 16;
std::atomic<int> g_argmax_poll_limit{kArgmaxPollLimit};  // mi_greedy_argmax_test_poll_limit

// One phase of chunk 0's polls (LOCAL: the L2 copy, else the mirror) of
// `set` (workgroup-uniform; lane j < splits reads slot j) until every slot
// carries `tag`, `it` reaches poll_limit or the clock passes t0 + ticks; k:
// the lane's key.  Returns whether every slot was seen.
template <bool LOCAL>
__device__ __forceinline__ bool argmax_poll(const uint64_t* set, int splits, uint32_t tag, int& it,
                                            int poll_limit, uint64_t t0, uint64_t ticks,
                                            uint64_t& k) {
    const int lane = threadIdx.x & (kWave - 1);
    for (; it < poll_limit; ++it) {
        if (it > 0 && __builtin_amdgcn_s_memrealtime() - t0 > ticks) return false;
        bool mine = true;
        k = 0;
        if (lane < splits) {
            uint64_t w[2];
            load_slot<LOCAL, 2>(set, static_cast<uint32_t>(lane) * 16, w);
            mine = static_cast<uint32_t>(w[0] >> 32) == tag && static_cast<uint32_t>(w[1] >> 32) == tag;
            k = (w[0] << 32) | (w[1] & 0xffffffffu);
        }
        if (__all(mine)) return true;
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

__global__ __launch_bounds__(256) void argmax_onepass_kernel(const half_t* __restrict__ x,
                                                             int64_t V, unsigned char* ws,
                                                             int32_t* __restrict__ out,
                                                             int poll_limit, int64_t B,
                                                             int splits, int local) {
    __shared__ uint64_t slots[256 / kWave];
    __shared__ int fallback_sh;
    // 1-D grid of splits x (B rounded up to kXcds): a row's chunks share one
    // XCD (row_exchange.h); rows past B - 1 do not exist
    int split, slot_row;
    chunk_of(blockIdx.x, splits, split, slot_row);
    const int64_t row = slot_row;
    if (row >= B) return;  // workgroup-uniform, before any barrier
    unsigned char* rec = ws + row * kArgmaxRecordBytes;
    uint64_t* epoch = reinterpret_cast<uint64_t*>(rec);
    uint64_t* slot = reinterpret_cast<uint64_t*>(rec + kRecordHeaderBytes);
    const half_t* xr = x + row * V;
    const int64_t b = split * kArgmaxOnePassChunk;
    const int64_t e = b + kArgmaxOnePassChunk < V ? b + kArgmaxOnePassChunk : V;
    // The row's epoch, read by every lane (one request per wave) ahead of the
    // chunk's loads and with no branch around it, so its first wait comes at
    // the publish: a lane-0 load followed by its store to LDS made wave 0
    // wait out a memory round trip before issuing its data loads (the counter
    // is in order).  The chunk's loads are unconditional for the same reason
    // (chunk_load).  6.85 -> 6.6 us at [64, 152064].
    const uint64_t E = __hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    h8 a[kArgmaxOnePassU];
    chunk_load<kArgmaxOnePassU>(xr, b, e, a);
    const uint64_t best = chunk_best_of<kArgmaxOnePassU>(a, b, slots);  // barrier inside
    const uint32_t tag = static_cast<uint32_t>(E + 1);
    if (threadIdx.x == 0) {
        const uint64_t w0 = (static_cast<uint64_t>(tag) << 32) | (best >> 32);
        const uint64_t w1 = (static_cast<uint64_t>(tag) << 32) | (best & 0xffffffffu);
        local_store(&slot[2 * split], w0);
        local_store(&slot[2 * split + 1], w1);
        device_store(&slot[kArgmaxMirror + 2 * split], w0);
        device_store(&slot[kArgmaxMirror + 2 * split + 1], w1);
    }
    if (split != 0) return;  // whole workgroup
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        uint64_t k = 0;
        // also bounded by kPollTicks (50 us) of the 100 MHz constant clock;
        // the L2 copy for the first kLocalPollTicks, then the mirror
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        int it = 0;
        bool all = local != 0 && argmax_poll<true>(slot, splits, tag, it, poll_limit, t0,
                                                   kLocalPollTicks, k);
        if (!all)
            all = argmax_poll<false>(slot + kArgmaxMirror, splits, tag, it, poll_limit, t0, kPollTicks,
                                     k);
        if (all) {
            k = wave_max_u64(k);
            if (lane == 0) out[row] = key_index(k);
        }
        if (lane == 0) fallback_sh = all ? 0 : 1;
    }
    __syncthreads();
    const bool fallback = fallback_sh != 0;
    if (fallback) {
        // the whole row from x (slots reused after the barrier above)
        const uint64_t k = chunk_best<8, 4>(xr, 0, V, slots);
        if (threadIdx.x == 0) out[row] = key_index(k);
    }
    if (threadIdx.x == 0)
        __hip_atomic_fetch_max(epoch, fallback ? E + 2 : E + 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

// Two-launch split rows: one key per chunk.
int64_t argmax_keys_bytes(int64_t B, int64_t V) {
    int64_t chunk;
    const int64_t sp = argmax_splits(B, V, chunk);
    return sp > 1 ? B * sp * static_cast<int64_t>(sizeof(uint64_t)) : 0;
}

// mi_greedy_argmax_ws_f16's workspace for split rows: the one-launch records
// of every possible row (fixed place whatever the call's shape), then the
// two-launch keys.
int64_t argmax_ws_bytes(int64_t B, int64_t V) {
    const int64_t keys = argmax_keys_bytes(B, V);
    return keys > 0 ? kArgmaxRecordRegion + keys : 0;
}

#ifndef MI_ARGMAX_ONEPASS
#define MI_ARGMAX_ONEPASS 1
#endif
#ifndef MI_ARGMAX_ROW_U
#define MI_ARGMAX_ROW_U 4
#endif
#ifndef MI_ARGMAX_ROW_DEEP
#define MI_ARGMAX_ROW_DEEP 16384
#endif

// What a workspace handed to argmax() holds.
enum class Ws {
    kKeys,             // the two-launch keys only (allocating entry point)
    kRecordsThenKeys,  // argmax_ws_bytes() layout (mi_greedy_argmax_ws_f16)
    kRecords,          // the one-launch row records only (library-held, stream 0)
};

// Whether [B, V] runs as the one-launch split form given row records.
bool argmax_onepass_ok(const void* logits, int64_t B, int64_t V) {
    if (!MI_ARGMAX_ONEPASS || B <= 0 || V <= 0 || B > 65535 || V > 0x7fffffff) return false;
    int64_t chunk;
    return argmax_splits(B, V, chunk) > 1 && V % 16 == 0 && aligned16(logits) &&
           ceil_div(V, kArgmaxOnePassChunk) <= kArgmaxOnePassMaxSplits;
}

int argmax(const void* logits, int64_t B, int64_t V, int32_t* out, void* ws, int64_t ws_bytes,
           Ws layout, void* stream) {
    if (B < 0 || V < 0 || ws_bytes < 0) return MI_ERR_INVALID_ARGUMENT;
    if (B == 0) return MI_OK;
    if (!logits || !out) return MI_ERR_INVALID_ARGUMENT;
    if (B > 65535) return MI_ERR_UNSUPPORTED;  // grid.y
    if (V > 0x7fffffff) return MI_ERR_UNSUPPORTED;
    int64_t chunk;
    const int64_t splits = V == 0 ? 1 : argmax_splits(B, V, chunk);
    if (V == 0) chunk = 0;
    const int64_t keys = splits > 1 ? B * splits * 8 : 0;
    const bool onepass = layout != Ws::kKeys && argmax_onepass_ok(logits, B, V);
    if (layout == Ws::kRecords && keys > 0 && !onepass)
        return MI_ERR_UNSUPPORTED;  // no keys to fall back on (callers check argmax_onepass_ok)
    const int64_t need = keys == 0 ? 0
                         : layout == Ws::kKeys ? keys
                         : layout == Ws::kRecords ? kArgmaxRecordRegion
                                                  : kArgmaxRecordRegion + keys;
    if (need > 0) {
        if (!ws || ws_bytes < need) return MI_ERR_INVALID_ARGUMENT;
        if (reinterpret_cast<uintptr_t>(ws) % 16 != 0) return MI_ERR_INVALID_ARGUMENT;
        if (overlaps(ws, need, logits, B * V * 2) || overlaps(ws, need, out, B * 4))
            return MI_ERR_ALIASING;
    }
    const hipStream_t st = as_stream(stream);
    const auto* x = static_cast<const half_t*>(logits);
    const bool vec = V % 16 == 0 && aligned16(logits);
    if (onepass) {
        const int64_t sp1 = ceil_div(V, kArgmaxOnePassChunk);
        const int64_t rows = ceil_div(B, kXcds) * kXcds;  // <= kArgmaxSplitMaxRows
        argmax_onepass_kernel<<<dim3(static_cast<unsigned>(sp1 * rows)), dim3(256), 0, st>>>(
            x, V, static_cast<unsigned char*>(ws), out, g_argmax_poll_limit.load(), B,
            static_cast<int>(sp1), exchange_test_mode().load() == 0 ? 1 : 0);
        return launch_status();
    }
    auto* w = reinterpret_cast<uint64_t*>(
        static_cast<unsigned char*>(ws) +
        (layout == Ws::kRecordsThenKeys && keys > 0 ? kArgmaxRecordRegion : 0));
    const dim3 g(static_cast<unsigned>(splits), static_cast<unsigned>(B));
    const bool two = splits == 1 || argmax_tile(B, V) == 4096;
    if (vec) {
        if (splits == 1 && V >= MI_ARGMAX_ROW_DEEP)
            // whole long rows (B >= 512): 4 vectors per lane per tile (2x the
            // bytes in flight; [512, 152064] 49% -> 69%, [600, 65536] 52% -> 66%)
            argmax_partial_kernel<8, MI_ARGMAX_ROW_U><<<g, dim3(256), 0, st>>>(x, V, chunk, w, out);
        else if (two)
            argmax_partial_kernel<8, 2><<<g, dim3(256), 0, st>>>(x, V, chunk, w, out);
        else
            argmax_partial_kernel<8, 1><<<g, dim3(256), 0, st>>>(x, V, chunk, w, out);
    } else {
        argmax_partial_kernel<1, 8><<<g, dim3(256), 0, st>>>(x, V, chunk, w, out);
    }
    if (splits > 1)
        argmax_final_kernel<<<dim3(static_cast<unsigned>(ceil_div(B, 256 / kWave))), dim3(256), 0,
                              st>>>(w, static_cast<int>(splits), B, out);
    return launch_status();
}

}  // namespace
}  // namespace mi

extern "C" int mi_paged_kv_scatter_f16(const void* src, void* cache, const int* block_table,
                                       const int* seq_len, const int* start_pos, int64_t B,
                                       int64_t S, int64_t layer, int64_t num_blocks, int64_t H_kv,
                                       int64_t D, int64_t block_size, int64_t max_blocks_per_seq,
                                       void* stream) {
    return mi::kv_scatter(src, cache, nullptr, nullptr, block_table, seq_len, start_pos, B, S,
                          layer, num_blocks, H_kv, D, block_size, max_blocks_per_seq, stream);
}

extern "C" int mi_paged_kv_scatter_kv_f16(const void* k_src, const void* v_src, void* k_cache,
                                          void* v_cache, const int* block_table,
                                          const int* seq_len, const int* start_pos, int64_t B,
                                          int64_t S, int64_t layer, int64_t num_blocks,
                                          int64_t H_kv, int64_t D, int64_t block_size,
                                          int64_t max_blocks_per_seq, void* stream) {
    if (!v_src || !v_cache) return MI_ERR_INVALID_ARGUMENT;
    return mi::kv_scatter(k_src, k_cache, v_src, v_cache, block_table, seq_len, start_pos, B, S,
                          layer, num_blocks, H_kv, D, block_size, max_blocks_per_seq, stream);
}

extern "C" int mi_paged_kv_scatter_kv_bias_f16(const void* k_src, const void* v_src,
                                               void* k_cache, void* v_cache, const void* k_bias,
                                               const void* v_bias, const int* block_table,
                                               const int* seq_len, const int* start_pos,
                                               int64_t B, int64_t S, int64_t layer,
                                               int64_t num_blocks, int64_t H_kv, int64_t D,
                                               int64_t block_size, int64_t max_blocks_per_seq,
                                               void* stream) {
    if (!v_src || !v_cache) return MI_ERR_INVALID_ARGUMENT;
    return mi::kv_scatter(k_src, k_cache, v_src, v_cache, block_table, seq_len, start_pos, B, S,
                          layer, num_blocks, H_kv, D, block_size, max_blocks_per_seq, stream,
                          k_bias, v_bias);
}

extern "C" int64_t mi_greedy_argmax_workspace_bytes(int64_t B, int64_t V) {
    if (B <= 0 || V <= 0) return 0;
    return mi::argmax_ws_bytes(B, V);
}

extern "C" int mi_greedy_argmax_ws_f16(const void* logits, int64_t B, int64_t V, int32_t* out,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
    return mi::argmax(logits, B, V, out, workspace, workspace_bytes, mi::Ws::kRecordsThenKeys,
                      stream);
}

extern "C" int mi_greedy_argmax_test_poll_limit(int limit) {
    if (limit < 0) return MI_ERR_INVALID_ARGUMENT;
    return mi::g_argmax_poll_limit.exchange(limit);
}

extern "C" int mi_greedy_argmax_f16(const void* logits, int64_t B, int64_t V, int32_t* out,
                                    void* stream) {
    const int64_t need = (B > 0 && V > 0) ? mi::argmax_keys_bytes(B, V) : 0;
    if (need == 0) return mi::argmax(logits, B, V, out, nullptr, 0, mi::Ws::kKeys, stream);
    if (!logits || !out) return MI_ERR_INVALID_ARGUMENT;
    const hipStream_t s = mi::as_stream(stream);
    // Few long rows on the default stream (the reference's callers pass 0):
    // one launch, with row records the library holds for stream 0.
    if (mi::argmax_onepass_ok(logits, B, V)) {
        void* rec = mi::default_stream_region(mi::kRegionArgmax, mi::kArgmaxRecordRegion, s);
        if (rec)
            return mi::argmax(logits, B, V, out, rec, mi::kArgmaxRecordRegion, mi::Ws::kRecords,
                              stream);
    }
    // Otherwise two launches with a stream-ordered keys workspace (a fresh
    // pool allocation is not zeroed, which the two-launch form does not need).
    void* ws = nullptr;
    hipError_t e = hipMallocAsync(&ws, static_cast<size_t>(need), s);
    if (e != hipSuccess) return static_cast<int>(e);
    const int st = mi::argmax(logits, B, V, out, ws, need, mi::Ws::kKeys, stream);
    e = hipFreeAsync(ws, s);
    if (st != MI_OK) return st;
    return e == hipSuccess ? MI_OK : static_cast<int>(e);
}
