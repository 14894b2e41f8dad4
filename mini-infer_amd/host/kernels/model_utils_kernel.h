// model_utils_kernel.h -- the model-chain utility launchers on the hot path,
// with the reference's signatures (src/kernels/model_utils_kernel.cuh:9-67).
#pragma once

#include <cstdint>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

// y[b * batch_stride + m * N + n] = half(y[...] + bias[n]) for
// b < batch_stride / (M * N): the QKV projections' bias, broadcast over rows.
void launch_add_bias(__half* y, const __half* bias, int M, int N, int batch_stride,
                     hipStream_t stream);

// y[i] = half(y[i] + x[i])
void launch_add_inplace(__half* y, const __half* x, int64_t n, hipStream_t s);

// out[b, s, :] = embed_table[token_ids[b, s], :]; table [V, H].  As in the
// reference, ids are not range-checked here (use the C ABI's vocab argument
// for a checked gather).
void launch_embedding_gather(const int64_t* token_ids, const __half* embed_table, __half* out,
                             int B, int S, int H, hipStream_t stream);

// y[i] = half(y[i] * scale)
void launch_scale_inplace(__half* y, float scale, int64_t n, hipStream_t stream);

// y[i] = half(y[i] * x[i])
void launch_mul_inplace(__half* y, const __half* x, int64_t n, hipStream_t stream);

// Scatter src [B, S, H_kv, D] into the paged cache [L, num_blocks, H_kv,
// block_size, D] of `layer`: token (b, s) at p = start_pos[b] + s goes to
// block block_table[b, p / block_size], slot p % block_size, when
// p < seq_len[b].  block_table / seq_len / start_pos are int32 on the GPU.
void launch_paged_kv_scatter(const __half* src, __half* cache, const int* block_table,
                             const int* seq_len, const int* start_pos, int B, int S, int layer,
                             int num_blocks, int H_kv, int D, int block_size,
                             int max_blocks_per_seq, hipStream_t stream);

// K and V together in one launch (same block table).
void launch_paged_kv_scatter_kv(const __half* k_src, const __half* v_src, __half* k_cache,
                                __half* v_cache, const int* block_table, const int* seq_len,
                                const int* start_pos, int B, int S, int layer, int num_blocks,
                                int H_kv, int D, int block_size, int max_blocks_per_seq,
                                hipStream_t stream);

// launch_paged_kv_scatter_kv with a projection bias added on the way: the
// caches receive half(k + k_bias), half(v + v_bias) (bias [H_kv * D], either
// may be null).  Replaces Qwen2's launch_add_bias of V and the two scatters.
void launch_paged_kv_scatter_kv_bias(const __half* k_src, const __half* v_src, __half* k_cache,
                                     __half* v_cache, const __half* k_bias, const __half* v_bias,
                                     const int* block_table, const int* seq_len,
                                     const int* start_pos, int B, int S, int layer,
                                     int num_blocks, int H_kv, int D, int block_size,
                                     int max_blocks_per_seq, hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
