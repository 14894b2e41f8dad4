// rope_kernel.h -- RoPE launchers with the reference's signatures
// (src/kernels/rope_kernel.cuh:11-28), plus the fused positions-driven Q+K
// rotation.  All forward to the C ABI (include/mi_kernels.h) and throw
// std::runtime_error if a launch is rejected.
#pragma once

#include <cstdint>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

// NeoX RoPE: x, y [B, S, H, D] (y may equal x), cos_t / sin_t [B*S, D/2].
void launch_rope(const __half* x, const __half* cos_t, const __half* sin_t, __half* y, int B,
                 int S, int H, int D, hipStream_t stream);

// cos/sin tables [S, half] from HOST inv_freq [half] and HOST positions [S].
void launch_rope_precompute(const float* inv_freq_h, const int64_t* positions_h, __half* cos_d,
                            __half* sin_d, int S, int half, hipStream_t stream);

// cos/sin tables [B*S, half] from HOST inv_freq [half] and HOST positions [B*S].
void launch_rope_precompute_batched(const float* inv_freq_h, const int64_t* positions_h,
                                    __half* cos_d, __half* sin_d, int B, int S, int half,
                                    hipStream_t stream);

// In-place NeoX RoPE of q [T, Hq, hd] and k [T, Hkv, hd] with cos/sin made in
// registers from DEVICE positions [T] and HOST inv_freq [hd/2]: no table, no
// copy, no allocation.  k may be null when Hkv == 0.
void launch_rope_qk(__half* q, __half* k, const int64_t* positions_d, const float* inv_freq_h,
                    int T, int Hq, int Hkv, int head_dim, hipStream_t stream);

// launch_rope_qk with the QKV projection bias added first (Qwen2):
// q = rope(half(q + q_bias)), k = rope(half(k + k_bias)); q_bias [Hq * hd],
// k_bias [Hkv * hd].  Replaces two launch_add_bias calls and the RoPE pair.
void launch_bias_rope_qk(__half* q, __half* k, const __half* q_bias, const __half* k_bias,
                         const int64_t* positions_d, const float* inv_freq_h, int T, int Hq,
                         int Hkv, int head_dim, hipStream_t stream);

// Attention pre-processing of one [B, S] batch without Q/K norm, in one
// launch where the shape allows: launch_rope_qk (launch_bias_rope_qk when the
// biases are given: all three or none) on q [B*S, Hq, hd] and k [B*S, Hkv, hd],
// then the rotated k and v (+ v_bias) into k_cache / v_cache as
// launch_paged_kv_scatter_kv places them (block_table [B, max_blocks_per_seq],
// seq_len [B], start_pos [B], device).  Shapes the one-launch kernel does not
// take run as those separate launches; results are the same bit for bit.
void launch_rope_kv_scatter(__half* q, __half* k, const __half* v, const __half* q_bias,
                            const __half* k_bias, const __half* v_bias,
                            const int64_t* positions_d, const float* inv_freq_h, int B, int S,
                            int Hq, int Hkv, int head_dim, __half* k_cache, __half* v_cache,
                            const int* block_table, const int* seq_len, const int* start_pos,
                            int layer, int num_blocks, int block_size, int max_blocks_per_seq,
                            hipStream_t stream);

// launch_rope_kv_scatter for a model with Q/K norm: launch_qk_norm_rope's
// per-head RMSNorm (q_weight / k_weight [head_dim], eps, add_one) before the
// rotation, then the scatter of the rotated K and of V, one launch where the
// shape allows (else the separate launches; the same results bit for bit).
void launch_qk_norm_rope_kv_scatter(__half* q, __half* k, const __half* v,
                                    const __half* q_weight, const __half* k_weight,
                                    const int64_t* positions_d, const float* inv_freq_h, int B,
                                    int S, int Hq, int Hkv, int head_dim, float eps, int add_one,
                                    __half* k_cache, __half* v_cache, const int* block_table,
                                    const int* seq_len, const int* start_pos, int layer,
                                    int num_blocks, int block_size, int max_blocks_per_seq,
                                    hipStream_t stream);

// In place: per-head RMSNorm of q / k with q_weight / k_weight [head_dim]
// (f(w) = w, or 1 + w when add_one), rounded to fp16, then the NeoX rotation
// of launch_rope_qk -- the Q/K-norm + RoPE sequence in one pass.
// head_dim must be 16, 32, 64, 128, 256 or 512.
void launch_qk_norm_rope(__half* q, __half* k, const __half* q_weight, const __half* k_weight,
                         const int64_t* positions_d, const float* inv_freq_h, int T, int Hq,
                         int Hkv, int head_dim, float eps, int add_one, hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
