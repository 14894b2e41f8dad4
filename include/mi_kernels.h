/*
 * mi_kernels.h -- C ABI of the MI355X (gfx950) layer-kernel library
 * (libmi_kernels.so).
 *
 * This is the drop-in boundary for mini-infer's non-GEMM layer kernels.  The
 * reference exposes them as C++ free functions in namespace
 * mini_infer::kernels (src/kernels/<name>_kernel.cuh); each entry point below names the
 * reference function it replaces.  The C++ launch_* wrappers with the
 * reference's exact names and argument order forward to these entry points
 * (mini-infer_amd/host/kernels/).
 *
 * Conventions (all entry points):
 *   - every tensor pointer is a DEVICE pointer owned by the caller; fp16
 *     tensors are IEEE binary16, row-major, contiguous;
 *   - sizes are int64_t element counts;
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream); the
 *     call only enqueues work and returns without synchronising;
 *   - the return value is 0 on success, a negative MI_ERR_* code for an
 *     argument error (nothing is launched), or a positive hipError_t when the
 *     HIP runtime refused the launch;
 *   - a size of zero is a successful no-op;
 *   - math is fp32 with fp16 storage; outputs are rounded to nearest even.
 * No entry point allocates device memory, except mi_softmax_f16 and
 * mi_greedy_argmax_f16 on their
 * split-row path (N < 512 rows of D >= 8192), which takes 8 bytes per row
 * chunk (<= 256 KiB) from the device's stream-ordered pool (hipMallocAsync /
 * hipFreeAsync on `stream`) for the duration of the call.
 */
#ifndef MI_KERNELS_H
#define MI_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_OK 0
#define MI_ERR_INVALID_ARGUMENT (-1) /* null pointer, negative or too-large size */
#define MI_ERR_UNSUPPORTED (-2)      /* shape outside what the kernels support */
#define MI_ERR_ALIASING (-3)         /* buffers overlap where they must not */

/* Human-readable text for a status code (never NULL). */
const char* mi_status_string(int status);

/* ABI version of this header; bumped on any incompatible change. */
#define MI_KERNELS_ABI_VERSION 2
int mi_abi_version(void);

/* RMSNorm: y = x * rsqrt(sum(x^2)/D + eps) * (add_one ? 1 + w : w).
 * x, y: [N, D]; weight: [D].  y may equal x (in place, as the Q/K-norm call
 * sites do, src/layers/attention.cpp:757-768); any other overlap is an error.
 * Replaces launch_rmsnorm (src/kernels/rmsnorm_kernel.cuh:19-20). */
int mi_rmsnorm_f16(const void* x, const void* weight, void* y, int64_t N,
                   int64_t D, float eps, int add_one, void* stream);

/* Residual add fused with RMSNorm, in one pass over each row:
 *   residual = half(residual + x);  y = rmsnorm(residual).
 * Replaces the pair launch_add_inplace(residual, x) + launch_rmsnorm that the
 * model chain issues (src/model/transformer_model.cpp:608-615 and :637;
 * src/kernels/model_utils_kernel.cuh:12, rmsnorm_kernel.cuh:19).  y may equal
 * x; residual must not overlap x or y. */
int mi_fused_add_rmsnorm_f16(const void* x, void* residual, const void* weight,
                             void* y, int64_t N, int64_t D, float eps,
                             int add_one, void* stream);

/* NeoX half-rotation RoPE from per-token cos/sin tables.
 * x, y: [B, S, H, D]; cos_t, sin_t: [B*S, D/2].  y may equal x.
 * Replaces launch_rope (src/kernels/rope_kernel.cuh:11). */
int mi_rope_neox_f16(const void* x, const void* cos_t, const void* sin_t,
                     void* y, int64_t B, int64_t S, int64_t H, int64_t D,
                     void* stream);

/* Positions (the tables entry below and the two fused entries after it):
 * any int64 value.  The angle float(pos) * inv_freq[i] is an fp32 value and
 * its cos/sin are evaluated to half(RN32(exact)) for every finite fp32 angle
 * (an fp32 form up to 2^20, Cody-Waite in fp64 to 2^24, Payne-Hanek
 * reduction above), so there is no range limit and nothing for the host to
 * check in the device-resident positions. */

/* cos/sin tables [N, half] for positions the device can read (device memory,
 * or pinned host memory from hipHostMalloc written before the call):
 * cos_t[n, i] = half(cos(float(positions[n]) * inv_freq[i])), likewise sin.
 * inv_freq is a HOST array of `half` floats (<= 256), passed to the kernel by
 * value, so nothing is allocated or copied.  Device part of
 * launch_rope_precompute / launch_rope_precompute_batched
 * (src/kernels/rope_kernel.cuh:16-28), which take host positions. */
int mi_rope_tables_f16(const float* inv_freq_host, const int64_t* positions,
                       void* cos_t, void* sin_t, int64_t N, int64_t half,
                       void* stream);

/* Fused, in-place NeoX RoPE over the Q and K of T tokens with cos/sin
 * generated in registers from DEVICE positions[T] and HOST inv_freq[hd/2]:
 * q: [T, Hq, hd], k: [T, Hkv, hd] (k may be NULL when Hkv == 0).  The result
 * equals mi_rope_tables_f16 followed by mi_rope_neox_f16 on q and on k.
 * Replaces the RoPE::forward_batched pair at src/layers/attention.cpp:779-780
 * (src/layers/rope.cpp:89-131): no table round trip, no host-to-device copy,
 * no allocation. */
int mi_rope_neox_qk_f16(void* q, void* k, const int64_t* positions,
                        const float* inv_freq_host, int64_t T, int64_t Hq,
                        int64_t Hkv, int64_t head_dim, void* stream);

/* mi_rope_neox_qk_f16 with the QKV projection bias added first: q = rope(
 * half(q + q_bias)), k = rope(half(k + k_bias)), in place; q_bias [Hq * hd],
 * k_bias [Hkv * hd] (Qwen2's q_proj / k_proj bias).  Equals mi_add_bias_f16 on
 * q and on k followed by mi_rope_neox_qk_f16, bit for bit, in one pass.
 * Replaces the Qwen2 sequence at src/layers/attention.cpp:717-780 (two
 * launch_add_bias calls, src/kernels/model_utils_kernel.cuh:9, two copies and
 * two RoPE::forward_batched calls). */
int mi_bias_rope_neox_qk_f16(void* q, void* k, const void* q_bias, const void* k_bias,
                             const int64_t* positions, const float* inv_freq_host, int64_t T,
                             int64_t Hq, int64_t Hkv, int64_t head_dim, void* stream);

/* Per-head RMSNorm of Q [T, Hq, hd] and K [T, Hkv, hd] in place, one launch:
 * each head normalised with its weight (q_weight / k_weight [hd]; f(w) = w,
 * or 1 + w when add_one).  Equals mi_rmsnorm_f16 on the T*Hq Q rows and on
 * the T*Hkv K rows (k may be NULL when Hkv == 0).  Replaces the Gemma-3 pair
 * of launch_rmsnorm calls at src/layers/attention.cpp:757-768
 * (src/kernels/rmsnorm_kernel.cuh:19). */
int mi_qk_rmsnorm_f16(void* q, void* k, const void* q_weight, const void* k_weight, int64_t T,
                      int64_t Hq, int64_t Hkv, int64_t head_dim, float eps, int add_one,
                      void* stream);

/* One group of sequences in the reference's [B, S] KV-scatter layout
 * (launch_paged_kv_scatter, src/kernels/model_utils_kernel.cuh:53-63):
 * tokens [token_offset, token_offset + B*S) of the step, with int32 DEVICE
 * block_table [B, max_blocks_per_seq], seq_len [B] and start_pos [B].  (The
 * same layout as mi_chain_kv_segment in mi_chain.h.) */
typedef struct mi_kv_segment {
    int64_t token_offset;
    int64_t B, S;
    const int* block_table;
    const int* seq_len;
    const int* start_pos;
    int64_t max_blocks_per_seq;
} mi_kv_segment;

/* Attention pre-processing without Q/K norm, one launch: NeoX RoPE of
 * q [T, Hq, hd] and k [T, Hkv, hd] in place (cos/sin from DEVICE positions and
 * HOST inv_freq, as mi_rope_neox_qk_f16), and the rotated K rows and the V
 * rows [T, Hkv, hd] written into the paged caches [>= layer + 1, num_blocks,
 * Hkv, block_size, hd] for the tokens of each segment (placement and skip
 * rules of mi_paged_kv_scatter_f16).  With q_bias / k_bias / v_bias (Qwen2;
 * all three or none) each tensor gets its bias added first, rounded to fp16
 * (v itself is not written).  Equals mi_rope_neox_qk_f16 (or
 * mi_bias_rope_neox_qk_f16) followed by mi_paged_kv_scatter_kv_f16 (or its
 * bias form) per segment, bit for bit.  hd a multiple of 16 (<= 512),
 * (Hq + Hkv) * hd / 16 <= 256, Hkv * hd <= 2048, at most 8 segments over
 * disjoint token ranges, 16-byte-aligned buffers; otherwise
 * MI_ERR_UNSUPPORTED (use the separate entry points).  Replaces src/layers/attention.cpp:717-780 (bias adds,
 * copies, RoPE pair) and :823-846 (the two scatters). */
int mi_rope_kv_scatter_f16(void* q, void* k, const void* v, const void* q_bias,
                           const void* k_bias, const void* v_bias, const int64_t* positions,
                           const float* inv_freq_host, int64_t T, int64_t Hq, int64_t Hkv,
                           int64_t head_dim, void* k_cache, void* v_cache, int64_t layer,
                           int64_t num_blocks, int64_t block_size,
                           const mi_kv_segment* segments, int num_segments, void* stream);

/* mi_rope_kv_scatter_f16 for a model with Q/K norm (Gemma 3): the per-head
 * RMSNorm of mi_qk_norm_rope_f16 (q_weight / k_weight [hd], f(w) = w or
 * 1 + w when add_one, eps), then the rotation, with the normalised, rotated
 * K rows and the V rows written into the paged caches, one launch.  Equals
 * mi_qk_norm_rope_f16 followed by mi_paged_kv_scatter_kv_f16 per segment,
 * bit for bit.  head_dim one of 16, 32, 64, 128, 256, 512, and the other
 * limits of mi_rope_kv_scatter_f16; otherwise MI_ERR_UNSUPPORTED.  Replaces
 * src/layers/attention.cpp:754-780 (two norms, RoPE pair) and :823-846. */
int mi_qk_norm_rope_kv_scatter_f16(void* q, void* k, const void* v, const void* q_weight,
                                   const void* k_weight, const int64_t* positions,
                                   const float* inv_freq_host, int64_t T, int64_t Hq,
                                   int64_t Hkv, int64_t head_dim, float eps, int add_one,
                                   void* k_cache, void* v_cache, int64_t layer,
                                   int64_t num_blocks, int64_t block_size,
                                   const mi_kv_segment* segments, int num_segments, void* stream);

/* Fused per-head RMSNorm + NeoX RoPE, in place, for Q [T, Hq, hd] and
 * K [T, Hkv, hd]: each head is normalised with its weight (q_weight or
 * k_weight, [hd]; f(w) = w, or 1 + w when add_one), rounded to fp16, then
 * rotated with cos/sin made from DEVICE positions[T] and HOST inv_freq
 * [hd/2].  Equals mi_rmsnorm_f16 on the Q rows and on the K rows followed by
 * mi_rope_neox_qk_f16, in one pass.  hd must be 16, 32, 64, 128, 256 or 512
 * and the buffers 16-byte aligned (else MI_ERR_UNSUPPORTED).  Replaces the
 * Q/K-norm + RoPE sequence at src/layers/attention.cpp:754-780 (two
 * launch_rmsnorm calls, src/kernels/rmsnorm_kernel.cuh:19, then two
 * RoPE::forward_batched calls). */
int mi_qk_norm_rope_f16(void* q, void* k, const void* q_weight, const void* k_weight,
                        const int64_t* positions, const float* inv_freq_host, int64_t T,
                        int64_t Hq, int64_t Hkv, int64_t head_dim, float eps, int add_one,
                        void* stream);

/* out = silu(gate) * up, elementwise over n.
 * Replaces launch_swiglu (src/kernels/swiglu_kernel.cuh:9). */
int mi_swiglu_f16(const void* gate, const void* up, void* out, int64_t n,
                  void* stream);

/* y = gelu_tanh(x) (y may equal x).
 * Replaces launch_gelu_tanh (src/kernels/gelu_kernel.cuh:15). */
int mi_gelu_tanh_f16(const void* x, void* y, int64_t n, void* stream);

/* out = gelu_tanh(gate) * up in one pass.  Replaces the pair
 * launch_gelu_tanh + launch_mul_inplace at src/layers/mlp.cpp:282-291. */
int mi_geglu_f16(const void* gate, const void* up, void* out, int64_t n,
                 void* stream);

/* y = half(y + x).  Replaces launch_add_inplace
 * (src/kernels/model_utils_kernel.cuh:12). */
int mi_add_inplace_f16(void* y, const void* x, int64_t n, void* stream);

/* y = half(y * x).  Replaces launch_mul_inplace
 * (src/kernels/model_utils_kernel.cuh:29). */
int mi_mul_inplace_f16(void* y, const void* x, int64_t n, void* stream);

/* y = half(y * scale).  Replaces launch_scale_inplace
 * (src/kernels/model_utils_kernel.cuh:23). */
int mi_scale_inplace_f16(void* y, float scale, int64_t n, void* stream);

/* Broadcast bias add: y[b * batch_stride + m * N + n] = half(y[...] + bias[n])
 * for b < batch_stride / (M * N), m < M, n < N (the QKV projections' bias).
 * M == 0 does nothing; batch_stride < M * N is an argument error (the
 * reference's grid would be empty).  Replaces launch_add_bias
 * (src/kernels/model_utils_kernel.cuh:9, src/kernels/model_utils_kernel.cu:11-28). */
int mi_add_bias_f16(void* y, const void* bias, int64_t M, int64_t N, int64_t batch_stride,
                    void* stream);

/* Row softmax, fp32 math: y = exp(x - max) / sum(exp(x - max)).
 * x, y: [N, D]; y may equal x.  Replaces launch_softmax
 * (src/kernels/softmax_kernel.cuh:12).  Few long rows (N < 512, D >= 8192;
 * N < 256 when D <= 65536) are split across workgroups, and so are many rows
 * longer than 32768 (N >= 512, or N >= 256 up to 65536; at most 64 x 8192
 * elements) when the call can run in one launch.  On the legacy default
 * stream (0, the reference's callers' stream) out-of-place aligned calls of
 * these shapes run in one launch, using 1,056,768 bytes of row records that
 * the library allocates and zeroes once per device, on first use, and keeps
 * until the process ends.  On other streams, or in place, few long rows take
 * two launches with a stream-ordered workspace for the call, and many long
 * rows one workgroup per row. */
int mi_softmax_f16(const void* x, void* y, int64_t N, int64_t D, void* stream);

/* Bytes of device workspace mi_softmax_ws_f16 needs for [N, D]: 0 when rows
 * are processed whole (N >= 512 or N >= 256 with D <= 65536, unless D is in
 * 32769 .. 64 x 8192; and D < 8192); 1,056,768 bytes of row records (fixed:
 * 512 rows x 2064 B) for many rows longer than 32768; for few long rows, the
 * records plus one fp32 (max, sum) pair per row chunk for the two-launch
 * form. */
int64_t mi_softmax_workspace_bytes(int64_t N, int64_t D);

/* mi_softmax_f16 with a caller-provided device workspace of at least
 * mi_softmax_workspace_bytes(N, D) bytes (may be NULL when that is 0;
 * 16-byte aligned), so the call allocates nothing and can be captured into a
 * HIP graph.  The workspace must hold zeros before its first use and then be
 * used only by this function (any shapes); each call leaves it valid for the
 * next.  With y != x and aligned rows of <= 64 x 8192 elements, split rows
 * run in ONE launch: chunks exchange (max, sum) through tagged per-row
 * records, with no atomics on a shared address -- every chunk of the grid
 * resident at once, or, for more rows than that, a resident grid that walks
 * the rows in rounds.  In place, or otherwise, few long rows take the
 * two-launch form and many long rows one workgroup per row.  Calls that share
 * one workspace must not overlap in time. */
int mi_softmax_ws_f16(const void* x, void* y, int64_t N, int64_t D, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* mi_softmax_f16 for callers that cannot allocate (no counterpart in the
 * reference; for code under HIP graph capture, tight serving loops and
 * harnesses that forbid hipMalloc): the same kernels as mi_softmax_ws_f16,
 * with the workspace taken from a file-scope device array of 2,424,832 bytes
 * per GPU (512 row records of 4,224 bytes plus 256 KiB of two-pass pairs)
 * that the library holds from load until the process ends.  The array is
 * zero from the library's load and each call leaves it valid for the next;
 * calls launch nothing but the softmax (a device's first call only looks up
 * the array's address), so the first call may itself be captured in a
 * graph.  Calls no hipMalloc / hipFree.  Shapes whose workspace would exceed
 * the array return MI_ERR_UNSUPPORTED.  Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (on different streams,
 * from different threads, or graph replays concurrent with other calls) are
 * UNDEFINED -- their results may be wrong, with no error reported.  Calls in
 * one stream's order, or otherwise ordered one after the other, are safe. */
int mi_softmax_noalloc_f16(const void* x, void* y, int64_t N, int64_t D, void* stream);

/* The sampling step over one set of logits [N, V] in one pass: probs =
 * softmax(logits) as mi_softmax_ws_f16 computes it, and out[n] = the greedy
 * argmax of row n as mi_greedy_argmax_f16 computes it (the reference's tie
 * order), reading the logits once.  Replaces launch_softmax + launch_greedy
 * _sample_batched over the same logits (src/kernels/softmax_kernel.cuh:12,
 * sampling_kernel.cuh:25-30).  Shapes the one-launch softmax takes (split
 * or many long rows, aligned, probs != logits) run as one kernel whose chunks
 * also publish their best key; others run the two entry points in turn.
 * The workspace (mi_softmax_argmax_workspace_bytes(N, V) bytes, 16-byte
 * aligned) must hold zeros before its first use and then serve only this
 * function; calls sharing it must not overlap.  N <= 65535. */
int64_t mi_softmax_argmax_workspace_bytes(int64_t N, int64_t V);
int mi_softmax_argmax_ws_f16(const void* logits, void* probs, int32_t* out, int64_t N, int64_t V,
                             void* workspace, int64_t workspace_bytes, void* stream);

/* Test hook (no counterpart in the reference): bound on the polls a one-pass
 * softmax chunk makes before computing its row's statistics from x itself;
 * 0 forces that fallback everywhere.  Returns the previous bound. */
int mi_softmax_test_poll_limit(int limit);

/* out[t, :] = table[ids[t], :] for t < T; table: [vocab, H], ids: int64 [T].
 * Bit-exact copy.  When vocab > 0, an id outside [0, vocab) yields a zero
 * row instead of an out-of-bounds read; vocab <= 0 disables that check
 * (the reference's behaviour).  Replaces launch_embedding_gather
 * (src/kernels/model_utils_kernel.cuh:14), where T = B*S. */
int mi_embedding_gather_f16(const int64_t* ids, const void* table, void* out,
                            int64_t T, int64_t H, int64_t vocab, void* stream);

/* Embedding gather fused with the first layer's input RMSNorm:
 * hidden[t, :] = half(table[ids[t], :] * scale) (the row itself when scale is
 * 1; ids outside [0, vocab) give a zero row when vocab > 0) and
 * y = rmsnorm(hidden) with weight [D] (f(w) = w, or 1 + w when add_one), in
 * one pass that writes hidden and y and never reads hidden back.  Equals
 * mi_embedding_gather_f16, then mi_scale_inplace_f16 when scale != 1, then
 * mi_rmsnorm_f16, bit for bit.  Replaces launch_embedding_gather (+
 * launch_scale_inplace for Gemma) and the first input_layernorm at
 * src/model/transformer_model.cpp:561-584 (with the device copies around
 * that norm).  hidden and y must not overlap. */
int mi_embedding_rmsnorm_f16(const int64_t* ids, const void* table, void* hidden,
                             const void* weight, void* y, int64_t T, int64_t D, int64_t vocab,
                             float scale, float eps, int add_one, void* stream);

/* Paged KV-cache scatter: token (b, s) of src [B, S, H_kv, D] at global
 * position p = start_pos[b] + s is copied, when p < seq_len[b], into physical
 * block block_table[b * max_blocks_per_seq + p / block_size], slot
 * p % block_size, of layer `layer` in cache [L, num_blocks, H_kv, block_size, D]
 * (bit-exact).  block_table, seq_len and start_pos are int32 DEVICE arrays.
 * Tokens whose block index or physical block falls outside the cache are
 * skipped.  Replaces launch_paged_kv_scatter
 * (src/kernels/model_utils_kernel.cuh:55-67, called at
 * src/layers/attention.cpp:600-623 and :823-846). */
int mi_paged_kv_scatter_f16(const void* src, void* cache, const int* block_table,
                            const int* seq_len, const int* start_pos, int64_t B, int64_t S,
                            int64_t layer, int64_t num_blocks, int64_t H_kv, int64_t D,
                            int64_t block_size, int64_t max_blocks_per_seq, void* stream);

/* K and V scattered in one launch with the same block table (the reference
 * issues two launch_paged_kv_scatter calls, src/layers/attention.cpp:823-846). */
int mi_paged_kv_scatter_kv_f16(const void* k_src, const void* v_src, void* k_cache,
                               void* v_cache, const int* block_table, const int* seq_len,
                               const int* start_pos, int64_t B, int64_t S, int64_t layer,
                               int64_t num_blocks, int64_t H_kv, int64_t D, int64_t block_size,
                               int64_t max_blocks_per_seq, void* stream);

/* mi_paged_kv_scatter_kv_f16 with a projection bias added on the way:
 * the caches receive half(k + k_bias) and half(v + v_bias) (bias [H_kv * D];
 * either may be NULL for none).  Equals mi_add_bias_f16 on k_src / v_src
 * followed by the scatter, bit for bit, without writing the sources.
 * Replaces Qwen2's launch_add_bias of V (src/layers/attention.cpp:735-739) and
 * the two scatters (:823-846) with one launch. */
int mi_paged_kv_scatter_kv_bias_f16(const void* k_src, const void* v_src, void* k_cache,
                                    void* v_cache, const void* k_bias, const void* v_bias,
                                    const int* block_table, const int* seq_len,
                                    const int* start_pos, int64_t B, int64_t S, int64_t layer,
                                    int64_t num_blocks, int64_t H_kv, int64_t D,
                                    int64_t block_size, int64_t max_blocks_per_seq, void* stream);

/* Greedy sampling: out[b] = argmax over logits[b, 0:V) (fp16 [B, V]; out int32
 * [B], DEVICE).  Ties resolve exactly as the reference's 256-thread kernel
 * does: among maximal entries, the one whose i mod 256 has the smallest 8-bit
 * bit reversal, then the smallest i; NaN is never chosen; -0 equals +0; a row
 * with nothing above -inf gives -1.
 * Replaces launch_greedy_sample / launch_greedy_sample_batched
 * (src/kernels/sampling_kernel.cuh:17-30; src/kernels/sampling_kernel.cu:14-76).
 * B < 512 rows of V >= 8192 are split across workgroups: on stream 0 (V % 16
 * == 0, aligned) in one launch with 532,480 bytes of row records the library
 * holds per device (allocated and zeroed on first use, kept until the process
 * ends), otherwise in two launches with <= 256 KiB of stream-ordered
 * workspace for the call. */
int mi_greedy_argmax_f16(const void* logits, int64_t B, int64_t V, int32_t* out, void* stream);

/* Workspace bytes mi_greedy_argmax_ws_f16 needs: 0 when rows are not split,
 * else 532,480 bytes of one-launch row records (512 rows x 1040 B) plus one
 * 64-bit key per row chunk for the two-launch form. */
int64_t mi_greedy_argmax_workspace_bytes(int64_t B, int64_t V);

/* mi_greedy_argmax_f16 with a caller-provided device workspace (allocates
 * nothing; graph-capturable; 16-byte aligned).  The workspace must hold zeros
 * before its first use and then be used only by this function (any shapes);
 * each call leaves it valid for the next.  Split rows with V % 16 == 0 and
 * V <= 64 x 8192 run in ONE launch: every chunk publishes its best key to a
 * tagged per-row record and only chunk 0 of each row waits to combine them.
 * Calls sharing a workspace must not overlap. */
int mi_greedy_argmax_ws_f16(const void* logits, int64_t B, int64_t V, int32_t* out,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* Test hook (no counterpart in the reference): bound on the polls chunk 0 of
 * a one-launch argmax row makes before scanning the row itself; 0 forces
 * that fallback everywhere.  Returns the previous bound. */
int mi_greedy_argmax_test_poll_limit(int limit);

/* Nucleus (top-p) sampling of one row of `vocab` fp16 logits into out[0]
 * (int32, device), with the reference's rule (launch_top_p_sample,
 * src/kernels/sampling_kernel.cu:86-221): above 30000 logits the greedy
 * argmax of mi_greedy_argmax_f16; otherwise, with q_i = exp(x_i/T - max) /
 * sum, the candidates at indices 0, 128, 256, ... in q-descending order
 * (ties: lower index), the first position i whose running sum reaches p, and
 * the index at slot floor(u * (i + 1)) with u from MurmurHash3's fmix64 of
 * seed ^ (index_i << 32); -1 when the sum never reaches p.  Finite logits,
 * temperature > 0; logits 2-byte aligned (else MI_ERR_INVALID_ARGUMENT). */
int mi_top_p_sample_f16(const void* logits, int64_t vocab, float p, float temperature,
                        uint64_t seed, int32_t* out, void* stream);

/* mi_top_p_sample_f16 over B rows of [B, vocab] logits into out[B], row b
 * with seed + b.  (The reference's launch_top_p_sample_batched,
 * sampling_kernel.cu:223-227, is an empty stub.) */
int mi_top_p_sample_batched_f16(const void* logits, int64_t B, int64_t vocab, float p,
                                float temperature, uint64_t seed, int32_t* out, void* stream);

/* Test hook (no counterpart in the reference): how the one-launch softmax,
 * argmax and softmax + argmax kernels read their row records.  0 (default):
 * the copy in the row's XCD L2 first, then the device-scope mirror; 1: the
 * mirror only.  Returns the previous mode, or MI_ERR_INVALID_ARGUMENT. */
int mi_exchange_test_mode(int mode);

#ifdef __cplusplus
}
#endif
#endif /* MI_KERNELS_H */
