/*
 * mi_oracle.h -- CPU restatement of mini-infer's layer-kernel arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP kernels
 * are compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the mini-infer source tree).  fp16 values travel as
 * uint16_t bit patterns; "float out" variants return the un-rounded fp32
 * reference that the reference's verify.py compares against with
 * allclose(rtol=1e-3, atol=1e-3) (tests/verify/verify.py:138-147).
 *
 * Row-parallel functions take `nthreads` (<=1 means single-threaded); the
 * threads split rows, so results do not depend on the thread count.
 */
#ifndef MI_ORACLE_H
#define MI_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 -> fp16 IEEE round-to-nearest-even: the rounding of the reference
 * kernels' __float2half (e.g. src/kernels/model_utils_kernel.cu:34) and of
 * the device's fp32 -> fp16 conversion. */
uint16_t mio_f32_to_f16(float f);
/* The fp32 -> fp16 converter the reference's kernel tests use to build their
 * fp16 inputs (tests/test_rmsnorm/main.cpp:40-67, duplicated in each
 * kernel test's main.cpp).  It is NOT round-to-nearest-even: with an even kept
 * LSB it truncates, and below 2^-14 it shifts one bit too far per binade.  It
 * is restated with those quirks so the reference's seeded test inputs are
 * regenerated bit for bit; nothing else uses it. */
uint16_t mio_reftest_f32_to_f16(float f);
void mio_reftest_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);
/* Exact fp16 -> fp32 widening (IEEE binary16 decode). */
float mio_f16_to_f32(uint16_t h);
void mio_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);
void mio_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);

/* xorshift32 uniform in [-scale, scale] (tests/test_helpers.h:46-57). */
void mio_fill_uniform(float* out, int64_t n, float scale, uint32_t seed);
/* xorshift32 integers in [lo, hi] (tests/test_helpers.h:60-68). */
void mio_fill_uniform_int64(int64_t* out, int64_t n, uint32_t seed,
                            int64_t lo, int64_t hi);

/* RMSNorm, fp32 result: y = x * rsqrt(mean(x^2) + eps) * f(w), f(w) = w or
 * 1 + w (tests/verify/verify.py:32-44; src/kernels/rmsnorm_kernel.cu:53-65).
 * The sum of squares is accumulated in double. */
void mio_rmsnorm(const uint16_t* x, const uint16_t* w, float* y,
                 int64_t N, int64_t D, float eps, int add_one, int nthreads);

/* Residual add then RMSNorm, as the model chain composes them:
 * residual = half(residual + x) (src/kernels/model_utils_kernel.cu:31-35,
 * called at src/model/transformer_model.cpp:608), then y = rmsnorm(residual)
 * (src/model/transformer_model.cpp:614-615).  residual is updated in place
 * (bit-exact fp16); y is the fp32 reference. */
void mio_fused_add_rmsnorm(const uint16_t* x, uint16_t* residual,
                           const uint16_t* w, float* y, int64_t N, int64_t D,
                           float eps, int add_one, int nthreads);

/* inv_freq[i] = 1 / theta^(2i/head_dim) in fp32 (src/layers/rope.cpp:20-28). */
void mio_rope_inv_freq(float* inv_freq, int head_dim, float theta);

/* cos/sin tables [N, half] as fp16 bits: angle = float(pos) * inv_freq[i] in
 * fp32 (src/kernels/rope_kernel.cu:74), value = half(cos(angle)) with the
 * fp32 cosine correctly rounded (the reference uses device cosf, and its test
 * uses host std::cos, tests/test_rope/main.cpp:89-100). */
void mio_rope_tables(const float* inv_freq, const int64_t* positions,
                     uint16_t* cos_t, uint16_t* sin_t, int64_t N, int half);

/* NeoX half rotation with per-token tables [T, hd/2] over x [T, H, hd]
 * (tests/verify/verify.py:47-66; src/kernels/rope_kernel.cu:27-54).
 * y1 = x1*c - x2*s, y2 = x2*c + x1*s, fp32 result. */
void mio_rope_neox(const uint16_t* x, const uint16_t* cos_t,
                   const uint16_t* sin_t, float* y, int64_t T, int H, int hd,
                   int nthreads);

/* silu(g) * u = g / (1 + exp(-g)) * u, fp32 result
 * (tests/verify/verify.py:76-82; src/kernels/swiglu_kernel.cu:16-26). */
void mio_swiglu(const uint16_t* g, const uint16_t* u, float* out, int64_t n,
                int nthreads);

/* gelu_tanh(x) = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), fp32
 * (tests/verify/verify.py:85-91; src/kernels/gelu_kernel.cu:23-35). */
void mio_gelu_tanh(const uint16_t* x, float* y, int64_t n, int nthreads);

/* GeGLU as one fp32 expression gelu_tanh(g) * u (the fp32-accumulated result
 * that the fused kernel is held to). */
void mio_geglu(const uint16_t* g, const uint16_t* u, float* out, int64_t n,
               int nthreads);

/* GeGLU as the reference composes it at src/layers/mlp.cpp:282-291:
 * a = half(gelu_tanh(g)); out = half(a * u), fp16 bits. */
void mio_geglu_composed(const uint16_t* g, const uint16_t* u, uint16_t* out,
                        int64_t n);

/* Elementwise fp16 ops, bit-exact (src/kernels/model_utils_kernel.cu):
 * add y = half(y + x) (:31-35), mul y = half(y * x) (:82-86),
 * scale y = half(y * s) (:68-72). */
void mio_add_inplace(uint16_t* y, const uint16_t* x, int64_t n);
void mio_mul_inplace(uint16_t* y, const uint16_t* x, int64_t n);
void mio_scale_inplace(uint16_t* y, float scale, int64_t n);

/* Broadcast bias add (src/kernels/model_utils_kernel.cu:11-28): for
 * b < batch_stride / (M * N), m < M, n < N,
 * y[b * batch_stride + m * N + n] = half(y[...] + bias[n]); M == 0 or an empty
 * batch count does nothing. */
void mio_add_bias(uint16_t* y, const uint16_t* bias, int64_t M, int64_t N,
                  int64_t batch_stride);

/* Row softmax, fp32 result (tests/verify/verify.py:69-73 torch.softmax;
 * src/kernels/softmax_kernel.cu:26-58).  Max-shifted, sums in double. */
void mio_softmax(const uint16_t* x, float* y, int64_t N, int64_t D,
                 int nthreads);

/* out[t, :] = table[ids[t], :] (src/kernels/model_utils_kernel.cu:45-56),
 * bit-exact.  Ids outside [0, vocab) give a zero row (the reference leaves
 * that case undefined). */
void mio_embedding_gather(const int64_t* ids, const uint16_t* table,
                          uint16_t* out, int64_t T, int64_t H, int64_t vocab,
                          int nthreads);

/* Paged KV scatter (src/kernels/model_utils_kernel.cu:108-145): token (b, s)
 * of src [B, S, H_kv, D] at position p = start_pos[b] + s goes, when
 * p < seq_len[b], to block block_table[b * max_blocks + p / bs], slot p % bs,
 * of `layer` in cache [L, num_blocks, H_kv, bs, D].  Entries outside the cache
 * are skipped (the reference writes out of bounds there). */
void mio_paged_kv_scatter(const uint16_t* src, uint16_t* cache, const int32_t* block_table,
                          const int32_t* seq_len, const int32_t* start_pos, int64_t B,
                          int64_t S, int64_t layer, int64_t num_blocks, int64_t H_kv, int64_t D,
                          int64_t block_size, int64_t max_blocks_per_seq);

/* Greedy argmax per row, simulating the reference kernel's 256-thread
 * strided scan and shared-memory tree reduction literally
 * (src/kernels/sampling_kernel.cu:52-76). */
void mio_greedy_argmax(const uint16_t* logits, int64_t B, int64_t V, int32_t* out);

/* MurmurHash3's 64-bit finaliser, the slot hash of the reference's top-p
 * (src/kernels/sampling_kernel.cu:177-180). */
uint64_t mio_fmix64(uint64_t s);

/* Top-p sampling of B rows, row b with seed + b, following
 * launch_top_p_sample (src/kernels/sampling_kernel.cu:86-221) step by step:
 * above 30000 logits the greedy argmax (mio_greedy_argmax); otherwise the
 * row maximum of x/T, probabilities expf(x/T - max) / sum, K = 256 rounds of
 * strict-greater selection over the first thread's stride-128 share of the
 * row (indices 0, 128, ...; empty rounds leave index -1 and -inf), the
 * insertion sort, the running sum over the 256 slots and the fmix64 slot
 * draw; when the sum never reaches p, slot 255 (index -1 below 30001
 * logits). */
void mio_top_p_sample(const uint16_t* logits, int64_t B, int64_t vocab, float p,
                      float temperature, uint64_t seed, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif
