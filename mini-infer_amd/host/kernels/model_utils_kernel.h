// model_utils_kernel.h -- the model-chain utility launchers on the hot path,
// with the reference's signatures (src/kernels/model_utils_kernel.cuh:12-29).
// launch_add_bias and launch_paged_kv_scatter belong to the attention path
// and are not part of this library.
#pragma once

#include <cstdint>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

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

}  // namespace kernels
}  // namespace mini_infer
