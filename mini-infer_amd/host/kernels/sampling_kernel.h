// sampling_kernel.h -- greedy sampling launchers with the reference's
// signatures (src/kernels/sampling_kernel.cuh:17-30).  Top-p sampling is not
// part of this library.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

// out[0] = argmax of logits [vocab] (int32 on the GPU); ties resolve as the
// reference's 256-thread kernel does.
void launch_greedy_sample(const __half* logits, int vocab, int* out, hipStream_t stream);

// out[b] = argmax of row b of logits [B, vocab].
void launch_greedy_sample_batched(const __half* logits, int B, int vocab, int* out,
                                  hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
