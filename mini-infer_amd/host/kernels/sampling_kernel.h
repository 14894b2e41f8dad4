// sampling_kernel.h -- sampling launchers with the reference's signatures
// (src/kernels/sampling_kernel.cuh:17-36): greedy and top-p.  The
// speculative-decoding accept/reject kernel (:38-57) is not part of this
// library: nothing in the reference calls it, and its draws come from a
// closed library's random stream.
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

// Top-p (nucleus) sample of logits [vocab] into out[0], the reference's rule:
// above 30000 logits the greedy argmax; otherwise the candidates at indices
// 0, 128, 256, ... by probability, the first whose running sum reaches p, a
// slot drawn from `seed`, and -1 when the sum never reaches p
// (mi_top_p_sample_f16 states it in full).
void launch_top_p_sample(const __half* logits, int vocab, float p, float temperature,
                         unsigned long long seed, int* out, hipStream_t stream);

// launch_top_p_sample on each row of logits [B, vocab], row b with seed + b.
// (The reference's batched launcher is an empty stub that writes nothing.)
void launch_top_p_sample_batched(const __half* logits, int B, int vocab, float p,
                                 float temperature, unsigned long long seed, int* out,
                                 hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
