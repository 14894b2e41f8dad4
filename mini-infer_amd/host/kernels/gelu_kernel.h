// gelu_kernel.h -- launch_gelu_tanh with the reference's signature
// (src/kernels/gelu_kernel.cuh:15), plus the fused GeGLU.
#pragma once

#include <cstdint>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

// y = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))); y may equal x.
void launch_gelu_tanh(const __half* x, __half* y, int64_t n, hipStream_t stream);

// out = gelu_tanh(gate) * up in one pass (replaces gelu then mul_inplace).
void launch_geglu(const __half* gate, const __half* up, __half* out, int64_t n,
                  hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
