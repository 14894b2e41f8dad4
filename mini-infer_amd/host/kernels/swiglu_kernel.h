// swiglu_kernel.h -- launch_swiglu with the reference's signature
// (src/kernels/swiglu_kernel.cuh:9): out = silu(gate) * up over n elements.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

void launch_swiglu(const __half* gate, const __half* up, __half* out, int n, hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
