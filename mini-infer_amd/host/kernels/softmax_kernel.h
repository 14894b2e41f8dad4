// softmax_kernel.h -- launch_softmax with the reference's signature
// (src/kernels/softmax_kernel.cuh:12): row softmax of x [N, D] into y.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

void launch_softmax(const __half* x, __half* y, int N, int D, hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
