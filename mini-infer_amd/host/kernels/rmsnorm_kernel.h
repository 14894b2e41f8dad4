// rmsnorm_kernel.h -- launch_rmsnorm with the reference's signature
// (src/kernels/rmsnorm_kernel.cuh:19-20), plus the fused residual-add variant.
// Both forward to the C ABI (include/mi_kernels.h) and throw
// std::runtime_error if the launch is rejected.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace mini_infer {
namespace kernels {

// y = (x / sqrt(mean(x^2) + eps)) * f(weight), f(w) = w or (1 + w) when
// add_one != 0.  x, y: [N, D] fp16 row-major on the GPU (y may equal x);
// weight: [D].
void launch_rmsnorm(const __half* x, const __half* weight, __half* y, int N, int D, float eps,
                    int add_one, hipStream_t stream);

// residual = half(residual + x); y = rmsnorm(residual) -- one pass replacing
// launch_add_inplace(residual, x) followed by launch_rmsnorm(residual).
void launch_fused_add_rmsnorm(const __half* x, __half* residual, const __half* weight, __half* y,
                              int N, int D, float eps, int add_one, hipStream_t stream);

// Per-head RMSNorm of q [T, Hq, hd] and k [T, Hkv, hd] in place, one launch
// replacing the Q-norm and K-norm launch_rmsnorm pair (Gemma 3); k may be
// null when Hkv == 0.
void launch_qk_rmsnorm(__half* q, __half* k, const __half* q_weight, const __half* k_weight,
                       int T, int Hq, int Hkv, int head_dim, float eps, int add_one,
                       hipStream_t stream);

}  // namespace kernels
}  // namespace mini_infer
