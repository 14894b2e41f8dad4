// rmsnorm.cpp -- RMSNorm layer (reference: src/layers/rmsnorm.cpp:11-83).
// Validation and error messages follow the reference: fp16 only, 2-D,
// contiguous, hidden dim equal to the layer's, same GPU.
#include "layers/rmsnorm.h"

#include <stdexcept>
#include <string>

#include "kernels/rmsnorm_kernel.h"

namespace mini_infer {

RMSNorm::RMSNorm(int64_t dim, float eps, int device_index, bool add_one)
    : dim_(dim), eps_(eps), device_index_(device_index), add_one_(add_one),
      weight_(Tensor::empty({dim}, DType::FP16, Device::cuda(device_index))) {}

RMSNorm::~RMSNorm() = default;

RMSNorm::RMSNorm(RMSNorm&& o) noexcept
    : dim_(o.dim_), eps_(o.eps_), device_index_(o.device_index_), add_one_(o.add_one_),
      weight_(std::move(o.weight_)) {}

RMSNorm& RMSNorm::operator=(RMSNorm&& o) noexcept {
    if (this != &o) {
        dim_ = o.dim_;
        eps_ = o.eps_;
        device_index_ = o.device_index_;
        add_one_ = o.add_one_;
        weight_ = std::move(o.weight_);
    }
    return *this;
}

void RMSNorm::set_dim_device(int64_t dim, int device_index) {
    if (dim_ == 0 && weight_.numel() == 0) {
        dim_ = dim;
        device_index_ = device_index;
        weight_ = Tensor::empty({dim}, DType::FP16, Device::cuda(device_index));
    }
}

void RMSNorm::set_weight(const Tensor& weight) {
    if (weight.dtype() != DType::FP16) throw std::runtime_error("RMSNorm::set_weight expects FP16");
    if (weight.numel() != dim_) throw std::runtime_error("RMSNorm::set_weight: weight size mismatch");
    weight_ = weight.to(Device::cuda(device_index_));
}

void RMSNorm::check_input_(const Tensor& x, const char* who) const {
    const std::string w(who);
    if (x.dtype() != DType::FP16) throw std::runtime_error(w + ": only FP16 supported");
    if (!x.device().is_cuda() || x.device().index != device_index_)
        throw std::runtime_error(w + ": device mismatch");
    if (x.ndim() != 2) throw std::runtime_error(w + ": only 2-D input supported");
    if (x.shape()[1] != dim_) throw std::runtime_error(w + ": hidden dim mismatch");
    if (!x.is_contiguous()) throw std::runtime_error(w + ": only contiguous input supported");
}

Tensor RMSNorm::forward(const Tensor& x) const {
    check_input_(x, "RMSNorm::forward");
    const int N = static_cast<int>(x.shape()[0]);
    const int D = static_cast<int>(x.shape()[1]);
    Tensor y = Tensor::empty({N, D}, DType::FP16, Device::cuda(device_index_));
    kernels::launch_rmsnorm(static_cast<const __half*>(x.data()),
                            static_cast<const __half*>(weight_.data()),
                            static_cast<__half*>(y.data()), N, D, eps_, add_one_ ? 1 : 0,
                            /*stream=*/0);
    return y;
}

void RMSNorm::forward_inplace(Tensor& x) const {
    check_input_(x, "RMSNorm::forward_inplace");
    const int N = static_cast<int>(x.shape()[0]);
    const int D = static_cast<int>(x.shape()[1]);
    kernels::launch_rmsnorm(static_cast<const __half*>(x.data()),
                            static_cast<const __half*>(weight_.data()),
                            static_cast<__half*>(x.data()), N, D, eps_, add_one_ ? 1 : 0, 0);
}

Tensor RMSNorm::forward_fused_add(const Tensor& x, Tensor& residual) const {
    check_input_(x, "RMSNorm::forward_fused_add");
    check_input_(residual, "RMSNorm::forward_fused_add(residual)");
    if (residual.shape() != x.shape())
        throw std::runtime_error("RMSNorm::forward_fused_add: residual shape mismatch");
    const int N = static_cast<int>(x.shape()[0]);
    const int D = static_cast<int>(x.shape()[1]);
    Tensor y = Tensor::empty({N, D}, DType::FP16, Device::cuda(device_index_));
    kernels::launch_fused_add_rmsnorm(static_cast<const __half*>(x.data()),
                                      static_cast<__half*>(residual.data()),
                                      static_cast<const __half*>(weight_.data()),
                                      static_cast<__half*>(y.data()), N, D, eps_,
                                      add_one_ ? 1 : 0, 0);
    return y;
}

}  // namespace mini_infer
