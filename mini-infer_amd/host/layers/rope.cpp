// rope.cpp -- RoPE layer (reference: src/layers/rope.cpp:11-131).
#include "layers/rope.h"

#include <cmath>
#include <stdexcept>
#include <string>

#include "kernels/rope_kernel.h"

namespace mini_infer {

RoPE::RoPE(int head_dim, float theta_base, int device_index)
    : head_dim_(head_dim), theta_base_(theta_base), device_index_(device_index) {
    if (head_dim_ <= 0 || (head_dim_ & 1) != 0)
        throw std::runtime_error("RoPE: head_dim must be positive even");
    recompute_inv_freq_();
}

// inv_freq[i] = 1 / theta^(2i / head_dim) in fp32, with the C library's powf.
void RoPE::recompute_inv_freq_() {
    const int half = head_dim_ / 2;
    inv_freq_.resize(half);
    for (int i = 0; i < half; ++i) {
        const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(head_dim_);
        inv_freq_[i] = 1.0f / std::pow(theta_base_, e);
    }
}

void RoPE::set_theta_base(float theta_base) {
    theta_base_ = theta_base;
    recompute_inv_freq_();
}

Tensor RoPE::rotate_(const Tensor& x, const std::vector<int64_t>& pos, const char* who) {
    const int B = static_cast<int>(x.shape()[0]);
    const int S = static_cast<int>(x.shape()[1]);
    const int H = static_cast<int>(x.shape()[2]);
    const int D = static_cast<int>(x.shape()[3]);
    const int half = D / 2;
    Tensor cos_t = Tensor::empty({static_cast<int64_t>(B) * S, half}, DType::FP16,
                                 Device::cuda(device_index_));
    Tensor sin_t = Tensor::empty({static_cast<int64_t>(B) * S, half}, DType::FP16,
                                 Device::cuda(device_index_));
    kernels::launch_rope_precompute_batched(inv_freq_.data(), pos.data(),
                                            static_cast<__half*>(cos_t.data()),
                                            static_cast<__half*>(sin_t.data()), B, S, half, 0);
    Tensor y = Tensor::empty({B, S, H, D}, DType::FP16, Device::cuda(device_index_));
    kernels::launch_rope(static_cast<const __half*>(x.data()),
                         static_cast<const __half*>(cos_t.data()),
                         static_cast<const __half*>(sin_t.data()), static_cast<__half*>(y.data()),
                         B, S, H, D, 0);
    (void)who;
    return y;
}

namespace {
void check_4d(const Tensor& x, int head_dim, int device_index, const char* who) {
    const std::string w(who);
    if (x.dtype() != DType::FP16) throw std::runtime_error(w + ": only FP16 supported");
    if (x.ndim() != 4) throw std::runtime_error(w + ": expect 4-D input [B,S,H,D]");
    if (x.shape()[3] != head_dim) throw std::runtime_error(w + ": head_dim mismatch");
    if (!x.is_contiguous()) throw std::runtime_error(w + ": only contiguous input supported");
    if (!x.device().is_cuda() || x.device().index != device_index)
        throw std::runtime_error(w + ": device mismatch");
}
}  // namespace

Tensor RoPE::forward(const Tensor& x, const std::vector<int64_t>& positions) {
    check_4d(x, head_dim_, device_index_, "RoPE::forward");
    const int B = static_cast<int>(x.shape()[0]);
    const int S = static_cast<int>(x.shape()[1]);
    if (static_cast<int>(positions.size()) != S)
        throw std::runtime_error("RoPE::forward: positions size must equal S");
    std::vector<int64_t> rep(static_cast<size_t>(B) * S);
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < S; ++s) rep[static_cast<size_t>(b) * S + s] = positions[s];
    return rotate_(x, rep, "RoPE::forward");
}

Tensor RoPE::forward_batched(const Tensor& x, const std::vector<int64_t>& positions) {
    check_4d(x, head_dim_, device_index_, "RoPE::forward_batched");
    const int64_t BS = x.shape()[0] * x.shape()[1];
    if (static_cast<int64_t>(positions.size()) != BS)
        throw std::runtime_error("RoPE::forward_batched: positions size must equal B*S");
    return rotate_(x, positions, "RoPE::forward_batched");
}

void RoPE::check_qk_(const Tensor& q, const Tensor& k, const Tensor& positions, const char* who,
                     int64_t& Tq, int64_t& Hq, int64_t& Hk) const {
    auto split = [&](const Tensor& t, const char* name, int64_t& T, int64_t& H) {
        const std::string w = std::string(who) + "(" + name + ")";
        if (t.dtype() != DType::FP16) throw std::runtime_error(w + ": only FP16 supported");
        if (t.ndim() < 3) throw std::runtime_error(w + ": expect [..., H, head_dim]");
        if (t.shape().back() != head_dim_) throw std::runtime_error(w + ": head_dim mismatch");
        if (!t.is_contiguous()) throw std::runtime_error(w + ": only contiguous input supported");
        if (!t.device().is_cuda() || t.device().index != device_index_)
            throw std::runtime_error(w + ": device mismatch");
        H = t.shape()[t.ndim() - 2];
        T = 1;
        for (int i = 0; i < t.ndim() - 2; ++i) T *= t.shape()[i];
    };
    int64_t Tk;
    split(q, "q", Tq, Hq);
    split(k, "k", Tk, Hk);
    if (Tq != Tk) throw std::runtime_error(std::string(who) + ": q and k token counts differ");
    if (positions.dtype() != DType::INT64 || positions.numel() != Tq ||
        !positions.device().is_cuda() || positions.device().index != device_index_)
        throw std::runtime_error(std::string(who) +
                                 ": positions must be int64 [T] on the layer's GPU");
}

void RoPE::forward_qk_inplace(Tensor& q, Tensor& k, const Tensor& positions) const {
    int64_t T, Hq, Hk;
    check_qk_(q, k, positions, "RoPE::forward_qk_inplace", T, Hq, Hk);
    kernels::launch_rope_qk(static_cast<__half*>(q.data()), static_cast<__half*>(k.data()),
                            static_cast<const int64_t*>(positions.data()), inv_freq_.data(),
                            static_cast<int>(T), static_cast<int>(Hq), static_cast<int>(Hk),
                            head_dim_, 0);
}

void RoPE::forward_qk_norm_inplace(Tensor& q, Tensor& k, const RMSNorm& q_norm,
                                   const RMSNorm& k_norm, const Tensor& positions) const {
    int64_t T, Hq, Hk;
    check_qk_(q, k, positions, "RoPE::forward_qk_norm_inplace", T, Hq, Hk);
    if (q_norm.dim() != head_dim_ || k_norm.dim() != head_dim_)
        throw std::runtime_error("RoPE::forward_qk_norm_inplace: norm dim must equal head_dim");
    if (q_norm.add_one() != k_norm.add_one() || q_norm.eps() != k_norm.eps())
        throw std::runtime_error(
            "RoPE::forward_qk_norm_inplace: q and k norms must share eps and add_one");
    kernels::launch_qk_norm_rope(static_cast<__half*>(q.data()), static_cast<__half*>(k.data()),
                                 static_cast<const __half*>(q_norm.weight().data()),
                                 static_cast<const __half*>(k_norm.weight().data()),
                                 static_cast<const int64_t*>(positions.data()), inv_freq_.data(),
                                 static_cast<int>(T), static_cast<int>(Hq), static_cast<int>(Hk),
                                 head_dim_, q_norm.eps(), q_norm.add_one() ? 1 : 0, 0);
}

}  // namespace mini_infer
