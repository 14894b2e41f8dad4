// rmsnorm.h -- RMSNorm layer: owns the [D] fp16 weight and launches the
// gfx950 kernel.  Same interface as the reference's RMSNorm
// (src/layers/rmsnorm.h:23-65) -- construction, set_weight, forward (which
// allocates and returns y), the Gemma (1 + w) switch -- plus two entry points
// the reference lacks: forward_inplace (the Q/K-norm usage) and
// forward_fused_add (residual += x; y = norm(residual) in one pass).
#pragma once

#include <cstdint>

#include "core/tensor.h"

namespace mini_infer {

class RMSNorm {
public:
    RMSNorm() = default;
    RMSNorm(int64_t dim, float eps = 1e-6f, int device_index = 0, bool add_one = false);
    ~RMSNorm();

    RMSNorm(const RMSNorm&) = delete;
    RMSNorm& operator=(const RMSNorm&) = delete;
    RMSNorm(RMSNorm&& other) noexcept;
    RMSNorm& operator=(RMSNorm&& other) noexcept;

    // y = rmsnorm(x); x: [N, D] fp16 on this layer's GPU; returns a new y.
    Tensor forward(const Tensor& x) const;

    // x = rmsnorm(x) in place (x: [N, D]).
    void forward_inplace(Tensor& x) const;

    // residual = half(residual + x); returns y = rmsnorm(residual).
    // x, residual: [N, D] fp16 on this layer's GPU.
    Tensor forward_fused_add(const Tensor& x, Tensor& residual) const;

    void set_weight(const Tensor& weight);
    void set_dim_device(int64_t dim, int device_index);
    void set_add_one(bool v) { add_one_ = v; }
    bool add_one() const { return add_one_; }
    const Tensor& weight() const { return weight_; }
    int64_t dim() const { return dim_; }
    float eps() const { return eps_; }

private:
    void check_input_(const Tensor& x, const char* who) const;

    int64_t dim_ = 0;
    float eps_ = 1e-6f;
    int device_index_ = 0;
    bool add_one_ = false;
    Tensor weight_;
};

}  // namespace mini_infer
