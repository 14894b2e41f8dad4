// rope.h -- RoPE layer.  Same interface as the reference's RoPE
// (src/layers/rope.h:16-44): inv_freq computed on the host from theta and
// head_dim, forward(x, positions[S]) and forward_batched(x, positions[B*S])
// returning a new rotated tensor, set_theta_base for Gemma-3's dual band.
// Added: forward_qk_inplace, which rotates Q and K in place in one launch
// with cos/sin made in registers from device positions.
#pragma once

#include <cstdint>
#include <vector>

#include "core/tensor.h"
#include "layers/rmsnorm.h"

namespace mini_infer {

class RoPE {
public:
    RoPE(int head_dim, float theta_base = 1000000.0f, int device_index = 0);

    // x: [B, S, H, head_dim] fp16; positions: [S] (shared by every batch row).
    Tensor forward(const Tensor& x, const std::vector<int64_t>& positions);

    // x: [B, S, H, head_dim]; positions: [B*S], one per token.
    Tensor forward_batched(const Tensor& x, const std::vector<int64_t>& positions);

    // In place: q [T, Hq, head_dim] and k [T, Hkv, head_dim] (either may be
    // 3-D or 4-D with leading dims multiplying to T); positions: int64 [T]
    // on the same GPU.
    void forward_qk_inplace(Tensor& q, Tensor& k, const Tensor& positions) const;

    // Gemma-3 style Q/K RMSNorm fused in front of the rotation, in place:
    // q = rope(q_norm(q)), k = rope(k_norm(k)), per head, in one pass.  The
    // norms' dim must equal head_dim (shapes as forward_qk_inplace).
    void forward_qk_norm_inplace(Tensor& q, Tensor& k, const RMSNorm& q_norm,
                                 const RMSNorm& k_norm, const Tensor& positions) const;

    void set_theta_base(float theta_base);

    int head_dim() const { return head_dim_; }
    int half_dim() const { return head_dim_ / 2; }
    float theta_base() const { return theta_base_; }
    const std::vector<float>& inv_freq() const { return inv_freq_; }

private:
    void recompute_inv_freq_();
    Tensor rotate_(const Tensor& x, const std::vector<int64_t>& flat_positions, const char* who);
    void check_qk_(const Tensor& q, const Tensor& k, const Tensor& positions, const char* who,
                   int64_t& T, int64_t& Hq, int64_t& Hk) const;

    int head_dim_;
    float theta_base_;
    int device_index_;
    std::vector<float> inv_freq_;
};

}  // namespace mini_infer
