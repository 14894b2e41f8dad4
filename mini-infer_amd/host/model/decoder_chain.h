// decoder_chain.h -- caller-side composition of the layer kernels: the
// non-GEMM launches of one decoder layer plus the sampling step, in the
// order of the reference's batched paged forward
// (src/model/transformer_model.cpp:545-660, src/layers/attention.cpp:689-846,
// src/layers/mlp.cpp:270-292), with the reference's device copies around
// every norm and its separate add / norm, Q-norm / K-norm / RoPE and K / V
// scatter launches replaced by the fused entry points.  The stage list and
// the C ABI over it are in include/mi_chain.h.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "mi_chain.h"

namespace mini_infer {

// The GEMM-shaped steps the chain leaves to its caller, called on the
// chain's stream at the point where the reference runs them.  Each fills the
// buffers named in its comment; the defaults do nothing (the buffers already
// hold the caller's data, e.g. fixed seeded stand-ins in a test).
class DecoderChainHooks {
public:
    virtual ~DecoderChainHooks() = default;
    virtual void qkv(const mi_chain_desc&, hipStream_t) {}        // normed -> q, k, v
    virtual void attention(const mi_chain_desc&, hipStream_t) {}  // q, caches -> attn_out
    virtual void gate_up(const mi_chain_desc&, hipStream_t) {}    // post_normed -> gate, up
    virtual void down(const mi_chain_desc&, hipStream_t) {}       // act_out -> mlp_out
    virtual void lm_head(const mi_chain_desc&, hipStream_t) {}    // final_normed -> logits
};

class DecoderChain {
public:
    // Copies the descriptor (and its KV segments), checks it for the stages
    // up to `last_stage`, and computes RoPE's inv_freq on the host
    // (src/layers/rope.cpp:20-28).  Throws std::invalid_argument on a bad
    // descriptor.
    explicit DecoderChain(const mi_chain_desc& d, int last_stage = MI_CHAIN_SAMPLE);

    // Enqueues the stages up to last_stage on `stream`; throws
    // std::runtime_error when a launch is refused.
    void run(hipStream_t stream, DecoderChainHooks* hooks = nullptr) const;

    const std::vector<float>& inv_freq() const { return inv_freq_; }

private:
    void validate_() const;
    bool rope_kv_fused(hipStream_t stream) const;

    mi_chain_desc d_;
    int last_;
    std::vector<mi_chain_kv_segment> segs_;
    std::vector<float> inv_freq_;
};

}  // namespace mini_infer
