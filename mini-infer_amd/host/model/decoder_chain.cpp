// decoder_chain.cpp -- the non-GEMM decoder step (reference:
// src/model/transformer_model.cpp:545-660 TransformerModel::forward_paged_batched,
// src/layers/attention.cpp:754-846, src/layers/mlp.cpp:270-292).
#include "model/decoder_chain.h"

#include <cmath>
#include <stdexcept>
#include <string>

#include "mi_kernels.h"

namespace mini_infer {
namespace {

// A refused launch, carrying the library's status code.
struct ChainError : std::runtime_error {
    int status;
    ChainError(int st, const std::string& what) : std::runtime_error(what), status(st) {}
};

void check(int st, const char* what) {
    if (st != MI_OK)
        throw ChainError(st, std::string("decoder chain: ") + what + ": " + mi_status_string(st));
}

void need(bool ok, const char* what) {
    if (!ok) throw std::invalid_argument(std::string("decoder chain: ") + what);
}

void* sv(hipStream_t s) { return reinterpret_cast<void*>(s); }

}  // namespace

DecoderChain::DecoderChain(const mi_chain_desc& d, int last_stage) : d_(d), last_(last_stage) {
    need(last_ >= MI_CHAIN_EMBED && last_ <= MI_CHAIN_SAMPLE, "last_stage out of range");
    need(d_.num_kv_segments >= 0, "num_kv_segments < 0");
    need(d_.num_kv_segments == 0 || d_.kv_segments, "kv_segments is null");
    segs_.assign(d_.kv_segments, d_.kv_segments + d_.num_kv_segments);
    d_.kv_segments = segs_.data();
    validate_();
    // inv_freq[i] = 1 / theta^(2i / head_dim) in fp32 (src/layers/rope.cpp:20-28)
    const int half = static_cast<int>(d_.head_dim / 2);
    inv_freq_.resize(half);
    for (int i = 0; i < half; ++i) {
        const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(d_.head_dim);
        inv_freq_[i] = 1.0f / std::pow(d_.rope_theta, e);
    }
}

void DecoderChain::validate_() const {
    const mi_chain_desc& d = d_;
    need(d.T >= 0 && d.hidden_size > 0 && d.vocab > 0, "T, hidden and vocab must be set");
    need(d.num_heads >= 0 && d.num_kv_heads >= 0 && d.head_dim > 0 && d.head_dim % 2 == 0 &&
             d.head_dim <= 512,
         "heads / head_dim");
    need(d.act == 0 || d.act == 1, "act must be 0 (SwiGLU) or 1 (GeGLU)");
    const int L = last_;
    need(d.ids && d.embed && d.hidden, "embed stage needs ids, embed, hidden");
    if (L >= MI_CHAIN_INPUT_NORM) need(d.input_norm && d.normed, "input norm needs input_norm, normed");
    const bool bias = d.q_bias || d.k_bias || d.v_bias;
    need(!bias || ((d.num_heads == 0 || d.q_bias) && (d.num_kv_heads == 0 || (d.k_bias && d.v_bias))),
         "qkv bias: set q_bias, k_bias and v_bias together");
    if (L >= MI_CHAIN_QK_ROPE) {
        need(d.positions && (d.num_heads == 0 || d.q) && (d.num_kv_heads == 0 || d.k),
             "rope needs positions, q, k");
        need(!d.use_qk_norm || ((d.num_heads == 0 || d.q_norm) && (d.num_kv_heads == 0 || d.k_norm)),
             "qk norm needs q_norm, k_norm");
    }
    if (L >= MI_CHAIN_KV_SCATTER && d.num_kv_segments > 0) {
        need(d.k && d.v && d.k_cache && d.v_cache, "kv scatter needs k, v, k_cache, v_cache");
        need(d.num_blocks > 0 && d.block_size > 0 && d.layer >= 0 && d.layer < d.num_layers,
             "kv cache geometry");
        for (const mi_chain_kv_segment& s : segs_) {
            need(s.B >= 0 && s.S >= 0 && s.token_offset >= 0 && s.token_offset + s.B * s.S <= d.T,
                 "kv segment outside the T tokens");
            need(s.B * s.S == 0 ||
                     (s.block_table && s.seq_len && s.start_pos && s.max_blocks_per_seq > 0),
                 "kv segment tables");
        }
    }
    if (L >= MI_CHAIN_POST_ATTN_NORM) {
        need(d.attn_out && d.post_attn_norm && d.post_normed, "post-attn norm buffers");
        need(!d.double_norm || d.pre_ff_norm, "double_norm needs pre_ff_norm");
    }
    if (L >= MI_CHAIN_ACTIVATION)
        need(d.intermediate_size > 0 && d.gate && d.up && d.act_out, "activation buffers");
    if (L >= MI_CHAIN_FINAL_NORM) {
        need(d.mlp_out && d.final_norm && d.final_normed, "final norm buffers");
        need(!d.double_norm || d.post_ff_norm, "double_norm needs post_ff_norm");
    }
    if (L >= MI_CHAIN_SAMPLE) {
        need(d.logit_rows > 0 && d.logits && d.probs && d.next_tokens, "sample buffers");
        need(d.logit_rows <= 65535, "logit_rows above 65535");
        need(d.sample_ws && d.sample_ws_bytes >= mi_softmax_argmax_workspace_bytes(d.logit_rows,
                                                                                  d.vocab),
             "sample workspace too small");
    }
}

// Steps 3 and 4 in one launch: the (Q/K-norm +) rotation pass also writes
// the rotated K rows and the V rows (+ V bias) into the paged cache, so K is
// not re-read.  False (nothing launched) for shapes the one-launch kernel
// does not take, and for a QKV bias together with Q/K norm; the caller then
// runs the two steps.
bool DecoderChain::rope_kv_fused(hipStream_t s) const {
    const mi_chain_desc& d = d_;
    const bool bias = d.q_bias != nullptr;
    if ((d.use_qk_norm && bias) || d.num_heads <= 0 || d.num_kv_heads <= 0) return false;
    mi_kv_segment fs[8];
    int n = 0;
    for (const mi_chain_kv_segment& g : segs_) {
        if (g.B * g.S == 0) continue;
        if (n == 8) return false;
        fs[n++] = mi_kv_segment{g.token_offset, g.B, g.S, g.block_table, g.seq_len,
                                g.start_pos, g.max_blocks_per_seq};
    }
    const int st =
        d.use_qk_norm
            ? mi_qk_norm_rope_kv_scatter_f16(d.q, d.k, d.v, d.q_norm, d.k_norm, d.positions,
                                             inv_freq_.data(), d.T, d.num_heads, d.num_kv_heads,
                                             d.head_dim, d.qk_norm_eps, /*add_one=*/0, d.k_cache,
                                             d.v_cache, d.layer, d.num_blocks, d.block_size, fs,
                                             n, sv(s))
            : mi_rope_kv_scatter_f16(d.q, d.k, d.v, d.q_bias, d.k_bias, d.v_bias, d.positions,
                                     inv_freq_.data(), d.T, d.num_heads, d.num_kv_heads,
                                     d.head_dim, d.k_cache, d.v_cache, d.layer, d.num_blocks,
                                     d.block_size, fs, n, sv(s));
    if (st == MI_ERR_UNSUPPORTED) return false;
    check(st, d.use_qk_norm ? "qk norm + rope + kv scatter"
                            : (bias ? "bias + rope + kv scatter" : "rope + kv scatter"));
    return true;
}

void DecoderChain::run(hipStream_t s, DecoderChainHooks* hooks) const {
    DecoderChainHooks none;
    DecoderChainHooks& h = hooks ? *hooks : none;
    const mi_chain_desc& d = d_;
    const int64_t T = d.T, D = d.hidden_size;
    const float eps = d.rms_eps;
    const int add1 = d.norm_add_one;
    if (T == 0) return;

    // 1-2. token embedding (+ Gemma's sqrt(D) scale) and the input_layernorm
    //    (transformer_model.cpp:561-584: gather, scale, copy hidden into a
    //    2-D tensor, normalise, copy back) in one pass that writes hidden and
    //    normed; stopping after the embedding takes the gather alone
    const float scale = d.embed_scale ? std::sqrt(static_cast<float>(D)) : 1.0f;
    if (last_ == MI_CHAIN_EMBED) {
        check(mi_embedding_gather_f16(d.ids, d.embed, d.hidden, T, D, d.vocab, sv(s)), "gather");
        if (d.embed_scale)
            check(mi_scale_inplace_f16(d.hidden, scale, T * D, sv(s)), "embed scale");
        return;
    }
    check(mi_embedding_rmsnorm_f16(d.ids, d.embed, d.hidden, d.input_norm, d.normed, T, D,
                                   d.vocab, scale, eps, add1, sv(s)),
          "gather + input norm");
    if (last_ == MI_CHAIN_INPUT_NORM) return;

    // 3. QKV GEMMs, then Q/K-norm + RoPE in one in-place pass
    //    (attention.cpp:717-780: Qwen2's bias adds, two copies, two norms,
    //    two RoPE forwards); with the bias and no Q/K norm (Qwen2) the bias
    //    add rides in the rotation pass; a chain that runs to the KV scatter
    //    does steps 3 and 4 in one launch
    h.qkv(d, s);
    const bool bias = d.q_bias != nullptr || d.k_bias != nullptr;
    if (last_ >= MI_CHAIN_KV_SCATTER && rope_kv_fused(s)) {
        if (last_ == MI_CHAIN_KV_SCATTER) return;
    } else {
        if (bias && d.use_qk_norm) {  // bias, then norm: no model has both; kept unfused
            const int64_t qn = d.num_heads * d.head_dim, kn = d.num_kv_heads * d.head_dim;
            if (d.num_heads > 0)
                check(mi_add_bias_f16(d.q, d.q_bias, T, qn, T * qn, sv(s)), "q bias");
            if (d.num_kv_heads > 0)
                check(mi_add_bias_f16(d.k, d.k_bias, T, kn, T * kn, sv(s)), "k bias");
        }
        if (bias && !d.use_qk_norm)
            check(mi_bias_rope_neox_qk_f16(d.q, d.k, d.q_bias, d.k_bias, d.positions,
                                           inv_freq_.data(), T, d.num_heads, d.num_kv_heads,
                                           d.head_dim, sv(s)),
                  "bias + rope");
        else if (d.use_qk_norm)
            check(mi_qk_norm_rope_f16(d.q, d.k, d.q_norm, d.k_norm, d.positions,
                                      inv_freq_.data(), T, d.num_heads, d.num_kv_heads,
                                      d.head_dim, d.qk_norm_eps, /*add_one=*/0, sv(s)),
                  "qk norm + rope");
        else
            check(mi_rope_neox_qk_f16(d.q, d.k, d.positions, inv_freq_.data(), T, d.num_heads,
                                      d.num_kv_heads, d.head_dim, sv(s)),
                  "rope");
        if (last_ == MI_CHAIN_QK_ROPE) return;

        // 4. K and V into the paged cache, one launch per segment
        //    (attention.cpp:819-846: one scatter for K, one for V; Qwen2's V bias
        //    added on the way, attention.cpp:735-739)
        const int64_t kv_row = d.num_kv_heads * d.head_dim;
        for (const mi_chain_kv_segment& g : segs_) {
            if (g.B * g.S == 0) continue;
            const auto* ks = static_cast<const uint16_t*>(d.k) + g.token_offset * kv_row;
            const auto* vs = static_cast<const uint16_t*>(d.v) + g.token_offset * kv_row;
            if (d.v_bias)
                check(mi_paged_kv_scatter_kv_bias_f16(
                          ks, vs, d.k_cache, d.v_cache, nullptr, d.v_bias, g.block_table,
                          g.seq_len, g.start_pos, g.B, g.S, d.layer, d.num_blocks,
                          d.num_kv_heads, d.head_dim, d.block_size, g.max_blocks_per_seq, sv(s)),
                      "kv scatter + v bias");
            else
                check(mi_paged_kv_scatter_kv_f16(ks, vs, d.k_cache, d.v_cache, g.block_table,
                                                 g.seq_len, g.start_pos, g.B, g.S, d.layer,
                                                 d.num_blocks, d.num_kv_heads, d.head_dim,
                                                 d.block_size, g.max_blocks_per_seq, sv(s)),
                      "kv scatter");
        }
        if (last_ == MI_CHAIN_KV_SCATTER) return;
    }

    // 5. attention + O GEMM, then residual add fused with the post-attention
    //    norm (transformer_model.cpp:591-603, 605-625)
    h.attention(d, s);
    if (d.double_norm) {
        check(mi_rmsnorm_f16(d.attn_out, d.post_attn_norm, d.attn_out, T, D, eps, add1, sv(s)),
              "post-attn norm");
        check(mi_fused_add_rmsnorm_f16(d.attn_out, d.hidden, d.pre_ff_norm, d.post_normed, T, D,
                                       eps, add1, sv(s)),
              "residual add + pre-ff norm");
    } else {
        check(mi_fused_add_rmsnorm_f16(d.attn_out, d.hidden, d.post_attn_norm, d.post_normed, T,
                                       D, eps, add1, sv(s)),
              "residual add + post-attn norm");
    }
    if (last_ == MI_CHAIN_POST_ATTN_NORM) return;

    // 6. gate / up GEMMs, then the activation (mlp.cpp:270-292)
    h.gate_up(d, s);
    const int64_t n = T * d.intermediate_size;
    if (d.act == 0)
        check(mi_swiglu_f16(d.gate, d.up, d.act_out, n, sv(s)), "swiglu");
    else
        check(mi_geglu_f16(d.gate, d.up, d.act_out, n, sv(s)), "geglu");
    if (last_ == MI_CHAIN_ACTIVATION) return;

    // 7. down GEMM, then residual add fused with the final norm
    //    (transformer_model.cpp:627-660; the next layer's input norm in a
    //    deeper model)
    h.down(d, s);
    if (d.double_norm)
        check(mi_rmsnorm_f16(d.mlp_out, d.post_ff_norm, d.mlp_out, T, D, eps, add1, sv(s)),
              "post-ff norm");
    check(mi_fused_add_rmsnorm_f16(d.mlp_out, d.hidden, d.final_norm, d.final_normed, T, D, eps,
                                   add1, sv(s)),
          "residual add + final norm");
    if (last_ == MI_CHAIN_FINAL_NORM) return;

    // 8. LM head, then the sampling step: softmax and greedy argmax of the
    //    logits rows in one pass
    h.lm_head(d, s);
    check(mi_softmax_argmax_ws_f16(d.logits, d.probs, d.next_tokens, d.logit_rows, d.vocab,
                                   d.sample_ws, d.sample_ws_bytes, sv(s)),
          "softmax + greedy argmax");
}

}  // namespace mini_infer

namespace {
thread_local std::string g_last_error;
}

extern "C" int mi_decoder_chain_run(const mi_chain_desc* d, int last_stage, void* stream) {
    g_last_error.clear();
    if (!d) {
        g_last_error = "decoder chain: descriptor is null";
        return MI_ERR_INVALID_ARGUMENT;
    }
    try {
        const mini_infer::DecoderChain chain(*d, last_stage);
        chain.run(reinterpret_cast<hipStream_t>(stream));
        return MI_OK;
    } catch (const mini_infer::ChainError& e) {
        g_last_error = e.what();
        return e.status;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return MI_ERR_INVALID_ARGUMENT;
    }
}

extern "C" const char* mi_decoder_chain_last_error(void) { return g_last_error.c_str(); }
