/*
 * mi_chain.h -- C ABI of the decoder-step chain (libmini_infer.so): the
 * non-GEMM launches of one decoder layer and of the sampling step, issued in
 * the order of the reference's batched paged forward
 * (src/model/transformer_model.cpp:545-660 with src/layers/attention.cpp:
 * 689-846 and src/layers/mlp.cpp:270-292), on one stream, with no device
 * copies between them and no allocation.
 *
 * The reference step, per layer, and what replaces each piece here:
 *   gather (+ embed scale), copy,     -> mi_embedding_rmsnorm_f16: hidden and `normed`
 *   input_layernorm, copy                in one pass
 *   [QKV GEMMs]                       -> the caller's q, k, v
 *   (Qwen2: 3x launch_add_bias)          (folded into the next two steps)
 *   copies, Q-norm, K-norm, 2x RoPE   -> mi_qk_norm_rope_f16 (or mi_rope_neox_qk_f16;
 *                                        Qwen2: mi_bias_rope_neox_qk_f16)
 *   2x launch_paged_kv_scatter        -> mi_paged_kv_scatter_kv_f16 per segment (Qwen2:
 *                                        mi_paged_kv_scatter_kv_bias_f16, V's bias)
 *   [attention, O GEMM]               -> the caller's attn_out
 *   (Gemma 2/3: post_attn norm of attn_out, in place)
 *   add_inplace, copy, post-attn norm -> mi_fused_add_rmsnorm_f16
 *   [gate / up GEMMs]                 -> the caller's gate, up
 *   SwiGLU, or gelu_tanh + mul        -> mi_swiglu_f16 / mi_geglu_f16
 *   [down GEMM]                       -> the caller's mlp_out
 *   (Gemma 2/3: post_ff norm of mlp_out, in place)
 *   add_inplace, copy, final norm     -> mi_fused_add_rmsnorm_f16 (with one layer the
 *                                        final norm stands where the next layer's input
 *                                        norm would)
 *   [LM head]                         -> the caller's logits
 *   sampling: softmax and argmax      -> mi_softmax_argmax_ws_f16 (one read of the logits)
 * The bracketed GEMM steps are not part of this library: their outputs are
 * buffers the caller fills (in the C++ interface, through hooks called at
 * those points; through this ABI, before the call).
 */
#ifndef MI_CHAIN_H
#define MI_CHAIN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One group of sequences in the reference's [B, S] KV-scatter layout
 * (launch_paged_kv_scatter, src/kernels/model_utils_kernel.cuh:55-67):
 * tokens [token_offset, token_offset + B*S) of k / v, with int32 DEVICE
 * block_table [B, max_blocks_per_seq], seq_len [B] and start_pos [B].  A mixed
 * continuous batch is several segments (decode tokens as B = n, S = 1;
 * prefills as B = m, S = prompt length). */
typedef struct mi_chain_kv_segment {
    int64_t token_offset;
    int64_t B, S;
    const int* block_table;
    const int* seq_len;
    const int* start_pos;
    int64_t max_blocks_per_seq;
} mi_chain_kv_segment;

typedef struct mi_chain_desc {
    /* shapes: T tokens; hidden_size D; intermediate_size I; heads Hq / Hkv x head_dim;
     * vocab V (embedding rows and logit columns); logit_rows N */
    int64_t T, hidden_size, intermediate_size, num_heads, num_kv_heads, head_dim, vocab, logit_rows;
    /* KV cache [num_layers, num_blocks, Hkv, block_size, head_dim] */
    int64_t layer, num_layers, num_blocks, block_size;
    float rms_eps, qk_norm_eps, rope_theta;
    int norm_add_one; /* Gemma (1 + w) norms */
    int use_qk_norm;  /* Gemma 3 per-head Q/K RMSNorm (attention.cpp:754-768) */
    int embed_scale;  /* Gemma: hidden *= sqrt(hidden) after the gather */
    int double_norm;  /* Gemma 2/3 post_attn / post_ff norms around the blocks */
    int act;          /* 0 = SwiGLU (ActKind::Silu), 1 = GeGLU (ActKind::GeluTanh) */
    /* weights (fp16, device) */
    const void* embed;          /* [V, D] */
    const void* input_norm;     /* [D] */
    const void* post_attn_norm; /* [D] */
    const void* pre_ff_norm;    /* [D], double_norm only */
    const void* post_ff_norm;   /* [D], double_norm only */
    const void* final_norm;     /* [D] */
    const void* q_norm;         /* [head_dim], use_qk_norm only */
    const void* k_norm;         /* [head_dim], use_qk_norm only */
    /* step inputs (device) */
    const int64_t* ids;       /* [T] */
    const int64_t* positions; /* [T] */
    int num_kv_segments;
    const mi_chain_kv_segment* kv_segments; /* host array */
    /* buffers (fp16, device) */
    void* hidden;       /* [T, D] residual stream */
    void* normed;       /* [T, D] input-norm output (QKV GEMM input) */
    void* q;            /* [T, Hq, hd] QKV GEMM output, rotated in place */
    void* k;            /* [T, Hkv, hd] */
    void* v;            /* [T, Hkv, hd] */
    void* k_cache;      /* KV cache */
    void* v_cache;
    void* attn_out;     /* [T, D] O GEMM output */
    void* post_normed;  /* [T, D] post-attention norm output (gate / up GEMM input) */
    void* gate;         /* [T, I] */
    void* up;           /* [T, I] */
    void* act_out;      /* [T, I] activation (down GEMM input) */
    void* mlp_out;      /* [T, D] down GEMM output */
    void* final_normed; /* [T, D] final norm output (LM head input) */
    void* logits;       /* [N, V] LM head output */
    void* probs;        /* [N, V] softmax */
    int32_t* next_tokens; /* [N] greedy argmax */
    void* sample_ws;    /* mi_softmax_argmax_workspace_bytes(N, V) bytes, zero before first use */
    int64_t sample_ws_bytes;
    /* Qwen2 QKV projection bias (fp16, device): q_bias [Hq * hd], k_bias and
     * v_bias [Hkv * hd]; all NULL for none, else all set.  q and k are biased
     * in place with the rotation; v's bias is added on its way into the cache
     * and v itself is left as it was (the reference's add_bias rewrites its
     * v scratch buffer, which nothing reads after the scatter). */
    const void* q_bias;
    const void* k_bias;
    const void* v_bias;
} mi_chain_desc;

/* Stages, in issue order; mi_decoder_chain_run stops after `last_stage`. */
enum {
    MI_CHAIN_EMBED = 1,          /* hidden = gather(ids) (* sqrt(D)) */
    MI_CHAIN_INPUT_NORM = 2,     /* normed = rmsnorm(hidden) */
    MI_CHAIN_QK_ROPE = 3,        /* q, k = rope(qk_norm(q (+ bias), k (+ bias))) in place */
    MI_CHAIN_KV_SCATTER = 4,     /* k, v -> paged cache */
    MI_CHAIN_POST_ATTN_NORM = 5, /* hidden += attn_out; post_normed = rmsnorm(hidden) */
    MI_CHAIN_ACTIVATION = 6,     /* act_out = act(gate) * up */
    MI_CHAIN_FINAL_NORM = 7,     /* hidden += mlp_out; final_normed = rmsnorm(hidden) */
    MI_CHAIN_SAMPLE = 8          /* probs = softmax(logits), next_tokens = argmax(logits) */
};

/* Validates `d` against every stage up to last_stage (MI_ERR_* of
 * mi_kernels.h when a pointer or size is missing or out of range; nothing is
 * launched then), then enqueues the stages on `stream` (hipStream_t; NULL =
 * the null stream) and returns without synchronising.  Allocates nothing, so
 * a call can be captured into a HIP graph. */
int mi_decoder_chain_run(const mi_chain_desc* d, int last_stage, void* stream);

/* Text of the last error mi_decoder_chain_run returned on this thread. */
const char* mi_decoder_chain_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* MI_CHAIN_H */
