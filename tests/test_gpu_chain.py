"""GPU parity of the decoder-step chain (include/mi_chain.h): every stage of
one non-GEMM decoder step, issued by the C++ chain through the C ABI, against
the oracle's composition of the same steps on the same seeded inputs.

The step follows the reference's batched paged forward
(src/model/transformer_model.cpp:545-660; attention.cpp:743-846;
mlp.cpp:270-292): gather -> input RMSNorm -> [QKV] -> Q/K-norm + RoPE ->
paged K/V scatter -> [attention] -> residual add + post-attention RMSNorm ->
[gate/up] -> SwiGLU -> [down] -> residual add + final RMSNorm -> [LM head]
-> softmax and greedy argmax.  The bracketed GEMMs are seeded stand-in
buffers.

The workload: 64 decode tokens at random positions
plus two 3000-token prefills (T = 6064), Qwen2.5-7B shapes, embedding table
[152064, 3584], logits [64, 152064].

Bars: gather, residual stream and KV cache bit-exact; plain RoPE bit-exact
(its tables and rotation are exact functions of the inputs); fp16 outputs
within rtol = atol = 1e-3 of the fp32 oracle (tests/verify/verify.py:142),
the fused Q/K-norm + RoPE as in test_gpu_rope (one ulp of the normalised
operands at fp16 rounding boundaries); argmax indices exact.
"""
import numpy as np
import pytest

from helpers import (assert_bits_equal, assert_close, assert_norm_rope_close, qk_norm_rope_ref,
                     to_host)

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def chain_mod(dev):
    import mi_chain
    mi_chain.load_library()
    return mi_chain


@pytest.fixture(scope="module")
def cfg5(chain_mod, dev):
    _case("building the config-5 workload (T = 6064, table [152064, 3584])")
    return chain_mod.Workload(dev, seed=5)


def _biased(orc, w, name):
    """The GEMM stand-in `name` (q, k or v) as the reference's add_bias leaves
    it (model_utils_kernel.cu:11-28), or as it is without a QKV bias."""
    h, s = w.host, w.shapes
    if not s.get("qkv_bias"):
        return h[name]
    x = h[name]
    n = x.shape[1] * x.shape[2]
    T = x.shape[0]
    return orc.add_bias(x.reshape(-1), h[name + "_bias"], T, n, T * n).reshape(x.shape)


def _check_kv(orc, w, k_src, what):
    """K and V caches against the oracle's scatter of (k_src, v) per segment."""
    s = w.shapes
    v_src = _biased(orc, w, "v")
    kc = np.zeros((s["num_layers"], s["num_blocks"], s["num_kv_heads"], s["block_size"],
                   s["head_dim"]), np.float16)
    vc = kc.copy()
    for g in w.groups:
        o, B, S = g["token_offset"], g["B"], g["S"]
        ks = k_src[o:o + B * S].reshape(B, S, s["num_kv_heads"], s["head_dim"])
        vs = v_src[o:o + B * S].reshape(B, S, s["num_kv_heads"], s["head_dim"])
        kc = orc.paged_kv_scatter(ks, kc, g["block_table"], g["seq_len"], g["start_pos"],
                                  s["layer"], s["block_size"])
        vc = orc.paged_kv_scatter(vs, vc, g["block_table"], g["seq_len"], g["start_pos"],
                                  s["layer"], s["block_size"])
    assert_bits_equal(to_host(w.t["k_cache"]), kc, what=f"{what}: k cache")
    assert_bits_equal(to_host(w.t["v_cache"]), vc, what=f"{what}: v cache")


def _check_chain(chain_mod, orc, w, what):
    """Runs the chain three times (to the embedding, to the post-attention
    norm, to the end) and checks every intermediate against the oracle."""
    S = chain_mod.Stage
    h, s = w.host, w.shapes
    eps, add1 = s["rms_eps"], bool(s["norm_add_one"])
    T, D = s["T"], s["hidden_size"]

    # 1. embedding (+ scale): hidden is the gathered rows, bit for bit
    w.run(S.EMBED)
    hid0 = h["embed"][h["ids"]]
    if s["embed_scale"]:
        hid0 = orc.f32_to_f16(hid0.astype(np.float32) * np.float32(np.sqrt(np.float32(D))))
    assert_bits_equal(to_host(w.t["hidden"]), hid0, what=f"{what}: gather")

    # 2-5: input norm, Q/K, KV scatter, residual add + post-attention norm
    w.reload("q", "k")
    w.run(S.POST_ATTN_NORM)
    assert_close(to_host(w.t["normed"]), orc.rmsnorm(hid0, h["input_norm"], eps, add1, nthreads=8),
                 what=f"{what}: input norm")
    inv = orc.rope_inv_freq(s["head_dim"], s["rope_theta"])
    pos = h["positions"]
    q_out, k_out = to_host(w.t["q"]), to_host(w.t["k"])
    qk_in = {n: _biased(orc, w, n) for n in ("q", "k")}
    if s["use_qk_norm"]:
        for name, got, wt in (("q", q_out, h["q_norm"]), ("k", k_out, h["k_norm"])):
            ref, n16 = qk_norm_rope_ref(orc, qk_in[name], wt, pos, inv, s["qk_norm_eps"])
            assert_norm_rope_close(got, ref, n16, what=f"{what}: qk-norm + rope {name}")
    else:
        c, sn = orc.rope_tables(inv, pos)
        for name, got in (("q", q_out), ("k", k_out)):
            assert_bits_equal(got, orc.rope_neox(qk_in[name], c, sn, nthreads=8).astype(np.float16),
                              what=f"{what}: rope {name}")
    if s.get("qkv_bias"):  # v is read, not rewritten
        assert_bits_equal(to_host(w.t["v"]), h["v"], what=f"{what}: v left as it was")
    _check_kv(orc, w, k_out, what)
    attn = h["attn_out"]
    if s["double_norm"]:
        attn = orc.f32_to_f16(orc.rmsnorm(attn, h["post_attn_norm"], eps, add1, nthreads=8))
        assert_close(to_host(w.t["attn_out"]), attn.astype(np.float32),
                     what=f"{what}: post-attn norm of attn_out")
        attn = to_host(w.t["attn_out"])  # the next step consumes the GPU's fp16 value
        w2 = h["pre_ff_norm"]
    else:
        w2 = h["post_attn_norm"]
    hid1, pn = orc.fused_add_rmsnorm(attn, hid0, w2, eps, add1, nthreads=8)
    assert_bits_equal(to_host(w.t["hidden"]), hid1, what=f"{what}: residual after attention")
    assert_close(to_host(w.t["post_normed"]), pn, what=f"{what}: post-attention norm")

    # 6-8: activation, residual add + final norm, softmax and argmax
    w.reload("q", "k")
    if s["double_norm"]:
        w.reload("attn_out", "mlp_out")
    w.run(S.SAMPLE)
    act = orc.geglu(h["gate"], h["up"], nthreads=8) if s["act"] else \
        orc.swiglu(h["gate"], h["up"], nthreads=8)
    assert_close(to_host(w.t["act_out"]), act, what=f"{what}: activation")
    mlp = h["mlp_out"]
    if s["double_norm"]:
        got = to_host(w.t["mlp_out"])
        assert_close(got, orc.rmsnorm(mlp, h["post_ff_norm"], eps, add1, nthreads=8),
                     what=f"{what}: post-ff norm of mlp_out")
        mlp = got
    hid2, fn = orc.fused_add_rmsnorm(mlp, hid1, h["final_norm"], eps, add1, nthreads=8)
    assert_bits_equal(to_host(w.t["hidden"]), hid2, what=f"{what}: residual after the MLP")
    assert_close(to_host(w.t["final_normed"]), fn, what=f"{what}: final norm")
    assert_close(to_host(w.t["probs"]), orc.softmax(h["logits"], nthreads=8),
                 what=f"{what}: softmax")
    assert (to_host(w.t["next_tokens"]) == orc.greedy_argmax(h["logits"])).all(), \
        f"{what}: greedy argmax"


def test_chain_config5_every_stage(chain_mod, orc, cfg5):
    """The decoder-chain workload through the whole chain, Gemma-3-style Q/K norm on."""
    _case("chain workload: T=6064, qk-norm + rope, SwiGLU [6064,18944], logits [64,152064]")
    _check_chain(chain_mod, orc, cfg5, "chain workload")


def test_chain_config5_plain_rope(chain_mod, orc, cfg5):
    """Qwen2.5 proper has no Q/K norm: the plain in-place RoPE on the chain's
    positions (64 decode tokens + two 3000-token prefills), bit-exact, and
    the scatter of its rotated K."""
    _case("chain workload without qk-norm: rope_neox_qk on the chain positions")
    import copy
    w = copy.copy(cfg5)
    w.shapes = dict(cfg5.shapes, use_qk_norm=0)
    w.desc, w._keep = chain_mod.make_desc(w.shapes, cfg5.t, cfg5.segments)
    w.reload("q", "k")
    w.run(chain_mod.Stage.KV_SCATTER)
    h = w.host
    inv = orc.rope_inv_freq(128, 1e6)
    c, sn = orc.rope_tables(inv, h["positions"])
    k_out = to_host(w.t["k"])
    assert_bits_equal(to_host(w.t["q"]), orc.rope_neox(h["q"], c, sn, nthreads=8).astype(np.float16),
                      what="rope q")
    assert_bits_equal(k_out, orc.rope_neox(h["k"], c, sn, nthreads=8).astype(np.float16),
                      what="rope k")
    _check_kv(orc, w, k_out, "plain rope")


def test_chain_config5_qwen2_bias(chain_mod, orc, dev, cfg5):
    """Qwen2.5 proper: the QKV projection bias and no Q/K norm, at the chain workload
    (T = 6064): Q/K biased and rotated in one pass (bit-exact against
    add_bias then RoPE), V's bias added on its way into the cache
    (bit-exact), then the rest of the step."""
    _case("chain workload, Qwen2 QKV bias, no qk-norm")
    import copy
    import torch
    w = copy.copy(cfg5)
    rng = np.random.default_rng(55)
    s = cfg5.shapes
    qn, kn = s["num_heads"] * s["head_dim"], s["num_kv_heads"] * s["head_dim"]
    w.host = dict(cfg5.host)
    w.t = dict(cfg5.t)
    for name, n in (("q_bias", qn), ("k_bias", kn), ("v_bias", kn)):
        w.host[name] = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.5)).astype(np.float16)
        w.t[name] = torch.from_numpy(w.host[name]).to(dev)
    w.t["k_cache"].zero_()
    w.t["v_cache"].zero_()
    w.shapes = dict(s, use_qk_norm=0, qkv_bias=1)
    w.desc, w._keep = chain_mod.make_desc(w.shapes, w.t, cfg5.segments)
    _check_chain(chain_mod, orc, w, "qwen2 bias")


def test_chain_bias_with_qk_norm(chain_mod, orc, dev):
    """QKV bias together with Q/K norm (the reference adds the bias, then
    normalises): the chain's unfused bias launches ahead of the fused
    Q/K-norm + RoPE, on a small batch."""
    _case("chain bias + qk-norm, small batch")
    w = chain_mod.Workload(dev, seed=41, n_decode=5, prefills=(29, 29), logit_rows=5,
                           hidden_size=256, intermediate_size=512, num_heads=4, num_kv_heads=2,
                           head_dim=64, vocab=777, use_qk_norm=1, qkv_bias=1)
    _check_chain(chain_mod, orc, w, "bias + qk-norm")


@pytest.mark.parametrize("act", [0, 1])
def test_chain_gemma_flags(chain_mod, orc, dev, act):
    """Gemma-style options on a small batch: (1 + w) norms, sqrt(D) embedding
    scale, the post-attention / post-feed-forward norms of Gemma 2/3, Q/K
    norm, and either activation; a single decode token and one prefill of 37."""
    _case(f"chain gemma flags act={act}")
    w = chain_mod.Workload(dev, seed=11 + act, n_decode=1, prefills=(37,), logit_rows=3,
                           hidden_size=256, intermediate_size=640, num_heads=4, num_kv_heads=2,
                           head_dim=64, vocab=999, rope_theta=1e4, norm_add_one=1, use_qk_norm=1,
                           embed_scale=1, double_norm=1, act=act)
    _check_chain(chain_mod, orc, w, f"gemma act={act}")


def test_chain_decode_only_split_logits(chain_mod, orc, dev):
    """Decode tokens only (no prefill segment) with logits long enough to be
    split across workgroups (one-launch softmax / argmax with the chain's
    workspaces)."""
    _case("chain decode only, logits [7, 50000]")
    w = chain_mod.Workload(dev, seed=21, n_decode=7, prefills=(), logit_rows=7, hidden_size=512,
                           intermediate_size=1024, num_heads=8, num_kv_heads=2, head_dim=128,
                           vocab=50000, use_qk_norm=0)
    _check_chain(chain_mod, orc, w, "decode only")


def test_chain_graph_replay(chain_mod, orc, dev):
    """The whole chain captured into one HIP graph and replayed: every replay
    (with eager work in between that restores the in-place Q / K inputs)
    reproduces the eager call's outputs bit for bit."""
    _case("chain graph replay")
    import torch
    w = chain_mod.Workload(dev, seed=31, n_decode=16, prefills=(200, 200), logit_rows=16,
                           vocab=40000)
    outs = ("hidden", "normed", "q", "k", "k_cache", "v_cache", "post_normed", "act_out",
            "final_normed", "probs", "next_tokens")
    w.run()
    ref = {n: to_host(w.t[n]).copy() for n in outs}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    w.reload("q", "k")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        w.run(stream=side)
    for i in range(3):
        w.reload("q", "k")
        w.t["hidden"].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n in outs:
            assert_bits_equal(to_host(w.t[n]), ref[n], what=f"replay {i}: {n}")
    del g
