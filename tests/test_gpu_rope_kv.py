"""GPU parity: RoPE of Q/K with the K and V rows written into the paged KV
cache in the same launch (mi_rope_kv_scatter_f16), with and without Qwen2's
q/k/v bias, and with Gemma 3's per-head Q/K RMSNorm before the rotation
(mi_qk_norm_rope_kv_scatter_f16).

The reference does this as the bias adds, the RoPE pair and one
launch_paged_kv_scatter per tensor and sequence group
(src/layers/attention.cpp:717-780, :823-846).  Expected values: the oracle's
add_bias, rope_neox and paged_kv_scatter applied per segment; every output is
compared bit for bit (fp16 in, fp16 out, the same fp32 roundings), and also
against this library's own separate launches.  Cases: the decoder chain's
continuous batch (64 decode tokens + two 3000-token prefills), head_dims
16..256, ragged segments (a token past its seq_len, unmapped or out-of-range
block ids, tokens outside every segment, an empty segment), no segment at
all, and the refusals (unsupported shapes, partial bias, aliasing).  The
norm form is bit-exact against this library's qk_norm_rope followed by the
scatters, its Q/K within the norm + RoPE tolerance of the oracle's
composition (tests/helpers.py), and its caches bit-exact against the oracle's
scatter of its own rotated K.
"""
import numpy as np
import pytest

from helpers import (assert_bits_equal, assert_norm_rope_close, normal_f16, qk_norm_rope_ref,
                     to_dev, to_host)

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _bias(orc, x, b):
    T, H, hd = x.shape
    return orc.add_bias(x.reshape(-1), b, T, H * hd, T * H * hd).reshape(x.shape)


def _segments(rng, kind, T, bs, NB):
    """Host segment dicts (token_offset, S, block_table, seq_len, start_pos)."""
    segs = []
    if kind == "chain":  # 64 decode tokens, then two prefills of 3000
        starts = rng.integers(0, 400, 64)
        spans = [(0, 64, 1, starts, starts + 1), (64, 1, 3000, [0], [3000]),
                 (3064, 1, 3000, [500], [3500])]
    elif kind == "ragged":
        # seg 0: b=1 stops at seq_len; seg 1 leaves tokens [30, 34) uncovered;
        # seg 2 is empty; seg 3 has an unmapped and an out-of-range block id
        spans = [(0, 3, 6, [0, 10, 20], [6, 14, 26]), (18, 2, 6, [3, 40], [9, 46]),
                 (30, 0, 5, [], []), (34, 2, 7, [0, 17], [7, 24])]
    else:
        spans = []
    used = rng.permutation(NB)
    nxt = 0
    for off, B, S, st, sl in spans:
        mb = max(1, -(-int(max(list(sl) + [1])) // bs))
        bt = used[nxt:nxt + B * mb].reshape(B, mb).astype(np.int32)
        nxt += B * mb
        segs.append(dict(token_offset=off, S=S, block_table=bt,
                         seq_len=np.asarray(sl, np.int32), start_pos=np.asarray(st, np.int32)))
    if kind == "ragged":
        segs[3]["block_table"][0, 0] = -1
        segs[3]["block_table"][1, 1] = NB + 5
    assert nxt <= NB
    return segs


def _expect(orc, q, k, v, pos, inv, kc, vc, segs, layer, bs, biases):
    if biases is not None:
        q, k, v = (_bias(orc, x, b) for x, b in zip((q, k, v), biases))
    c, s = orc.rope_tables(inv, pos)
    qr = orc.rope_neox(q, c, s, nthreads=8).astype(np.float16)
    kr = orc.rope_neox(k, c, s, nthreads=8).astype(np.float16)
    H, hd = k.shape[1:]
    for g in segs:
        B, S, o = g["block_table"].shape[0], g["S"], g["token_offset"]
        if B * S == 0:
            continue
        args = (g["block_table"], g["seq_len"], g["start_pos"], layer, bs)
        kc = orc.paged_kv_scatter(kr[o:o + B * S].reshape(B, S, H, hd), kc, *args)
        vc = orc.paged_kv_scatter(v[o:o + B * S].reshape(B, S, H, hd), vc, *args)
    return qr, kr, kc, vc


def _dev_segs(segs, dev):
    return [dict(g, block_table=to_dev(g["block_table"], dev), seq_len=to_dev(g["seq_len"], dev),
                 start_pos=to_dev(g["start_pos"], dev)) for g in segs]


@pytest.mark.parametrize("T,Hq,Hkv,hd,kind", [
    (6064, 28, 4, 128, "chain"),   # Qwen2.5-7B heads, the chain's continuous batch
    (48, 16, 8, 64, "ragged"),
    (48, 8, 4, 256, "ragged"),
    (48, 4, 2, 16, "ragged"),
    (48, 15, 1, 32, "ragged"),     # 16 units per token: Q/K lanes < 256, 4 V lanes
    (48, 16, 16, 128, "ragged"),   # MHA at the limit: 256 Q/K units and 256 V vectors
    (20, 8, 8, 128, "none"),       # no segment: RoPE only
])
@pytest.mark.parametrize("bias", [False, True])
def test_rope_kv_scatter_vs_oracle(mk, orc, dev, T, Hq, Hkv, hd, kind, bias):
    _case(f"rope + kv scatter T={T} Hq={Hq} Hkv={Hkv} hd={hd} {kind} bias={bias}")
    rng = np.random.default_rng(T + Hq * 7 + hd + bias)
    bs, L, layer = 16, 2, 1
    NB = 2100 if kind == "chain" else 40
    segs = _segments(rng, kind, T, bs, NB)
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    v = normal_f16(rng, (T, Hkv, hd))
    kc = normal_f16(rng, (L, NB, Hkv, bs, hd))
    vc = normal_f16(rng, (L, NB, Hkv, bs, hd))
    pos = rng.integers(0, 32000, T).astype(np.int64)
    biases = None
    if bias:
        biases = (normal_f16(rng, (Hq * hd,), 0, 0.5), normal_f16(rng, (Hkv * hd,), 0, 0.5),
                  normal_f16(rng, (Hkv * hd,), 0, 0.5))
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd, vd, kcd, vcd = (to_dev(x, dev) for x in (q, k, v, kc, vc))
    bd = [to_dev(b, dev) for b in biases] if bias else [None] * 3
    mk.rope_kv_scatter(qd, kd, vd, to_dev(pos, dev), inv, kcd, vcd, layer, bs,
                       _dev_segs(segs, dev), *bd)
    qr, kr, kcr, vcr = _expect(orc, q, k, v, pos, inv, kc, vc, segs, layer, bs, biases)
    assert_bits_equal(to_host(qd), qr, what="q")
    assert_bits_equal(to_host(kd), kr, what="k")
    assert_bits_equal(to_host(vd), v, what="v source untouched")
    assert_bits_equal(to_host(kcd), kcr, what="k cache")
    assert_bits_equal(to_host(vcd), vcr, what="v cache")


@pytest.mark.parametrize("bias", [False, True])
def test_rope_kv_scatter_equals_separate_launches(mk, orc, dev, bias):
    """Against this library's rope (or bias + rope) and per-segment K+V
    scatter (with the V bias) at the chain's shape."""
    _case(f"rope + kv scatter == separate launches, bias={bias}")
    rng = np.random.default_rng(500 + bias)
    T, Hq, Hkv, hd, bs, NB = 6064, 28, 4, 128, 16, 2100
    segs = _segments(rng, "chain", T, bs, NB)
    q, k, v = (normal_f16(rng, (T, h, hd)) for h in (Hq, Hkv, Hkv))
    kc = normal_f16(rng, (1, NB, Hkv, bs, hd))
    vc = normal_f16(rng, (1, NB, Hkv, bs, hd))
    pos = to_dev(rng.integers(0, 32000, T).astype(np.int64), dev)
    inv = orc.rope_inv_freq(hd, 1e6)
    bq, bk, bv = (to_dev(normal_f16(rng, (h * hd,), 0, 0.5), dev) for h in (Hq, Hkv, Hkv))
    dsegs = _dev_segs(segs, dev)
    qa, ka, va, kca, vca = (to_dev(x, dev) for x in (q, k, v, kc, vc))
    if bias:
        mk.bias_rope_neox_qk(qa, ka, bq, bk, pos, inv)
    else:
        mk.rope_neox_qk(qa, ka, pos, inv)
    for g in dsegs:
        B, S, o = g["block_table"].shape[0], g["S"], g["token_offset"]
        src = ka[o:o + B * S].reshape(B, S, Hkv, hd)
        vsrc = va[o:o + B * S].reshape(B, S, Hkv, hd)
        mk.paged_kv_scatter(src, kca, g["block_table"], g["seq_len"], g["start_pos"], 0, bs,
                            v_src=vsrc, v_cache=vca, v_bias=bv if bias else None)
    qb, kb, vb, kcb, vcb = (to_dev(x, dev) for x in (q, k, v, kc, vc))
    extra = (bq, bk, bv) if bias else ()
    mk.rope_kv_scatter(qb, kb, vb, pos, inv, kcb, vcb, 0, bs, dsegs, *extra)
    for name, a, b in (("q", qa, qb), ("k", ka, kb), ("k cache", kca, kcb),
                       ("v cache", vca, vcb)):
        assert_bits_equal(to_host(b), to_host(a), what=name)


def test_rope_kv_scatter_refusals(mk, orc, dev):
    import torch
    _case("rope + kv scatter refusals")
    rng = np.random.default_rng(9)
    bs, NB = 16, 40

    def bufs(T, Hq, Hkv, hd):
        q, k, v = (to_dev(normal_f16(rng, (T, h, hd)), dev) for h in (Hq, Hkv, Hkv))
        kc = torch.zeros((1, NB, Hkv, bs, hd), dtype=torch.float16, device=dev)
        return q, k, v, kc, torch.zeros_like(kc)

    segs = _dev_segs(_segments(rng, "ragged", 48, bs, NB), dev)
    pos = to_dev(rng.integers(0, 1000, 48).astype(np.int64), dev)
    # head_dim 6 and too many units per token: the separate entry points' shapes
    for Hq, Hkv, hd in ((4, 2, 6), (60, 8, 64)):
        q, k, v, kc, vc = bufs(48, Hq, Hkv, hd)
        with pytest.raises(RuntimeError, match="status -2"):
            mk.rope_kv_scatter(q, k, v, pos, orc.rope_inv_freq(hd), kc, vc, 0, bs, segs)
    q, k, v, kc, vc = bufs(48, 8, 2, 64)
    inv = orc.rope_inv_freq(64)
    with pytest.raises(RuntimeError, match="status -2"):  # nine segments
        mk.rope_kv_scatter(q, k, v, pos, inv, kc, vc, 0, bs, [segs[0]] * 9)
    with pytest.raises(RuntimeError, match="status -2"):  # overlapping token ranges
        mk.rope_kv_scatter(q, k, v, pos, inv, kc, vc, 0, bs,
                           [segs[0], dict(segs[0], token_offset=2)])
    with pytest.raises(RuntimeError, match="status -3"):  # K and V caches the same buffer
        mk.rope_kv_scatter(q, k, v, pos, inv, kc, kc, 0, bs, segs)
    with pytest.raises(RuntimeError, match="status -1"):  # segment past T
        mk.rope_kv_scatter(q, k, v, pos, inv, kc, vc, 0, bs, [dict(segs[0], token_offset=40)])
    bq = torch.zeros(8 * 64, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError, match="together"):
        mk.rope_kv_scatter(q, k, v, pos, inv, kc, vc, 0, bs, segs, q_bias=bq)
    # nothing written by a refused call
    assert int(torch.count_nonzero(kc)) == 0 and int(torch.count_nonzero(vc)) == 0


@pytest.mark.parametrize("T,Hq,Hkv,hd,kind", [
    (6064, 28, 4, 128, "chain"),   # the chain workload: Qwen2.5-7B heads, Gemma-3-style Q/K norm
    (48, 16, 8, 64, "ragged"),
    (48, 8, 4, 256, "ragged"),
    (48, 4, 2, 16, "ragged"),
    (48, 2, 1, 512, "ragged"),     # 32 lanes per head
    (20, 8, 8, 128, "none"),
])
@pytest.mark.parametrize("add_one", [False, True])
def test_qk_norm_rope_kv_scatter(mk, orc, dev, T, Hq, Hkv, hd, kind, add_one):
    _case(f"qk norm + rope + kv scatter T={T} Hq={Hq} Hkv={Hkv} hd={hd} {kind} "
          f"add_one={add_one}")
    rng = np.random.default_rng(T + Hq * 3 + hd + add_one)
    bs, L, layer = 16, 2, 1
    NB = 2100 if kind == "chain" else 40
    segs = _segments(rng, kind, T, bs, NB)
    q = normal_f16(rng, (T, Hq, hd), 0, 3)
    k = normal_f16(rng, (T, Hkv, hd), 0, 3)
    v = normal_f16(rng, (T, Hkv, hd))
    kc = normal_f16(rng, (L, NB, Hkv, bs, hd))
    vc = normal_f16(rng, (L, NB, Hkv, bs, hd))
    wq = normal_f16(rng, (hd,), 0 if add_one else 1, 0.1)
    wk = normal_f16(rng, (hd,), 0 if add_one else 1, 0.1)
    wq[3] = np.float16(-0.0)  # a -0 weight keeps the sign of zero through the norm
    pos = rng.integers(0, 32000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    posd, wqd, wkd = to_dev(pos, dev), to_dev(wq, dev), to_dev(wk, dev)
    dsegs = _dev_segs(segs, dev)
    # this library's two steps
    qa, ka, va, kca, vca = (to_dev(x, dev) for x in (q, k, v, kc, vc))
    mk.qk_norm_rope(qa, ka, wqd, wkd, posd, inv, eps=1e-6, add_one=add_one)
    for g in dsegs:
        B, S, o = g["block_table"].shape[0], g["S"], g["token_offset"]
        if B * S == 0:
            continue
        mk.paged_kv_scatter(ka[o:o + B * S].reshape(B, S, Hkv, hd), kca, g["block_table"],
                            g["seq_len"], g["start_pos"], layer, bs,
                            v_src=va[o:o + B * S].reshape(B, S, Hkv, hd), v_cache=vca)
    # one launch
    qb, kb, vb, kcb, vcb = (to_dev(x, dev) for x in (q, k, v, kc, vc))
    mk.qk_norm_rope_kv_scatter(qb, kb, vb, wqd, wkd, posd, inv, kcb, vcb, layer, bs, dsegs,
                               eps=1e-6, add_one=add_one)
    for name, a, b in (("q", qa, qb), ("k", ka, kb), ("k cache", kca, kcb),
                       ("v cache", vca, vcb)):
        assert_bits_equal(to_host(b), to_host(a), what=f"{name} vs qk_norm_rope + scatter")
    assert_bits_equal(to_host(vb), v, what="v source untouched")
    # the oracle: norm + RoPE within tolerance, cache placement bit-exact
    kh = to_host(kb)
    for x, w, got, what in ((q, wq, to_host(qb), "q"), (k, wk, kh, "k")):
        ref, n16 = qk_norm_rope_ref(orc, x, w, pos, inv, 1e-6, add_one)
        assert_norm_rope_close(got, ref, n16, what=f"{what} vs oracle")
    kcr, vcr = kc, vc
    for g in segs:
        B, S, o = g["block_table"].shape[0], g["S"], g["token_offset"]
        if B * S == 0:
            continue
        args = (g["block_table"], g["seq_len"], g["start_pos"], layer, bs)
        kcr = orc.paged_kv_scatter(kh[o:o + B * S].reshape(B, S, Hkv, hd), kcr, *args)
        vcr = orc.paged_kv_scatter(v[o:o + B * S].reshape(B, S, Hkv, hd), vcr, *args)
    assert_bits_equal(to_host(kcb), kcr, what="k cache vs oracle scatter")
    assert_bits_equal(to_host(vcb), vcr, what="v cache vs oracle scatter")


def test_qk_norm_rope_kv_scatter_refusals(mk, orc, dev):
    import torch
    _case("qk norm + rope + kv scatter refusals")
    rng = np.random.default_rng(10)
    bs, NB, T = 16, 40, 48
    segs = _dev_segs(_segments(rng, "ragged", T, bs, NB), dev)
    pos = to_dev(rng.integers(0, 1000, T).astype(np.int64), dev)
    hd = 48  # a multiple of 16 but not 16 * 2^k: no compile-time lane group
    q, k, v = (to_dev(normal_f16(rng, (T, h, hd)), dev) for h in (4, 2, 2))
    kc = torch.zeros((1, NB, 2, bs, hd), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    w = to_dev(normal_f16(rng, (hd,), 1, 0.1), dev)
    with pytest.raises(RuntimeError, match="status -2"):
        mk.qk_norm_rope_kv_scatter(q, k, v, w, w, pos, orc.rope_inv_freq(hd), kc, vc, 0, bs,
                                   segs)
    assert int(torch.count_nonzero(kc)) == 0 and int(torch.count_nonzero(vc)) == 0


@pytest.mark.parametrize("bias", [False, True])
def test_rope_kv_scatter_in_a_graph(mk, orc, dev, bias):
    """Captured once and replayed with q / k restored eagerly between the
    replays (they are rotated in place): every replay equals the eager call."""
    import torch
    _case(f"rope + kv scatter graph replays, bias={bias}")
    rng = np.random.default_rng(91 + bias)
    T, Hq, Hkv, hd, bs, NB = 48, 16, 8, 64, 16, 40
    segs = _dev_segs(_segments(rng, "ragged", T, bs, NB), dev)
    q, k, v = (normal_f16(rng, (T, h, hd)) for h in (Hq, Hkv, Hkv))
    pos = to_dev(rng.integers(0, 32000, T).astype(np.int64), dev)
    inv = orc.rope_inv_freq(hd, 1e6)
    extra = tuple(to_dev(normal_f16(rng, (h * hd,), 0, 0.5), dev) for h in (Hq, Hkv, Hkv)) \
        if bias else ()
    q0, k0 = to_dev(q, dev), to_dev(k, dev)
    qd, kd, vd = q0.clone(), k0.clone(), to_dev(v, dev)
    kc = torch.zeros((1, NB, Hkv, bs, hd), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    mk.rope_kv_scatter(qd, kd, vd, pos, inv, kc, vc, 0, bs, segs, *extra)
    torch.cuda.synchronize()
    want = [to_host(t) for t in (qd, kd, kc, vc)]
    qd.copy_(q0); kd.copy_(k0); kc.zero_(); vc.zero_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mk.rope_kv_scatter(qd, kd, vd, pos, inv, kc, vc, 0, bs, segs, *extra)
    for _ in range(3):
        qd.copy_(q0); kd.copy_(k0); kc.zero_(); vc.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("q", "k", "k cache", "v cache"), (qd, kd, kc, vc), want):
            assert_bits_equal(to_host(a), b, what=f"replay {name}")
    del graph
