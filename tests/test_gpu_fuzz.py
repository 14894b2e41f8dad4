"""GPU parity over seeded random shapes: every kernel, many small cases.

Each case draws its shape and options from a fixed-seed generator, so a
failure names a reproducible case.  The draws reach the paths the fixed-shape
tests pin one at a time:
* vector (16-byte) and scalar paths: sizes not a multiple of 8, and buffers
  misaligned by one fp16 element (a contiguous view at storage offset 1);
* in-place and out-of-place calls;
* split and whole rows for softmax / argmax, and many long softmax rows
  (the persistent one-launch form, rows in rounds);
* invalid ids and KV blocks, and random segment tables for the one-launch
  RoPE + K/V scatter;
* ties, NaN and -inf in argmax rows.
The bar is the same as everywhere: bit-exact for copies, RoPE and argmax;
rtol = atol = 1e-3 for the fp32-math outputs (norm-then-rope with its
documented one-ulp intermediate allowance).
"""
import os

import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close, normal_f16, to_host

pytestmark = pytest.mark.gpu
CASES = int(os.environ.get("MI_FUZZ_CASES", "32"))  # a deeper run: MI_FUZZ_CASES=256


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _dev_array(a, dev, misalign=False):
    """`a` on the device, optionally at a 2-byte-misaligned address."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if not misalign:
        return t.to(dev)
    flat = torch.empty(t.numel() + 1, dtype=t.dtype, device=dev)
    view = flat[1:].view(t.shape)
    view.copy_(t.to(dev))
    return view


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_rmsnorm(mk, orc, dev, seed):
    rng = np.random.default_rng(1000 + seed)
    N = int(rng.integers(1, 200))
    D = int(rng.choice([int(rng.integers(1, 600)), 8 * int(rng.integers(1, 1200)),
                        int(rng.integers(600, 9000))]))
    add_one = bool(rng.integers(0, 2))
    mis = bool(rng.integers(0, 4) == 0)
    inplace = bool(rng.integers(0, 2))
    _case(f"rmsnorm seed={seed} N={N} D={D} add_one={add_one} misaligned={mis} inplace={inplace}")
    x, w = normal_f16(rng, (N, D)), normal_f16(rng, (D,), 1.0, 0.1)
    xd = _dev_array(x, dev, mis)
    y = mk.rmsnorm(xd, _dev_array(w, dev), y=xd if inplace else None, add_one=add_one)
    assert_close(to_host(y), orc.rmsnorm(x, w, add_one=add_one), what="rmsnorm")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_fused_add_rmsnorm(mk, orc, dev, seed):
    rng = np.random.default_rng(2000 + seed)
    N = int(rng.integers(1, 200))
    D = int(rng.choice([int(rng.integers(1, 600)), 8 * int(rng.integers(1, 1200))]))
    add_one = bool(rng.integers(0, 2))
    mis = bool(rng.integers(0, 4) == 0)
    _case(f"fused_add_rmsnorm seed={seed} N={N} D={D} add_one={add_one} misaligned={mis}")
    x, r = normal_f16(rng, (N, D)), normal_f16(rng, (N, D))
    w = normal_f16(rng, (D,), 1.0, 0.1)
    rd = _dev_array(r, dev, mis)
    y = mk.fused_add_rmsnorm(_dev_array(x, dev, mis), rd, _dev_array(w, dev), add_one=add_one)
    r_ref, y_ref = orc.fused_add_rmsnorm(x, r, w, add_one=add_one)
    assert_bits_equal(to_host(rd), r_ref, what="residual")
    assert_close(to_host(y), y_ref, what="y")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_rope_qk(mk, orc, dev, seed):
    rng = np.random.default_rng(3000 + seed)
    T = int(rng.integers(1, 300))
    hd = int(rng.choice([2, 6, 16, 32, 64, 96, 128, 256, 512]))
    Hq, Hkv = int(rng.integers(0, 40)), int(rng.integers(0, 9))
    if Hq + Hkv == 0:
        Hq = 1
    theta = float(rng.choice([1e4, 1e6]))
    _case(f"rope_neox_qk seed={seed} T={T} Hq={Hq} Hkv={Hkv} hd={hd} theta={theta}")
    q, k = normal_f16(rng, (T, Hq, hd)), normal_f16(rng, (T, Hkv, hd))
    pos = rng.integers(0, 1 << int(rng.integers(4, 22)), T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, theta)
    qd, kd = _dev_array(q, dev), _dev_array(k, dev)
    mk.rope_neox_qk(qd, kd if Hkv else None, _dev_array(pos, dev), inv)
    c, s = orc.rope_tables(inv, pos)
    if Hq:
        assert_bits_equal(to_host(qd), orc.rope_neox(q, c, s).astype(np.float16), what="q")
    if Hkv:
        assert_bits_equal(to_host(kd), orc.rope_neox(k, c, s).astype(np.float16), what="k")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_qk_norm_rope(mk, orc, dev, seed):
    from helpers import assert_norm_rope_close, qk_norm_rope_ref
    rng = np.random.default_rng(4000 + seed)
    T = int(rng.integers(1, 400))
    hd = int(rng.choice([16, 32, 64, 128, 256, 512]))
    Hq, Hkv = int(rng.integers(0, 50)), int(rng.integers(0, 9))
    if Hq + Hkv == 0:
        Hkv = 1
    _case(f"qk_norm_rope seed={seed} T={T} Hq={Hq} Hkv={Hkv} hd={hd}")
    q, k = normal_f16(rng, (T, Hq, hd)), normal_f16(rng, (T, Hkv, hd))
    wq, wk = normal_f16(rng, (hd,), 1.0, 0.1), normal_f16(rng, (hd,), 1.0, 0.1)
    pos = rng.integers(0, 40000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd = _dev_array(q, dev), _dev_array(k, dev)
    mk.qk_norm_rope(qd, kd if Hkv else None, _dev_array(wq, dev), _dev_array(wk, dev),
                    _dev_array(pos, dev), inv)
    if Hq:
        assert_norm_rope_close(to_host(qd), *qk_norm_rope_ref(orc, q, wq, pos, inv), what="q")
    if Hkv:
        assert_norm_rope_close(to_host(kd), *qk_norm_rope_ref(orc, k, wk, pos, inv), what="k")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_activations(mk, orc, dev, seed):
    rng = np.random.default_rng(5000 + seed)
    n = int(rng.choice([int(rng.integers(1, 100)), int(rng.integers(100, 200000)),
                        8 * int(rng.integers(1, 100000))]))
    mis = bool(rng.integers(0, 4) == 0)
    _case(f"activations seed={seed} n={n} misaligned={mis}")
    g, u = normal_f16(rng, (n,), 0.0, 3.0), normal_f16(rng, (n,))
    gd, ud = _dev_array(g, dev, mis), _dev_array(u, dev, mis)
    assert_close(to_host(mk.swiglu(gd, ud)), orc.swiglu(g, u), what="swiglu")
    assert_close(to_host(mk.geglu(gd, ud)), orc.geglu(g, u), what="geglu")
    assert_close(to_host(mk.gelu_tanh(gd)), orc.gelu_tanh(g), what="gelu_tanh")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_softmax(mk, orc, dev, seed):
    rng = np.random.default_rng(6000 + seed)
    split = bool(rng.integers(0, 2))
    N = int(rng.integers(1, 64)) if split else int(rng.integers(1, 700))
    D = (int(rng.integers(8192, 300000)) if split
         else int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 8192)),
                              8 * int(rng.integers(1, 1024))])))
    pick = int(rng.integers(0, 8)) if not split else -1
    if pick in (0, 1):  # many rows of up to 65536 (register rows, or persistent past 32768)
        N, D = int(rng.integers(512, 1200)), 8 * int(rng.integers(1, 8193))
    elif pick == 2:  # many long rows (persistent one-launch form; rounds of rows)
        N, D = int(rng.integers(100, 900)), int(rng.integers(32769, 200000))
        if rng.integers(0, 2):
            D -= D % 8
    mis = bool(rng.integers(0, 4) == 0)
    inplace = bool(rng.integers(0, 4) == 0)
    _case(f"softmax seed={seed} N={N} D={D} misaligned={mis} inplace={inplace}")
    x = normal_f16(rng, (N, D), 0.0, 4.0)
    xd = _dev_array(x, dev, mis)
    y = mk.softmax(xd, y=xd if inplace else None)
    assert_close(to_host(y), orc.softmax(x, nthreads=8), what="softmax")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_gather(mk, orc, dev, seed):
    rng = np.random.default_rng(7000 + seed)
    T = int(rng.integers(1, 500))
    H = int(rng.choice([int(rng.integers(1, 300)), 8 * int(rng.integers(1, 600)),
                        8 * int(rng.integers(600, 2100))]))  # up to 4 waves per row
    V = int(rng.integers(1, 3000))
    mis = bool(rng.integers(0, 4) == 0)
    _case(f"gather seed={seed} T={T} H={H} V={V} misaligned={mis}")
    table = normal_f16(rng, (V, H), 0.0, 0.02)
    ids = rng.integers(-3, V + 3, T).astype(np.int64)
    out = mk.embedding_gather(_dev_array(ids, dev), _dev_array(table, dev, mis))
    assert_bits_equal(to_host(out), orc.embedding_gather(ids, table), what="gather")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_argmax(mk, orc, dev, seed):
    rng = np.random.default_rng(8000 + seed)
    split = bool(rng.integers(0, 2))
    B = int(rng.integers(1, 64)) if split else int(rng.integers(1, 700))
    V = int(rng.integers(8192, 200000)) if split else int(rng.integers(1, 8192))
    if not split and rng.integers(0, 4) == 0:  # whole long rows (deep tiles)
        B, V = int(rng.integers(512, 700)), int(rng.integers(16384, 70000))
    levels = int(rng.choice([0, 1, 3, 50]))
    _case(f"argmax seed={seed} B={B} V={V} levels={levels}")
    if levels:
        x = rng.integers(-levels, levels + 1, (B, V)).astype(np.float16)
    else:
        x = normal_f16(rng, (B, V), 0.0, 4.0)
    special = rng.random((B, V))
    x[special < 0.001] = np.nan
    x[(special >= 0.001) & (special < 0.002)] = -np.inf
    got = to_host(mk.greedy_argmax(_dev_array(x, dev)))
    ref = orc.greedy_argmax(x)
    assert (got == ref).all(), f"{int((got != ref).sum())} rows differ"


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_kv_scatter(mk, orc, dev, seed):
    rng = np.random.default_rng(9000 + seed)
    B = int(rng.integers(1, 9))
    S = int(rng.integers(1, 70))
    H = int(rng.integers(1, 9))
    D = int(rng.choice([6, 8, 64, 128, 136]))
    bs = int(rng.choice([1, 4, 16, 32]))
    L = int(rng.integers(1, 4))
    starts = rng.integers(0, 200, B)
    seqs = starts + rng.integers(0, S + 20, B)
    mb = max(1, -(-int(seqs.max() + 1) // bs))
    NB = B * mb + 2
    _case(f"kv scatter seed={seed} B={B} S={S} H={H} D={D} bs={bs} L={L}")
    src = normal_f16(rng, (B, S, H, D))
    cache = normal_f16(rng, (L, NB, H, bs, D))
    # distinct physical blocks (two tokens on one cache slot would race, in the
    # reference too), ~10% of entries invalid: -1 or past num_blocks
    bt = rng.permutation(NB)[:B * mb].reshape(B, mb).astype(np.int32)
    bad = rng.random((B, mb)) < 0.1
    bt[bad] = rng.choice([-1, NB, NB + 7], int(bad.sum())).astype(np.int32)
    sl, sp = seqs.astype(np.int32), starts.astype(np.int32)
    layer = int(rng.integers(0, L))
    cd = _dev_array(cache, dev)
    mk.paged_kv_scatter(_dev_array(src, dev), cd, _dev_array(bt, dev), _dev_array(sl, dev),
                        _dev_array(sp, dev), layer=layer, block_size=bs)
    assert_bits_equal(to_host(cd), orc.paged_kv_scatter(src, cache, bt, sl, sp, layer, bs),
                      what="cache")


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_bias_paths(mk, orc, dev, seed):
    """Qwen2's QKV bias: the bias add alone (batches, gaps, misaligned y), fused
    into RoPE (bit-exact against add_bias + rope), and the Q/K norm pair in one
    launch against the oracle."""
    rng = np.random.default_rng(11000 + seed)
    # add_bias
    M, N = int(rng.integers(1, 200)), int(rng.choice([int(rng.integers(1, 100)), 8 * int(rng.integers(1, 600))]))
    batches, gap = int(rng.integers(1, 4)), int(rng.choice([0, 0, int(rng.integers(1, 40))]))
    mis = bool(rng.integers(0, 4) == 0)
    stride = M * N + gap
    _case(f"bias seed={seed} add_bias M={M} N={N} batches={batches} gap={gap} misaligned={mis}")
    y = normal_f16(rng, ((batches - 1) * stride + M * N,), 0, 20)
    b = normal_f16(rng, (N,), 0, 20)
    yd = _dev_array(y, dev, mis)
    mk.add_bias(yd, _dev_array(b, dev), M, N, stride)
    assert_bits_equal(to_host(yd), orc.add_bias(y, b, M, N, stride), what="add_bias")
    # bias + rope
    T = int(rng.integers(1, 300))
    hd = int(rng.choice([2, 6, 16, 64, 128, 256]))
    Hq, Hkv = int(rng.integers(0, 30)), int(rng.integers(0, 6))
    if Hq + Hkv == 0:
        Hq = 1
    _case(f"bias seed={seed} bias_rope T={T} Hq={Hq} Hkv={Hkv} hd={hd}")
    q, k = normal_f16(rng, (T, Hq, hd)), normal_f16(rng, (T, Hkv, hd))
    bq, bk = normal_f16(rng, (Hq * hd,), 0, 1), normal_f16(rng, (Hkv * hd,), 0, 1)
    pos = rng.integers(0, 1 << int(rng.integers(4, 22)), T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd = _dev_array(q, dev), _dev_array(k, dev)
    if Hq:
        mk.bias_rope_neox_qk(qd, kd if Hkv else None, _dev_array(bq, dev),
                             _dev_array(bk, dev) if Hkv else None, _dev_array(pos, dev), inv)
    else:  # K alone goes in the Q slot of the binding
        mk.bias_rope_neox_qk(kd, None, _dev_array(bk, dev), None, _dev_array(pos, dev), inv)
    c, s = orc.rope_tables(inv, pos)
    for name, x, bz, got in (("q", q, bq, qd), ("k", k, bk, kd)):
        if x.shape[1] == 0:
            continue
        n = x.shape[1] * hd
        xb = orc.add_bias(x.reshape(-1), bz, T, n, T * n).reshape(x.shape)
        assert_bits_equal(to_host(got), orc.rope_neox(xb, c, s).astype(np.float16), what=name)
    # Q/K norm in one launch
    hd2 = int(rng.choice([8, 16, 64, 128, 256, 512, 40]))
    T2, Hq2, Hkv2 = int(rng.integers(1, 200)), int(rng.integers(1, 30)), int(rng.integers(0, 6))
    add_one = bool(rng.integers(0, 2))
    _case(f"bias seed={seed} qk_rmsnorm T={T2} Hq={Hq2} Hkv={Hkv2} hd={hd2} add_one={add_one}")
    q2, k2 = normal_f16(rng, (T2, Hq2, hd2)), normal_f16(rng, (T2, Hkv2, hd2))
    wq, wk = normal_f16(rng, (hd2,), 1.0, 0.1), normal_f16(rng, (hd2,), 1.0, 0.1)
    qd2, kd2 = _dev_array(q2, dev), _dev_array(k2, dev)
    mk.qk_rmsnorm(qd2, kd2 if Hkv2 else None, _dev_array(wq, dev),
                  _dev_array(wk, dev) if Hkv2 else None, add_one=add_one)
    assert_close(to_host(qd2).reshape(-1, hd2), orc.rmsnorm(q2.reshape(-1, hd2), wq, add_one=add_one),
                 what="q norm")
    if Hkv2:
        assert_close(to_host(kd2).reshape(-1, hd2),
                     orc.rmsnorm(k2.reshape(-1, hd2), wk, add_one=add_one), what="k norm")


def _fuzz_segments(rng, T, bs):
    """Up to 8 segments over disjoint token ranges of [0, T) (gaps between
    them), ragged sequences (some stop before S), distinct blocks with a few
    unmapped (-1) or out-of-range ids; returns (segments, num_blocks)."""
    nseg = int(rng.integers(0, 9))
    cuts = np.sort(rng.choice(np.arange(T + 1), size=min(2 * nseg, T + 1), replace=False))
    segs, nxt, raw = [], 0, []
    for a, b in zip(cuts[0::2], cuts[1::2]):
        n = int(b - a)
        S = int(rng.integers(1, min(n, 48) + 1))  # small caches: B <= 6, positions < 88
        B = int(rng.integers(1, min(n // S, 6) + 1))
        start = rng.integers(0, 40, B)
        sl = start + S - rng.integers(0, 3, B)
        mb = max(1, -(-int(sl.max()) // bs))
        raw.append((int(a), B, S, start, sl, mb, nxt))
        nxt += B * mb
    NB = max(1, nxt)
    perm = rng.permutation(NB)
    for a, B, S, start, sl, mb, off in raw:
        bt = perm[off:off + B * mb].reshape(B, mb).astype(np.int32)
        for _ in range(int(rng.integers(0, 3))):
            bt[rng.integers(0, B), rng.integers(0, mb)] = rng.choice([-1, NB + 3])
        segs.append(dict(token_offset=a, S=S, block_table=bt, seq_len=sl.astype(np.int32),
                         start_pos=start.astype(np.int32)))
    return segs, NB


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_rope_kv_scatter(mk, orc, dev, seed):
    """RoPE + K/V into the paged cache in one launch (plain, QKV bias, Q/K
    norm) against this library's separate launches, bit for bit, over random
    head layouts, head_dims and segment tables."""
    import torch
    rng = np.random.default_rng(12000 + seed)
    mode = ("plain", "bias", "norm")[seed % 3]
    while True:
        hd = int(rng.choice([16, 32, 64, 128, 256]))
        Hkv = int(rng.integers(1, 9))
        Hq = Hkv * int(rng.integers(1, 8))
        if (Hq + Hkv) * hd // 16 <= 256:
            break
    T, bs, L = int(rng.integers(1, 300)), int(rng.choice([1, 4, 16, 32])), 2
    layer = int(rng.integers(0, L))
    segs, NB = _fuzz_segments(rng, T, bs)
    _case(f"rope_kv seed={seed} {mode} T={T} Hq={Hq} Hkv={Hkv} hd={hd} bs={bs} "
          f"segments={len(segs)} NB={NB}")
    q, k, v = (normal_f16(rng, (T, h, hd)) for h in (Hq, Hkv, Hkv))
    kc, vc = (normal_f16(rng, (L, NB, Hkv, bs, hd)) for _ in range(2))
    pos = rng.integers(0, 1 << int(rng.integers(4, 20)), T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    posd = _dev_array(pos, dev)
    dsegs = [dict(g, block_table=_dev_array(g["block_table"], dev),
                  seq_len=_dev_array(g["seq_len"], dev), start_pos=_dev_array(g["start_pos"], dev))
             for g in segs]
    bias = [_dev_array(normal_f16(rng, (h * hd,), 0, 1), dev) for h in (Hq, Hkv, Hkv)]
    w = [_dev_array(normal_f16(rng, (hd,), 1, 0.1), dev) for _ in range(2)]
    qa, ka, va, kca, vca = (_dev_array(x, dev) for x in (q, k, v, kc, vc))
    if mode == "plain":
        mk.rope_neox_qk(qa, ka, posd, inv)
    elif mode == "bias":
        mk.bias_rope_neox_qk(qa, ka, bias[0], bias[1], posd, inv)
    else:
        mk.qk_norm_rope(qa, ka, w[0], w[1], posd, inv)
    for g in dsegs:
        B, S, o = g["block_table"].shape[0], g["S"], g["token_offset"]
        mk.paged_kv_scatter(ka[o:o + B * S].reshape(B, S, Hkv, hd), kca, g["block_table"],
                            g["seq_len"], g["start_pos"], layer, bs,
                            v_src=va[o:o + B * S].reshape(B, S, Hkv, hd), v_cache=vca,
                            v_bias=bias[2] if mode == "bias" else None)
    qb, kb, vb, kcb, vcb = (_dev_array(x, dev) for x in (q, k, v, kc, vc))
    if mode == "norm":
        mk.qk_norm_rope_kv_scatter(qb, kb, vb, w[0], w[1], posd, inv, kcb, vcb, layer, bs, dsegs)
    else:
        extra = bias if mode == "bias" else ()
        mk.rope_kv_scatter(qb, kb, vb, posd, inv, kcb, vcb, layer, bs, dsegs, *extra)
    torch.cuda.synchronize()
    for name, a, b in (("q", qa, qb), ("k", ka, kb), ("k cache", kca, kcb),
                       ("v cache", vca, vcb), ("v", va, vb)):
        assert_bits_equal(to_host(b), to_host(a), what=name)


@pytest.mark.parametrize("seed", range(CASES))
def test_fuzz_top_p(mk, orc, dev, seed):
    """Top-p sampling against the oracle over random batch sizes,
    vocabularies either side of the 30000 greedy boundary, p, temperature
    and seeds; rows whose outcome sits near a rounding boundary of the fp32
    probabilities are redrawn (tests/test_gpu_top_p.py states the screen)."""
    from test_gpu_top_p import _safe
    rng = np.random.default_rng(13000 + seed)
    B = int(rng.integers(1, 40))
    V = int(rng.choice([int(rng.integers(1, 30001)), int(rng.integers(30001, 160000))]))
    p = float(rng.choice([0.05, 0.3, 0.7, 0.9, 0.99]))
    T = float(rng.choice([0.5, 0.8, 1.0, 1.7]))
    draw = int(rng.integers(0, 1 << 62))
    _case(f"top-p seed={seed} B={B} V={V} p={p} T={T}")
    rows = []
    while len(rows) < B:
        x = normal_f16(rng, (V,), 0, float(rng.choice([0.5, 2, 6])))
        if V <= 30000:
            nc = (V + 127) // 128
            hot = rng.choice(np.arange(0, V, 128), size=min(int(rng.integers(0, 6)), nc),
                             replace=False)
            x[hot] = (rng.random(hot.size) * 10).astype(np.float16)
            if not _safe(x, p, T):
                continue
        rows.append(x)
    x = np.stack(rows)
    got = to_host(mk.top_p_sample(_dev_array(x, dev, misalign=bool(rng.integers(0, 2))), p, T,
                                  draw))
    np.testing.assert_array_equal(got, orc.top_p_sample(x, p, T, draw))
