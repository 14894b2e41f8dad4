"""GPU parity: NeoX RoPE (table-driven, table generation, fused Q+K from
positions) vs the CPU oracle.

Tables are compared bit for bit: both sides produce half(RN32(cos(angle))) of
the fp32 angle float(pos) * inv_freq[i] (src/kernels/rope_kernel.cu:74-76).
Rotated outputs are compared bit for bit as well: each output is one fp32
rounding of x1*c - x2*s whose products are exact, so any FMA contraction or
evaluation order gives the same fp32 value.  (The north-star tolerance,
rtol = atol = 1e-3, is therefore met with zero error.)
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import (assert_bits_equal, assert_close, assert_norm_rope_close, normal_f16,
                     qk_norm_rope_ref, to_dev, to_host)

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).resolve().parent / "golden" / "ref_cases.npz")


def _case(msg):
    print(f"[case] {msg}", flush=True)


def config3_positions(rng, total=4096, nseq=8, max_start=28000):
    """8 sequences of uniform-random lengths summing to `total`, each starting
    at a uniform offset in [0, max_start) (the RoPE benchmark workload)."""
    cuts = np.sort(rng.choice(np.arange(1, total), nseq - 1, replace=False))
    lengths = np.diff(np.concatenate([[0], cuts, [total]]))
    starts = rng.integers(0, max_start, nseq)
    return np.concatenate([s + np.arange(n) for s, n in zip(starts, lengths)]).astype(np.int64)


def test_reference_case(mk, orc, dev):
    """tests/test_rope/main.cpp:63-80: x [2,16,4,64] seed 101, positions seed
    2024 in [0, 4096] (replicated over the batch, src/layers/rope.cpp:66-71)."""
    _case("rope reference [2,16,4,64]")
    x = GOLD["rope_x"]
    B, S, H, D = x.shape
    inv = orc.rope_inv_freq(D, 1e6)
    assert (inv == GOLD["rope_inv_freq"]).all()
    pos = np.tile(GOLD["rope_pos"], B)
    c, s = mk.rope_tables(inv, to_dev(pos, dev))
    assert_bits_equal(to_host(c)[:S], GOLD["rope_cos"], what="cos table")
    assert_bits_equal(to_host(s)[:S], GOLD["rope_sin"], what="sin table")
    y = to_host(mk.rope_neox(to_dev(x, dev), c, s))
    assert_close(y, GOLD["rope_y"], what="rope vs golden")
    c_ref, s_ref = orc.rope_tables(inv, pos)
    assert_bits_equal(y, orc.rope_neox(x, c_ref, s_ref).astype(np.float16), what="rope vs oracle")


def test_tables_large_positions(mk, orc, dev):
    """Every position 0..32767 for head_dim 128: the fp16 tables are exact."""
    _case("rope tables 32768 x 64")
    inv = orc.rope_inv_freq(128, 1e6)
    pos = np.arange(32768, dtype=np.int64)
    c, s = mk.rope_tables(inv, to_dev(pos, dev))
    c_ref, s_ref = orc.rope_tables(inv, pos)
    assert_bits_equal(to_host(c), c_ref, what="cos")
    assert_bits_equal(to_host(s), s_ref, what="sin")


@pytest.mark.parametrize("lo,hi", [(1 << 20, 1 << 22), (1 << 22, 1 << 24),
                                   ((1 << 24) - 2048, (1 << 24) + 2048), (1 << 24, 1 << 40),
                                   (1 << 40, 1 << 62), (-(1 << 62), 0)])
def test_tables_huge_positions(mk, orc, dev, lo, hi):
    """Positions past 2^20 (angles beyond the fp32 sin/cos range, evaluated in
    fp64 directly; past 2^24 with the Payne-Hanek reduction), up to 2^62 and
    negative, theta 1e4 and 1e6: still bit-exact."""
    _case(f"rope tables positions in [{lo}, {hi})")
    rng = np.random.default_rng(abs(lo) % (1 << 32))
    pos = rng.integers(lo, hi, 4096).astype(np.int64)
    for theta in (1e4, 1e6):
        inv = orc.rope_inv_freq(128, theta)
        c, s = mk.rope_tables(inv, to_dev(pos, dev))
        c_ref, s_ref = orc.rope_tables(inv, pos)
        assert_bits_equal(to_host(c), c_ref, what=f"cos theta={theta}")
        assert_bits_equal(to_host(s), s_ref, what=f"sin theta={theta}")


def test_config3_fused_qk(mk, orc, dev):
    """The RoPE benchmark workload: Q [4096,28,128], K [4096,4,128] in place, theta 1e6."""
    _case("rope fused qk [4096,28|4,128]")
    rng = np.random.default_rng(33)
    T, Hq, Hkv, hd = 4096, 28, 4, 128
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    pos = config3_positions(rng)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    mk.rope_neox_qk(qd, kd, to_dev(pos, dev), inv)
    c, s = orc.rope_tables(inv, pos)
    assert_bits_equal(to_host(qd), orc.rope_neox(q, c, s, nthreads=8).astype(np.float16), what="q")
    assert_bits_equal(to_host(kd), orc.rope_neox(k, c, s, nthreads=8).astype(np.float16), what="k")


def test_fused_equals_tables_plus_rotation(mk, dev, orc):
    _case("rope fused == tables + rope_neox")
    rng = np.random.default_rng(34)
    T, Hq, Hkv, hd = 300, 28, 4, 128
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    pos = rng.integers(0, 32000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd, pd = to_dev(q, dev), to_dev(k, dev), to_dev(pos, dev)
    c, s = mk.rope_tables(inv, pd)
    yq = mk.rope_neox(to_dev(q, dev).view(1, T, Hq, hd), c, s)
    yk = mk.rope_neox(to_dev(k, dev).view(1, T, Hkv, hd), c, s)
    mk.rope_neox_qk(qd, kd, pd, inv)
    assert_bits_equal(to_host(qd), to_host(yq).reshape(T, Hq, hd), what="q")
    assert_bits_equal(to_host(kd), to_host(yk).reshape(T, Hkv, hd), what="k")


@pytest.mark.parametrize("T,Hq,Hkv,hd", [(1, 1, 0, 2), (7, 3, 1, 6), (5, 2, 2, 64), (64, 28, 4, 128),
                                         (3, 8, 1, 256), (2, 4, 2, 512), (9, 0, 3, 128)])
def test_shapes(mk, orc, dev, T, Hq, Hkv, hd):
    _case(f"rope fused T={T} Hq={Hq} Hkv={Hkv} hd={hd}")
    rng = np.random.default_rng(T * 1000 + hd)
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    pos = rng.integers(0, 32000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    mk.rope_neox_qk(qd, kd if Hkv else None, to_dev(pos, dev), inv)
    c, s = orc.rope_tables(inv, pos)
    if Hq:
        assert_bits_equal(to_host(qd), orc.rope_neox(q, c, s).astype(np.float16), what="q")
    if Hkv:
        assert_bits_equal(to_host(kd), orc.rope_neox(k, c, s).astype(np.float16), what="k")


# Shapes for the contiguous-row kernel (rope_rows_kernel): head_dim 64 / 128 /
# 256; 1-4 rounds of 256 vectors per token (R); every tokens-per-workgroup
# choice (1, 2, 4, 6, 8 on a 256-CU part) with a partial last workgroup; Q-only
# and K-only; a grid past 4 workgroups per CU; 1024 vectors (the largest it
# takes) and 1032 (past it: the one-token kernel).
@pytest.mark.parametrize("T,Hq,Hkv,hd", [
    (1, 28, 4, 128), (1029, 28, 4, 128), (2047, 28, 4, 128), (4099, 28, 4, 128),
    (8191, 28, 4, 128), (9001, 28, 4, 128), (2050, 8, 8, 128), (3000, 32, 8, 128),
    (700, 56, 8, 128), (1500, 12, 2, 64), (2100, 16, 8, 256), (77, 0, 8, 128),
    (100, 5, 0, 128), (33, 129, 0, 64)])
def test_rows_shapes(mk, orc, dev, T, Hq, Hkv, hd):
    _case(f"rope rows T={T} Hq={Hq} Hkv={Hkv} hd={hd}")
    rng = np.random.default_rng(T * 7 + Hq * 131 + hd)
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    pos = rng.integers(0, 40000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    mk.rope_neox_qk(qd, kd if Hkv else None, to_dev(pos, dev), inv)
    c, s = orc.rope_tables(inv, pos)
    if Hq:
        assert_bits_equal(to_host(qd), orc.rope_neox(q, c, s).astype(np.float16), what="q")
    if Hkv:
        assert_bits_equal(to_host(kd), orc.rope_neox(k, c, s).astype(np.float16), what="k")


def test_out_of_place_table_path(mk, orc, dev):
    _case("rope table path out of place")
    rng = np.random.default_rng(35)
    B, S, H, D = 3, 50, 5, 96
    x = normal_f16(rng, (B, S, H, D))
    pos = rng.integers(0, 10000, B * S).astype(np.int64)
    inv = orc.rope_inv_freq(D, 10000.0)
    c, s = orc.rope_tables(inv, pos)
    xd = to_dev(x, dev)
    y = mk.rope_neox(xd, to_dev(c, dev), to_dev(s, dev))
    assert_bits_equal(to_host(xd), x, what="input untouched")
    assert_bits_equal(to_host(y), orc.rope_neox(x, c, s).astype(np.float16), what="y")


def test_position_zero_is_identity(mk, orc, dev):
    _case("rope pos 0")
    rng = np.random.default_rng(36)
    q = normal_f16(rng, (4, 2, 128))
    qd = to_dev(q, dev)
    mk.rope_neox_qk(qd, None, to_dev(np.zeros(4, np.int64), dev), orc.rope_inv_freq(128, 1e6))
    assert_bits_equal(to_host(qd), q, what="identity")


@pytest.mark.parametrize("T,Hq,Hkv,hd", [(6064, 28, 4, 128), (37, 8, 2, 64), (5, 3, 1, 256),
                                         (9, 2, 2, 16), (3, 4, 0, 128), (4, 0, 2, 128),
                                         (2, 2, 1, 512), (11, 5, 3, 32), (20000, 8, 2, 64),
                                         (3001, 40, 8, 128), (500, 64, 32, 128),
                                         (50, 128, 16, 128)])
def test_qk_norm_rope(mk, orc, dev, T, Hq, Hkv, hd):
    """Fused Q/K RMSNorm + RoPE == the reference's norm-then-rope composition
    (src/layers/attention.cpp:754-780), within rtol = atol = 1e-3.  Shapes
    cover both launch forms: the pipelined kernel (at most 256 lanes per
    token) with token groups of 1 to 32 tokens, a ragged last group and
    groups walked several times per workgroup (T = 20000, 6064); and the
    one-round kernel at 48, 96 and 144 heads of 128 (384 to 1152 lanes per
    token, one to five units per lane)."""
    _case(f"qk_norm_rope T={T} Hq={Hq} Hkv={Hkv} hd={hd}")
    rng = np.random.default_rng(T * 7 + hd)
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    wq = normal_f16(rng, (hd,), 1.0, 0.1)
    wk = normal_f16(rng, (hd,), 1.0, 0.1)
    pos = rng.integers(0, 32000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    mk.qk_norm_rope(qd, kd if Hkv else None, to_dev(wq, dev), to_dev(wk, dev), to_dev(pos, dev), inv)
    if Hq:
        ref, n16 = qk_norm_rope_ref(orc, q, wq, pos, inv)
        assert_norm_rope_close(to_host(qd), ref, n16, what="q")
    if Hkv:
        ref, n16 = qk_norm_rope_ref(orc, k, wk, pos, inv)
        assert_norm_rope_close(to_host(kd), ref, n16, what="k")


def test_qk_norm_rope_huge_positions(mk, orc, dev):
    """Positions up to 2^23 and, every third token, up to 2^62: the in-kernel
    table takes the fp64 paths."""
    _case("qk_norm_rope positions up to 2^62")
    rng = np.random.default_rng(23)
    T, Hq, Hkv, hd = 300, 28, 4, 128
    q = normal_f16(rng, (T, Hq, hd)); k = normal_f16(rng, (T, Hkv, hd))
    wq = normal_f16(rng, (hd,), 1.0, 0.1); wk = normal_f16(rng, (hd,), 1.0, 0.1)
    pos = rng.integers(0, 1 << 23, T).astype(np.int64)
    pos[::3] = rng.integers(1 << 24, 1 << 62, len(pos[::3]))  # Payne-Hanek path
    inv = orc.rope_inv_freq(hd, 1e4)
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    mk.qk_norm_rope(qd, kd, to_dev(wq, dev), to_dev(wk, dev), to_dev(pos, dev), inv)
    assert_norm_rope_close(to_host(qd), *qk_norm_rope_ref(orc, q, wq, pos, inv), what="q")
    assert_norm_rope_close(to_host(kd), *qk_norm_rope_ref(orc, k, wk, pos, inv), what="k")


def test_qk_norm_rope_vs_two_launches(mk, orc, dev):
    """Against this library's own two-launch sequence (rmsnorm then rope):
    identical except where the normalised fp16 value sits on a rounding
    boundary (different fp32 summation order), never more than 1 ulp there."""
    _case("qk_norm_rope vs rmsnorm + rope_neox_qk")
    rng = np.random.default_rng(71)
    T, Hq, Hkv, hd = 512, 28, 4, 128
    q = normal_f16(rng, (T, Hq, hd)); k = normal_f16(rng, (T, Hkv, hd))
    wq = normal_f16(rng, (hd,), 1.0, 0.1); wk = normal_f16(rng, (hd,), 1.0, 0.1)
    pos = rng.integers(0, 32000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    wqd, wkd, pd = to_dev(wq, dev), to_dev(wk, dev), to_dev(pos, dev)
    q1, k1 = to_dev(q, dev), to_dev(k, dev)
    mk.qk_norm_rope(q1, k1, wqd, wkd, pd, inv)
    q2, k2 = to_dev(q, dev), to_dev(k, dev)
    mk.rmsnorm(q2.view(T * Hq, hd), wqd, y=q2.view(T * Hq, hd))
    mk.rmsnorm(k2.view(T * Hkv, hd), wkd, y=k2.view(T * Hkv, hd))
    mk.rope_neox_qk(q2, k2, pd, inv)
    a, b = to_host(q1), to_host(q2)
    assert_close(a, b.astype(np.float32), what="q vs two launches")
    assert (a.view(np.uint16) == b.view(np.uint16)).mean() > 0.99


def _bias_ref(orc, x, bias):
    T = x.shape[0]
    n = x.shape[1] * x.shape[2]
    return orc.add_bias(x.reshape(-1), bias, T, n, T * n).reshape(x.shape)


@pytest.mark.parametrize("T,Hq,Hkv,hd,chain", [(6064, 28, 4, 128, True), (4096, 28, 4, 128, False),
                                               (7, 3, 1, 6, False), (5, 0, 2, 64, False),
                                               (3, 8, 1, 256, False)])
def test_bias_rope(mk, orc, dev, T, Hq, Hkv, hd, chain):
    """Qwen2's q_proj / k_proj bias with the rotation in one pass, bit-exact
    against launch_add_bias followed by RoPE (attention.cpp:717-780): at the
    chain's tokens and positions, the RoPE workload's, a head_dim of 6 (scalar path)
    and K-only."""
    _case(f"bias + rope T={T} Hq={Hq} Hkv={Hkv} hd={hd}")
    rng = np.random.default_rng(T + Hq * 10 + hd)
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    bq = normal_f16(rng, (Hq * hd,), 0, 0.5)
    bk = normal_f16(rng, (Hkv * hd,), 0, 0.5)
    if chain:
        dec = rng.integers(0, 28000, 64)
        pos = np.concatenate([dec, 100 + np.arange(3000), 9000 + np.arange(3000)]).astype(np.int64)
    elif T == 4096:
        pos = config3_positions(rng)
    else:
        pos = rng.integers(0, 32000, T).astype(np.int64)
    inv = orc.rope_inv_freq(hd, 1e6)
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    mk.bias_rope_neox_qk(qd, kd if Hkv else None, to_dev(bq, dev), to_dev(bk, dev) if Hkv else None,
                         to_dev(pos, dev), inv)
    c, s = orc.rope_tables(inv, pos)
    if Hq:
        want = orc.rope_neox(_bias_ref(orc, q, bq), c, s, nthreads=8).astype(np.float16)
        assert_bits_equal(to_host(qd), want, what="q")
    if Hkv:
        want = orc.rope_neox(_bias_ref(orc, k, bk), c, s, nthreads=8).astype(np.float16)
        assert_bits_equal(to_host(kd), want, what="k")


def test_bias_rope_equals_two_launches(mk, orc, dev):
    """The fused pass against this library's own add_bias + rope_neox_qk."""
    _case("bias + rope == add_bias + rope_neox_qk")
    rng = np.random.default_rng(77)
    T, Hq, Hkv, hd = 500, 28, 4, 128
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    bq = normal_f16(rng, (Hq * hd,), 0, 2)
    bk = normal_f16(rng, (Hkv * hd,), 0, 2)
    pos = to_dev(rng.integers(0, 1 << 20, T).astype(np.int64), dev)
    inv = orc.rope_inv_freq(hd, 1e6)
    qa, ka = to_dev(q, dev), to_dev(k, dev)
    mk.add_bias(qa, to_dev(bq, dev), T, Hq * hd, T * Hq * hd)
    mk.add_bias(ka, to_dev(bk, dev), T, Hkv * hd, T * Hkv * hd)
    mk.rope_neox_qk(qa, ka, pos, inv)
    qb, kb = to_dev(q, dev), to_dev(k, dev)
    mk.bias_rope_neox_qk(qb, kb, to_dev(bq, dev), to_dev(bk, dev), pos, inv)
    assert_bits_equal(to_host(qb), to_host(qa), what="q")
    assert_bits_equal(to_host(kb), to_host(ka), what="k")
