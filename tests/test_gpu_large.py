"""GPU parity past 2^31 elements: every kernel family on a tensor whose
element (and byte) offsets do not fit 32 bits, so any 32-bit index or offset
on the way shows up as a wrong or missing result.

Inputs are generated on the device (seeded); only slices are brought back --
at the start, around element 2^31 and at the end -- and checked against the
oracle on those slices, to the same bar as everywhere: bit-exact for copies,
residual sums, RoPE, argmax and the KV scatter; rtol = atol = 1e-3 for the
fp32-math outputs.  Each test frees its buffers before the next (peak ~13 GB
of the GPU's 288 GB).
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close, to_host

pytestmark = pytest.mark.gpu

BIG = 1 << 31


def _case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(autouse=True)
def _needs_memory(dev):
    import torch
    free, _ = torch.cuda.mem_get_info(dev)
    if free < (40 << 30):
        pytest.skip("needs 40 GB of free device memory")
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _randn16(dev, n, seed, std=1.0, mean=0.0):
    """n seeded ~N(mean, std) fp16 values on the device, made in slices."""
    import torch
    t = torch.empty(n, dtype=torch.float16, device=dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    step = 1 << 27
    for i in range(0, n, step):
        m = min(step, n - i)
        t[i:i + m] = (torch.randn(m, generator=g, device=dev) * std + mean).half()
    return t


def _spots(n, w):
    """Index windows [a, a + w) at the start, around 2^31 and at the end."""
    return [0, BIG - w // 2, n - w]


@pytest.mark.parametrize("n", [BIG + 4104, BIG + 5])  # vector and scalar paths
def test_large_elementwise(mk, orc, dev, n):
    _case(f"elementwise n={n}")
    g = _randn16(dev, n, 1, 3.0)
    u = _randn16(dev, n, 2)
    out = mk.swiglu(g, u)
    for a in _spots(n, 4096):
        sl = slice(a, a + 4096)
        gh, uh = to_host(g[sl]), to_host(u[sl])
        assert_close(to_host(out[sl]), orc.swiglu(gh, uh), what=f"swiglu @{a}")
    mk.geglu(g, u, out=out)
    a = BIG - 2048
    gh, uh = to_host(g[a:a + 4096]), to_host(u[a:a + 4096])
    assert_close(to_host(out[a:a + 4096]), orc.geglu(gh, uh), what="geglu @2^31")
    keep = {a: to_host(u[a:a + 4096]) for a in _spots(n, 4096)}
    mk.add_inplace(u, g)
    for a, uh in keep.items():
        assert_bits_equal(to_host(u[a:a + 4096]), orc.add(uh, to_host(g[a:a + 4096])),
                          what=f"add_inplace @{a}")
    del g, u, out


def test_large_fused_add_rmsnorm(mk, orc, dev):
    N, D = 600000, 3584  # 2.15e9 elements per tensor
    _case(f"fused add + rmsnorm [{N},{D}]")
    x = _randn16(dev, N * D, 3).view(N, D)
    r = _randn16(dev, N * D, 4).view(N, D)
    w = _randn16(dev, D, 5, 0.1, 1.0)
    rows = [0, BIG // D, N - 3]  # the second straddles element 2^31
    r_before = {i: to_host(r[i:i + 3]) for i in rows}
    y = mk.fused_add_rmsnorm(x, r, w)
    wh = to_host(w)
    for i in rows:
        xh = to_host(x[i:i + 3])
        ref_r, ref_y = orc.fused_add_rmsnorm(xh, r_before[i], wh)
        assert_bits_equal(to_host(r[i:i + 3]), ref_r, what=f"residual rows {i}..")
        assert_close(to_host(y[i:i + 3]), ref_y, what=f"y rows {i}..")
    del x, r, y


def test_large_softmax(mk, orc, dev):
    N, V = 16384, 152064  # 2.49e9 elements
    _case(f"softmax [{N},{V}]")
    x = _randn16(dev, N * V, 6, 4.0).view(N, V)
    y = mk.softmax(x)
    for i in (0, BIG // V, N - 1):
        xh = to_host(x[i:i + 1])
        assert_close(to_host(y[i:i + 1]), orc.softmax(xh), what=f"softmax row {i}")
    del x, y


def test_large_argmax(mk, orc, dev):
    import torch
    B, V = 16384, 152064
    _case(f"greedy argmax [{B},{V}]")
    x = _randn16(dev, B * V, 7, 4.0).view(B, V)
    rows = [0, BIG // V, BIG // V + 1, B - 1]
    x[rows[1], V - 1] = 60.0  # maxima placed past element 2^31
    x[rows[3], 12345] = 60.0
    out = mk.greedy_argmax(x)
    got = to_host(out)
    for i in rows:
        assert int(got[i]) == int(orc.greedy_argmax(to_host(x[i:i + 1]))[0]), f"row {i}"
    assert int(got[rows[1]]) == V - 1 and int(got[rows[3]]) == 12345
    del x, out
    torch.cuda.synchronize()


def test_large_gather(mk, dev):
    import torch
    Vb, H = 640000, 3584  # a 2.29e9-element table
    _case(f"embedding gather from [{Vb},{H}]")
    table = _randn16(dev, Vb * H, 8, 0.02).view(Vb, H)
    ids_h = np.array([0, 1, BIG // H, BIG // H + 1, Vb - 2, Vb - 1] * 4, dtype=np.int64)
    ids = torch.from_numpy(ids_h).to(dev)
    out = mk.embedding_gather(ids, table)
    for t, i in enumerate(ids_h):
        assert_bits_equal(to_host(out[t]), to_host(table[int(i)]), what=f"row {i}")
    del table, out


def test_large_rope(mk, orc, dev):
    import torch
    T, Hq, Hkv, hd = 600000, 28, 4, 128  # q: 2.15e9 elements
    _case(f"rope Q [{T},{Hq},{hd}] + K")
    q = _randn16(dev, T * Hq * hd, 9).view(T, Hq, hd)
    k = _randn16(dev, T * Hkv * hd, 10).view(T, Hkv, hd)
    rng = np.random.default_rng(11)
    pos_h = rng.integers(0, 32000, T).astype(np.int64)
    pos = torch.from_numpy(pos_h).to(dev)
    toks = [0, BIG // (Hq * hd), T - 2]
    q_before = {t: to_host(q[t:t + 2]) for t in toks}
    k_before = {t: to_host(k[t:t + 2]) for t in toks}
    inv = orc.rope_inv_freq(hd, 1e6)
    mk.rope_neox_qk(q, k, pos, inv)
    for t in toks:
        c, s = orc.rope_tables(inv, pos_h[t:t + 2])
        for x, before, name in ((q, q_before, "q"), (k, k_before, "k")):
            want = orc.rope_neox(before[t], c, s).astype(np.float16)
            assert_bits_equal(to_host(x[t:t + 2]), want, what=f"{name} tokens {t}..")
    del q, k


def test_large_kv_cache(mk, orc, dev):
    """K and V into caches of 2.29e9 elements each (layer 1, blocks near the
    end), with the separate scatter and with RoPE + scatter in one launch."""
    import torch
    L, NB, H, bs, hd = 2, 70000, 8, 16, 128
    _case(f"kv caches [{L},{NB},{H},{bs},{hd}]")
    kc = torch.zeros((L, NB, H, bs, hd), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    S = 64
    rng = np.random.default_rng(12)
    blocks = np.array([NB - 1, NB - 7, NB // 2, 3], dtype=np.int32)  # 4 blocks of 16
    bt = torch.from_numpy(blocks.reshape(1, 4)).to(dev)
    sl = torch.tensor([S], dtype=torch.int32, device=dev)
    sp = torch.tensor([0], dtype=torch.int32, device=dev)
    src_h = rng.standard_normal((1, S, H, hd)).astype(np.float16)
    v_h = rng.standard_normal((1, S, H, hd)).astype(np.float16)
    src, vsrc = torch.from_numpy(src_h).to(dev), torch.from_numpy(v_h).to(dev)
    mk.paged_kv_scatter(src, kc, bt, sl, sp, 1, bs, v_src=vsrc, v_cache=vc)
    for j, b in enumerate(blocks):
        want_k = np.transpose(src_h[0, j * bs:(j + 1) * bs], (1, 0, 2))  # [H, bs, hd]
        want_v = np.transpose(v_h[0, j * bs:(j + 1) * bs], (1, 0, 2))
        assert_bits_equal(to_host(kc[1, int(b)]), want_k, what=f"k block {b}")
        assert_bits_equal(to_host(vc[1, int(b)]), want_v, what=f"v block {b}")
    assert int(torch.count_nonzero(kc[0])) == 0  # layer 0 untouched
    # the same tokens through the one-launch RoPE + scatter (24 Q heads: 256
    # (head, slice) units per token)
    q = torch.from_numpy(rng.standard_normal((S, 24, hd)).astype(np.float16)).to(dev)
    k = src.view(S, H, hd).clone()
    pos_h = np.arange(S, dtype=np.int64) + 100
    inv = orc.rope_inv_freq(hd, 1e6)
    kc.zero_()
    vc.zero_()
    seg = [dict(token_offset=0, S=S, block_table=bt, seq_len=sl, start_pos=sp)]
    mk.rope_kv_scatter(q, k, vsrc.view(S, H, hd), torch.from_numpy(pos_h).to(dev), inv, kc, vc,
                       1, bs, seg)
    c, s = orc.rope_tables(inv, pos_h)
    k_rot = orc.rope_neox(src_h.reshape(S, H, hd), c, s).astype(np.float16)
    for j, b in enumerate(blocks):
        assert_bits_equal(to_host(kc[1, int(b)]),
                          np.transpose(k_rot[j * bs:(j + 1) * bs], (1, 0, 2)),
                          what=f"rotated k block {b}")
        assert_bits_equal(to_host(vc[1, int(b)]),
                          np.transpose(v_h[0, j * bs:(j + 1) * bs], (1, 0, 2)),
                          what=f"v block {b} (one launch)")
    del kc, vc
