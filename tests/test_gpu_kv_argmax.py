"""GPU parity: paged KV-cache scatter and greedy argmax sampling (bit-exact:
both are selections, with no arithmetic to round)."""
import numpy as np
import pytest

from helpers import assert_bits_equal, normal_f16, to_dev, to_host

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _paged_setup(rng, B, S, H, D, bs, L, NB, starts, seqs):
    mb = max(1, -(-int(max(seqs)) // bs))
    src = normal_f16(rng, (B, S, H, D))
    cache = normal_f16(rng, (L, NB, H, bs, D))
    bt = rng.permutation(NB)[:B * mb].reshape(B, mb).astype(np.int32)
    return src, cache, bt, np.asarray(seqs, np.int32), np.asarray(starts, np.int32)


@pytest.mark.parametrize("B,S,starts,seqs", [
    (1, 3000, [0], [3000]),                      # a prefill
    (64, 1, list(range(100, 6500, 100)), [p + 1 for p in range(100, 6500, 100)]),  # decode batch
    (3, 17, [0, 5, 40], [17, 20, 57]),           # ragged: b=1 stops at s = 15
])
def test_kv_scatter_vs_oracle(mk, orc, dev, B, S, starts, seqs):
    _case(f"kv scatter B={B} S={S}")
    rng = np.random.default_rng(B * 1000 + S)
    H, D, bs, L = 4, 128, 16, 2
    NB = B * (max(seqs) // bs + 2) + 3
    src, cache, bt, sl, sp = _paged_setup(rng, B, S, H, D, bs, L, NB, starts, seqs)
    cd = to_dev(cache, dev)
    mk.paged_kv_scatter(to_dev(src, dev), cd, to_dev(bt, dev), to_dev(sl, dev), to_dev(sp, dev),
                        layer=1, block_size=bs)
    ref = orc.paged_kv_scatter(src, cache, bt, sl, sp, layer=1, block_size=bs)
    assert_bits_equal(to_host(cd), ref, what="cache")


def test_kv_scatter_pair_and_bad_blocks(mk, orc, dev):
    """K and V in one launch; a -1 / out-of-range block entry is skipped."""
    _case("kv scatter K+V, bad blocks")
    rng = np.random.default_rng(7)
    B, S, H, D, bs, L = 4, 40, 4, 128, 16, 3
    NB = 30
    starts, seqs = [0, 10, 0, 7], [40, 50, 33, 47]
    k, kc, bt, sl, sp = _paged_setup(rng, B, S, H, D, bs, L, NB, starts, seqs)
    v = normal_f16(rng, k.shape)
    vc = normal_f16(rng, kc.shape)
    bt[1, 1] = -1
    bt[3, 2] = NB + 5
    kcd, vcd = to_dev(kc, dev), to_dev(vc, dev)
    args = (to_dev(bt, dev), to_dev(sl, dev), to_dev(sp, dev))
    mk.paged_kv_scatter(to_dev(k, dev), kcd, *args, layer=2, block_size=bs, v_src=to_dev(v, dev),
                        v_cache=vcd)
    assert_bits_equal(to_host(kcd), orc.paged_kv_scatter(k, kc, bt, sl, sp, 2, bs), what="k")
    assert_bits_equal(to_host(vcd), orc.paged_kv_scatter(v, vc, bt, sl, sp, 2, bs), what="v")


@pytest.mark.parametrize("D", [128, 6])
def test_kv_scatter_with_bias(mk, orc, dev, D):
    """Qwen2's V bias (and a K bias) added on the way into the cache:
    bit-exact against launch_add_bias then the scatter
    (attention.cpp:735-739, :823-846); the sources are not written.  D = 6
    takes the scalar path."""
    _case(f"kv scatter K+V with bias, D={D}")
    rng = np.random.default_rng(90 + D)
    B, S, H, bs, L = 3, 37, 4, 16, 2
    NB = 20
    starts, seqs = [0, 9, 30], [37, 46, 60]
    k, kc, bt, sl, sp = _paged_setup(rng, B, S, H, D, bs, L, NB, starts, seqs)
    v = normal_f16(rng, k.shape)
    vc = normal_f16(rng, kc.shape)
    kb = normal_f16(rng, (H * D,), 0, 0.5)
    vb = normal_f16(rng, (H * D,), 0, 0.5)
    args = (to_dev(bt, dev), to_dev(sl, dev), to_dev(sp, dev))
    for use_k in (False, True):
        kcd, vcd = to_dev(kc, dev), to_dev(vc, dev)
        kd, vd = to_dev(k, dev), to_dev(v, dev)
        mk.paged_kv_scatter(kd, kcd, *args, layer=1, block_size=bs, v_src=vd, v_cache=vcd,
                            k_bias=to_dev(kb, dev) if use_k else None, v_bias=to_dev(vb, dev))
        n = B * S
        vbias = orc.add_bias(v.reshape(-1), vb, n, H * D, n * H * D).reshape(v.shape)
        kbias = orc.add_bias(k.reshape(-1), kb, n, H * D, n * H * D).reshape(k.shape) if use_k else k
        assert_bits_equal(to_host(kcd), orc.paged_kv_scatter(kbias, kc, bt, sl, sp, 1, bs),
                          what=f"k (k bias {use_k})")
        assert_bits_equal(to_host(vcd), orc.paged_kv_scatter(vbias, vc, bt, sl, sp, 1, bs),
                          what=f"v (k bias {use_k})")
        assert_bits_equal(to_host(vd), v, what="v source untouched")
        assert_bits_equal(to_host(kd), k, what="k source untouched")


def test_kv_scatter_odd_head_dim(mk, orc, dev):
    _case("kv scatter D=6 (scalar path)")
    rng = np.random.default_rng(8)
    src, cache, bt, sl, sp = _paged_setup(rng, 2, 5, 3, 6, 4, 1, 10, [0, 3], [5, 8])
    cd = to_dev(cache, dev)
    mk.paged_kv_scatter(to_dev(src, dev), cd, to_dev(bt, dev), to_dev(sl, dev), to_dev(sp, dev),
                        layer=0, block_size=4)
    assert_bits_equal(to_host(cd), orc.paged_kv_scatter(src, cache, bt, sl, sp, 0, 4), what="cache")


@pytest.mark.parametrize("B,V,levels", [(64, 152064, None), (64, 152064, 7), (1, 152064, None),
                                        (600, 4096, 5), (3, 1000, 3), (5, 100003, 9),
                                        (2, 17, None), (512, 152064, None),
                                        (512, 152064, 3), (700, 65536, 5), (513, 16392, None)])
def test_greedy_argmax_vs_oracle(mk, orc, dev, B, V, levels):
    """levels: values drawn from a few integers, so maxima tie often and the
    reference's tie order decides."""
    _case(f"argmax [{B},{V}] levels={levels}")
    rng = np.random.default_rng(B + V)
    if levels is None:
        x = normal_f16(rng, (B, V), 0, 4)
    else:
        x = rng.integers(-levels, levels + 1, (B, V)).astype(np.float16)
    got = to_host(mk.greedy_argmax(to_dev(x, dev)))
    ref = orc.greedy_argmax(x)
    assert (got == ref).all(), f"{int((got != ref).sum())} rows differ"


def test_greedy_argmax_specials(mk, orc, dev):
    _case("argmax NaN / -inf / -0")
    x = np.zeros((4, 9000), dtype=np.float16)
    x[0, :] = -np.inf                   # nothing eligible -> -1
    x[1, ::2] = np.nan
    x[1, 5] = 3.0                       # NaN never chosen
    x[2, :] = -0.0
    x[2, 4000] = 0.0                    # -0 ties +0
    x[3, 17] = np.inf
    got = to_host(mk.greedy_argmax(to_dev(x, dev)))
    assert (got == orc.greedy_argmax(x)).all()
    assert got[0] == -1 and got[1] == 5 and got[3] == 17


def test_greedy_argmax_onepass_specials(mk, orc, dev):
    """The one-launch shape [64, 152064] with values that steer the wave-level
    search: signalling and quiet NaNs (a lane of only NaNs, an sNaN beside the
    row's maximum), rows of -inf, -0/+0 maxima in many lanes, the maximum tied
    in several lanes of one wave and across waves, and +inf."""
    _case("argmax one-launch specials [64,152064]")
    rng = np.random.default_rng(31)
    V = 152064
    x = normal_f16(rng, (64, V), 0, 1)
    bits = x.view(np.uint16)
    bits[0, :] = 0xfc00                          # all -inf -> -1
    bits[1, ::3] = 0x7d00                        # signalling NaNs everywhere
    bits[2, 8000:8032] = 0x7e00                  # one lane's 32 elements all quiet NaN
    bits[3, 100] = 0x7d01; x[3, 101] = 20.0      # sNaN next to the maximum
    x[4, :] = -1.0; bits[4, ::5] = 0x8000; bits[4, 7::11] = 0x0000   # -0 / +0 maxima
    x[5, :] = 0.0; bits[5, :] = 0x8000           # only -0
    x[6, :] = -3.0; x[6, [5, 6, 13, 77, 200, 2048 + 9, 8000, 150000]] = 7.0  # ties in a wave
    x[7, :] = -3.0; x[7, 1::257] = 7.0           # ties over every wave and chunk
    x[8, 123456] = np.inf
    x[9, :] = np.inf                             # every element ties
    bits[10, :] = 0x7e00; x[10, 99999] = -65504.0  # one finite value among NaNs
    x[11] = rng.integers(-1, 2, V).astype(np.float16)   # heavy ties
    bits[12, :] = 0x7e00                         # only NaN -> -1
    bits[13, :] = rng.integers(0x8001, 0x8400, V)  # negative subnormals ...
    bits[13, 4000:4100] = rng.integers(1, 0x400, 100)  # ... and positive ones, max subnormal
    bits[14, :] = rng.integers(1, 0x400, V); x[14, 777] = 6e-5   # smallest normal beside subnormals
    got = to_host(mk.greedy_argmax(to_dev(x, dev)))
    ref = orc.greedy_argmax(x)
    assert (got == ref).all(), f"rows {np.nonzero(got != ref)[0].tolist()} differ"
    assert got[0] == -1 and got[12] == -1 and got[3] == 101 and got[8] == 123456
    assert got[10] == 99999


def test_greedy_argmax_workspace_graph(mk, orc, dev):
    _case("argmax with workspace in a graph")
    import torch
    rng = np.random.default_rng(9)
    x = normal_f16(rng, (64, 152064), 0, 4)
    xd = to_dev(x, dev)
    ws = torch.zeros(max(1, mk.greedy_argmax_workspace_bytes(64, 152064)), dtype=torch.uint8,
                     device=dev)
    out = torch.empty(64, dtype=torch.int32, device=dev)
    mk.greedy_argmax(xd, out=out, workspace=ws)
    ref = orc.greedy_argmax(x)
    assert (to_host(out) == ref).all()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        mk.greedy_argmax(xd, out=out, workspace=ws)
    for _ in range(3):
        out.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        assert (to_host(out) == ref).all()


def test_greedy_argmax_max_at_every_vector_position(mk, orc, dev):
    """Regression: one unique maximum per row at offsets 0..15 inside a
    16-element pair of vectors, at the start, middle and end of long rows."""
    _case("argmax max at every vector lane")
    V = 152064
    rows = []
    for base in (0, 74000 - 74000 % 16, V - 16):
        for k in range(16):
            r = np.zeros(V, dtype=np.float16)
            r[base + k] = 1.0
            rows.append(r)
    x = np.stack(rows)
    got = to_host(mk.greedy_argmax(to_dev(x, dev)))
    want = np.array([int(np.argmax(r)) for r in rows], dtype=np.int32)
    assert (got == want).all() and (orc.greedy_argmax(x) == want).all()


def test_greedy_argmax_workspace_reuse(mk, orc, dev):
    """One zeroed workspace serves calls of different shapes in turn, one-
    launch (V % 16 == 0) and two-launch (V % 16 != 0) alike: no record left by
    an earlier call passes for fresh."""
    _case("argmax workspace reuse across shapes")
    import torch
    ws = torch.zeros(max(1, mk.greedy_argmax_workspace_bytes(511, 600000)), dtype=torch.uint8,
                     device=dev)
    rng = np.random.default_rng(12)
    for B, V, levels in ((64, 152064, None), (3, 152064, 2), (64, 100000, None), (1, 32768, 1),
                         (64, 152064, 3), (5, 100003, None), (300, 600000, None),
                         (3, 152064, 2)):
        assert mk.greedy_argmax_workspace_bytes(B, V) <= ws.numel()
        x = (normal_f16(rng, (B, V), 0, 4) if levels is None
             else rng.integers(-levels, levels + 1, (B, V)).astype(np.float16))
        got = to_host(mk.greedy_argmax(to_dev(x, dev), workspace=ws))
        assert (got == orc.greedy_argmax(x)).all(), f"[{B},{V}]"


def test_greedy_argmax_onepass_forced_fallback(mk, orc, dev):
    """Chunk 0's bounded poll, forced to run out from the host (bound 0): it
    scans its whole row itself; results match, and later one-launch calls on
    the same workspace are still right."""
    _case("argmax one-launch forced fallback")
    import torch
    rng = np.random.default_rng(13)
    ws = torch.zeros(mk.greedy_argmax_workspace_bytes(64, 152064), dtype=torch.uint8, device=dev)
    x = rng.integers(-3, 4, (64, 152064)).astype(np.float16)
    prev = mk.greedy_argmax_test_poll_limit(0)
    try:
        got = to_host(mk.greedy_argmax(to_dev(x, dev), workspace=ws))
    finally:
        mk.greedy_argmax_test_poll_limit(prev)
    assert (got == orc.greedy_argmax(x)).all()
    for i in range(3):
        x2 = normal_f16(rng, (64, 152064), 0, 4)
        got = to_host(mk.greedy_argmax(to_dev(x2, dev), workspace=ws))
        assert (got == orc.greedy_argmax(x2)).all(), f"call {i} after the fallback"


def test_greedy_argmax_onepass_epoch_past_32_bits(mk, orc, dev):
    """Row epochs are 64-bit: started just below 2^32, successive calls on new
    logits return the new rows' maxima and the epoch grows past 2^32."""
    _case("argmax one-pass epoch past 2^32")
    import torch
    rng = np.random.default_rng(59)
    B, V, rec = 8, 40000, 2176 // 8  # 2176-byte row records
    ws = torch.zeros(mk.greedy_argmax_workspace_bytes(B, V), dtype=torch.uint8, device=dev)
    e64 = ws[: 512 * 2176].view(torch.int64)
    start = (1 << 32) - 3
    e64[0:B * rec:rec] = start
    for i in range(5):
        x = normal_f16(rng, (B, V), 0, 4)
        got = to_host(mk.greedy_argmax(to_dev(x, dev), workspace=ws))
        assert (got == orc.greedy_argmax(x)).all(), f"call {i}"
    epochs = e64[0:B * rec:rec].cpu().numpy()
    assert (epochs == start + 5).all(), epochs


def test_greedy_argmax_allocating_entry_paths(mk, orc, dev):
    """mi_greedy_argmax_f16 at split shapes: one launch on stream 0 with the
    library's row records (fresh logits each call, a forced fallback in the
    middle), two launches on another stream."""
    _case("argmax allocating entry: stream 0 one launch, side stream two launches")
    import torch
    rng = np.random.default_rng(62)
    assert torch.cuda.current_stream().cuda_stream == 0
    for i, (B, V) in enumerate([(64, 152064), (8, 40000), (64, 152064), (3, 65536)]):
        x = normal_f16(rng, (B, V), 0, 4)
        prev = mk.greedy_argmax_test_poll_limit(0) if i == 2 else None
        try:
            got = to_host(mk.greedy_argmax(to_dev(x, dev)))
        finally:
            if prev is not None:
                mk.greedy_argmax_test_poll_limit(prev)
        assert (got == orc.greedy_argmax(x)).all(), f"stream 0, call {i} [{B},{V}]"
    side = torch.cuda.Stream()
    for B, V in [(64, 152064), (8, 40000)]:
        x = normal_f16(rng, (B, V), 0, 4)
        xd = to_dev(x, dev)
        side.wait_stream(torch.cuda.current_stream())
        got = mk.greedy_argmax(xd, stream=side)
        torch.cuda.current_stream().wait_stream(side)
        assert (to_host(got) == orc.greedy_argmax(x)).all(), f"side stream [{B},{V}]"
