"""GPU parity: row softmax (row-per-workgroup and split-row paths) and the
token-embedding gather.

Softmax outputs are held within rtol = atol = 1e-3 of the fp32 oracle
(tests/verify/verify.py:142); the gather is a copy and must be bit-exact.
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close, normal_f16, to_dev, to_host

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).resolve().parent / "golden" / "ref_cases.npz")


def _case(msg):
    print(f"[case] {msg}", flush=True)


def test_softmax_reference_case(mk, orc, dev):
    """tests/test_softmax/main.cpp:63-66: [8, 1024], seed 555 x4."""
    _case("softmax reference [8,1024]")
    x = GOLD["softmax_x"]
    y = to_host(mk.softmax(to_dev(x, dev)))
    assert_close(y, GOLD["softmax_y"], what="vs golden")
    assert_close(y, orc.softmax(x), what="vs oracle")


def test_softmax_lm_head_config(mk, orc, dev):
    """The decoder chain's sampling softmax: logits [64, 152064] ~N(0,4) (split-row path)."""
    _case("softmax [64,152064]")
    rng = np.random.default_rng(51)
    x = normal_f16(rng, (64, 152064), 0, 4)
    y = to_host(mk.softmax(to_dev(x, dev)))
    ref = orc.softmax(x, nthreads=8)
    assert_close(y, ref, what="cfg5")
    np.testing.assert_allclose(y.astype(np.float64).sum(-1), 1.0, rtol=2e-3)


@pytest.mark.parametrize("N,D", [(1, 1), (3, 7), (57344, 512), (600, 10000), (2, 8192),
                                 (5, 100003), (511, 9000), (1, 300000), (130, 24), (2, 600000),
                                 (3, 8200), (64, 16384)])
def test_softmax_shapes(mk, orc, dev, N, D):
    _case(f"softmax [{N},{D}]")
    rng = np.random.default_rng(N * 31 + D)
    x = normal_f16(rng, (N, D), 0, 4)
    y = to_host(mk.softmax(to_dev(x, dev)))
    assert_close(y, orc.softmax(x, nthreads=8), what=f"[{N},{D}]")


def test_softmax_in_place_and_neg_inf(mk, orc, dev):
    _case("softmax in place, -inf entries")
    rng = np.random.default_rng(52)
    for N, D in ((64, 152064), (16, 2048)):
        x = normal_f16(rng, (N, D), 0, 4)
        x[:, ::3] = -np.inf  # masked logits
        xd = to_dev(x, dev)
        mk.softmax(xd, y=xd)
        assert_close(to_host(xd), orc.softmax(x, nthreads=8), what=f"in place [{N},{D}]")


def test_gather_chain_config(mk, orc, dev):
    """The decoder chain's gather: table [152064, 3584] ~N(0, 0.02), 6064 uniform ids."""
    _case("gather [6064] from [152064,3584]")
    import torch
    g = torch.Generator(device=dev).manual_seed(53)
    table = (torch.randn(152064, 3584, generator=g, device=dev) * 0.02).half()
    rng = np.random.default_rng(53)
    ids = rng.integers(0, 152064, 6064).astype(np.int64)
    out = to_host(mk.embedding_gather(to_dev(ids, dev), table))
    table_h = to_host(table)
    assert_bits_equal(out, orc.embedding_gather(ids, table_h, nthreads=8), what="gather")


@pytest.mark.parametrize("H", [3584, 3585, 8, 1, 1000])
def test_gather_shapes_and_bad_ids(mk, orc, dev, H):
    _case(f"gather H={H}")
    rng = np.random.default_rng(H)
    V = 300
    table = normal_f16(rng, (V, H), 0, 0.02)
    ids = rng.integers(0, V, (3, 37)).astype(np.int64)
    ids[0, 0] = -1
    ids[1, 5] = V
    ids[2, 7] = V - 1
    out = to_host(mk.embedding_gather(to_dev(ids, dev), to_dev(table, dev)))
    assert_bits_equal(out, orc.embedding_gather(ids, table), what=f"H={H}")
    assert (out[0, 0] == 0).all() and (out[1, 5] == 0).all()


@pytest.mark.parametrize("T", [613, 2051])
@pytest.mark.parametrize("D,scale,add_one", [(3584, 1.0, False), (3584, 3584 ** 0.5, True),
                                             (8192, 1.0, False), (2048, 2048 ** 0.5, False),
                                             (1000, 1.0, False), (3585, 59.87, True)])
def test_embedding_rmsnorm(mk, orc, dev, D, scale, add_one, T):
    """Gather fused with the input RMSNorm: hidden is the gathered row (scaled
    and rounded as mi_scale_inplace_f16 does), bit for bit, and y the oracle's
    RMSNorm of that fp16 hidden, rtol = atol = 1e-3.  Vector and scalar
    paths, out-of-range ids (zero rows), Gemma's scale and (1 + w); T = 613
    runs a workgroup per row, T = 2051 a wave per row (four rows per
    workgroup, the last one partial); y equals the unfused GPU sequence bit
    for bit either way."""
    _case(f"embedding+rmsnorm T={T} D={D} scale={scale:.3f} add_one={add_one}")
    rng = np.random.default_rng(D + T)
    V = 700
    table = normal_f16(rng, (V, D), 0, 0.02)
    w = normal_f16(rng, (D,), 0.0 if add_one else 1.0, 0.1)
    ids = rng.integers(0, V, T).astype(np.int64)
    ids[3] = -5
    ids[10] = V
    hid, y = mk.embedding_rmsnorm(to_dev(ids, dev), to_dev(table, dev), to_dev(w, dev),
                                  scale=scale, eps=1e-6, add_one=add_one)
    ref_h = orc.embedding_gather(ids, table)
    if scale != 1.0:
        ref_h = orc.scale(ref_h, np.float32(scale))
    assert_bits_equal(to_host(hid), ref_h, what="hidden")
    assert_close(to_host(y), orc.rmsnorm(ref_h, w, 1e-6, add_one), what="y")
    # the unfused sequence on the GPU gives the same bits
    g = mk.embedding_gather(to_dev(ids, dev), to_dev(table, dev))
    if scale != 1.0:
        mk.scale_inplace(g, scale)
    y2 = mk.rmsnorm(g, to_dev(w, dev), eps=1e-6, add_one=add_one)
    assert_bits_equal(to_host(y), to_host(y2), what="fused vs gather + scale + rmsnorm")


def test_softmax_workspace_variant(mk, orc, dev):
    _case("softmax with caller workspace")
    import torch
    rng = np.random.default_rng(54)
    x = normal_f16(rng, (64, 152064), 0, 4)
    xd = to_dev(x, dev)
    nb = mk.softmax_workspace_bytes(64, 152064)
    assert nb > 0
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    y1 = to_host(mk.softmax(xd, workspace=ws))  # one launch (out of place)
    y2 = to_host(mk.softmax(xd))                # two launches (pool workspace)
    ref = orc.softmax(x, nthreads=8)
    assert_close(y1, ref, what="one-pass vs oracle")
    assert_close(y2, ref, what="two-pass vs oracle")
    for _ in range(3):
        assert_bits_equal(to_host(mk.softmax(xd, workspace=ws)), y1, what="repeat")
    with pytest.raises(RuntimeError, match="status -1"):
        mk.softmax(xd, workspace=ws[: nb - 8])


def test_softmax_onepass_workspace_across_shapes(mk, orc, dev):
    """One zeroed workspace through calls of different shapes, an in-place
    call (two-launch form) in between, and calls repeated: every result
    matches the oracle, so no record left by an earlier call passes for
    fresh."""
    _case("softmax one-pass workspace across shapes")
    import torch
    rng = np.random.default_rng(56)
    ws = torch.zeros(mk.softmax_workspace_bytes(511, 524288), dtype=torch.uint8, device=dev)
    for N, D, inplace in ((64, 152064, False), (3, 100000, False), (64, 152064, False),
                          (17, 8192, True), (64, 152064, False), (200, 524288, False),
                          (5, 600000, False), (3, 100000, False)):
        x = normal_f16(rng, (N, D), 0, 4)
        xd = to_dev(x, dev)
        y = mk.softmax(xd, y=xd if inplace else None, workspace=ws)
        assert_close(to_host(y), orc.softmax(x, nthreads=8), what=f"[{N},{D}] inplace={inplace}")


def test_softmax_onepass_forced_fallback(mk, orc, dev):
    """The bounded-poll fallback, forced from the host (poll bound 0): every
    chunk computes its row's statistics from x; the results still match, and
    normal one-pass calls afterwards are still right (the fallback's epoch
    step keeps its tags from passing for fresh)."""
    _case("softmax one-pass forced fallback")
    import torch
    rng = np.random.default_rng(57)
    ws = torch.zeros(mk.softmax_workspace_bytes(64, 152064), dtype=torch.uint8, device=dev)
    x = normal_f16(rng, (64, 152064), 0, 4)
    xd = to_dev(x, dev)
    ref = orc.softmax(x, nthreads=8)
    prev = mk.softmax_test_poll_limit(0)
    try:
        assert_close(to_host(mk.softmax(xd, workspace=ws)), ref, what="forced fallback")
    finally:
        mk.softmax_test_poll_limit(prev)
    x2 = normal_f16(rng, (64, 152064), 0, 4)
    ref2 = orc.softmax(x2, nthreads=8)
    for i in range(3):
        assert_close(to_host(mk.softmax(to_dev(x2, dev), workspace=ws)), ref2,
                     what=f"after fallback, call {i}")


def test_softmax_multiround_fallback_is_bounded(mk, orc, dev):
    """Persistent one-launch rows over several rounds per row slot, with a
    poll bound small enough that some chunks give up: a chunk that has fallen
    back computes every later round's statistics from x without polling
    again, so the call stays correct and its time stays bounded (with the
    bound 1, a chunk that kept polling each round would still finish; the
    wall-time check guards the path that stops polling)."""
    _case("softmax multi-round fallback [4096,65600] poll bound 1")
    import time
    import torch
    rng = np.random.default_rng(58)
    N, D = 4096, 65600
    ws = torch.zeros(mk.softmax_workspace_bytes(N, D), dtype=torch.uint8, device=dev)
    x = normal_f16(rng, (N, D), 0, 4)
    xd = to_dev(x, dev)
    ref = orc.softmax(x, nthreads=8)
    for limit in (1, 0):
        prev = mk.softmax_test_poll_limit(limit)
        try:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            y = mk.softmax(xd, workspace=ws)
            torch.cuda.synchronize()
            el = time.perf_counter() - t0
        finally:
            mk.softmax_test_poll_limit(prev)
        print(f"[case]   poll bound {limit}: {el * 1e3:.2f} ms", flush=True)
        assert el < 0.5, f"poll bound {limit}: {el:.3f} s"
        assert_close(to_host(y), ref, what=f"poll bound {limit}")
    assert_close(to_host(mk.softmax(xd, workspace=ws)), ref, what="after the fallbacks")


def test_softmax_graph_replay(mk, orc, dev):
    """The split-row kernels inside a captured graph, replayed several times
    with eager work in between; every replay matches the eager call."""
    _case("softmax graph replay [64,152064]")
    import torch
    rng = np.random.default_rng(55)
    x = normal_f16(rng, (64, 152064), 0, 4)
    xd = to_dev(x, dev)
    ws = torch.zeros(mk.softmax_workspace_bytes(64, 152064), dtype=torch.uint8, device=dev)
    y = torch.empty_like(xd)
    ref = to_host(mk.softmax(xd, workspace=ws))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mk.softmax(xd, y=y, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mk.softmax(xd, y=y, workspace=ws)
    for i in range(4):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        assert_bits_equal(to_host(y), ref, what=f"replay {i}")
        mk.softmax(xd, workspace=ws)  # eager call between replays
    assert_close(ref, orc.softmax(x, nthreads=8), what="vs oracle")


def test_softmax_onepass_epoch_past_32_bits(mk, orc, dev):
    """Row epochs are 64-bit: started just below 2^32 (as after ~4e9 calls on
    a row), successive calls on new logits stay right and the epoch keeps
    growing past 2^32 (a 32-bit epoch would stick at 2^32 - 1 and let the
    next call take the previous call's slots as fresh)."""
    _case("softmax one-pass epoch past 2^32")
    import torch
    rng = np.random.default_rng(58)
    N, D, rec = 8, 40000, 4224 // 8  # 4224-byte row records
    ws = torch.zeros(mk.softmax_workspace_bytes(N, D), dtype=torch.uint8, device=dev)
    e64 = ws[: 512 * 4224].view(torch.int64)
    start = (1 << 32) - 3
    e64[0:N * rec:rec] = start
    for i in range(5):
        x = normal_f16(rng, (N, D), 0, 4)
        assert_close(to_host(mk.softmax(to_dev(x, dev), workspace=ws)), orc.softmax(x),
                     what=f"call {i}")
    epochs = e64[0:N * rec:rec].cpu().numpy()
    assert (epochs == start + 5).all(), epochs


def test_softmax_allocating_entry_paths(mk, orc, dev):
    """mi_softmax_f16 at split shapes: on stream 0 (the reference's callers'
    stream) one launch with row records the library holds -- fresh logits on
    every call, a forced-fallback call in the middle -- and on another stream
    two launches with a stream-ordered workspace."""
    _case("softmax allocating entry: stream 0 one launch, side stream two launches")
    import torch
    rng = np.random.default_rng(61)
    assert torch.cuda.current_stream().cuda_stream == 0
    for i, (N, D) in enumerate([(64, 152064), (8, 40000), (64, 152064), (3, 65536)]):
        x = normal_f16(rng, (N, D), 0, 4)
        prev = mk.softmax_test_poll_limit(0) if i == 2 else None
        try:
            y = to_host(mk.softmax(to_dev(x, dev)))
        finally:
            if prev is not None:
                mk.softmax_test_poll_limit(prev)
        assert_close(y, orc.softmax(x, nthreads=8), what=f"stream 0, call {i} [{N},{D}]")
    side = torch.cuda.Stream()
    for N, D in [(64, 152064), (8, 40000)]:
        x = normal_f16(rng, (N, D), 0, 4)
        xd = to_dev(x, dev)
        side.wait_stream(torch.cuda.current_stream())
        y = mk.softmax(xd, stream=side)
        torch.cuda.current_stream().wait_stream(side)
        assert_close(to_host(y), orc.softmax(x, nthreads=8), what=f"side stream [{N},{D}]")


def test_softmax_persistent_rows(mk, orc, dev):
    """Many long rows in the persistent one-launch form (a resident grid of
    chunk workgroups walking rows in rounds, the next row's loads in flight
    during each exchange): the caller-workspace entry and the allocating
    entry on stream 0, ragged last rounds, rows too many for the one-pass
    grid below 512 rows, -inf entries, and an in-place call (a workgroup
    per row)."""
    _case("softmax persistent rows")
    import torch
    rng = np.random.default_rng(62)
    shapes = ((512, 152064), (200, 152064), (1000, 70000), (700, 65544), (513, 100008),
              (4100, 65600), (300, 40000), (256, 32776), (2048, 40000))
    nb = max(mk.softmax_workspace_bytes(N, D) for N, D in shapes)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    for N, D in shapes:
        print(f"[case] persistent [{N},{D}]", flush=True)
        x = normal_f16(rng, (N, D), 0, 4)
        x[:, rng.integers(0, D, 16)] = -np.inf
        ref = orc.softmax(x, nthreads=8)
        xd = to_dev(x, dev)
        assert_close(to_host(mk.softmax(xd, workspace=ws)), ref, what=f"workspace [{N},{D}]")
        assert_close(to_host(mk.softmax(xd)), ref, what=f"stream 0 [{N},{D}]")
        del xd
    x = normal_f16(rng, (512, 152064), 0, 4)
    ref = orc.softmax(x, nthreads=8)
    xd = to_dev(x, dev)
    assert_close(to_host(mk.softmax(xd, y=xd, workspace=ws)), ref, what="in place")


def test_softmax_persistent_forced_fallback(mk, orc, dev):
    """The persistent form with the poll bound forced to 0 from the host:
    every chunk of every round computes its row's statistics from x.  Calls
    afterwards, persistent and one-pass on the same records, stay right."""
    _case("softmax persistent forced fallback")
    import torch
    rng = np.random.default_rng(63)
    nb = max(mk.softmax_workspace_bytes(N, D) for N, D in ((64, 152064), (300, 152064)))
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    x = normal_f16(rng, (600, 100000), 0, 4)
    ref = orc.softmax(x, nthreads=8)
    xd = to_dev(x, dev)
    prev = mk.softmax_test_poll_limit(0)
    try:
        assert_close(to_host(mk.softmax(xd, workspace=ws)), ref, what="forced fallback")
    finally:
        mk.softmax_test_poll_limit(prev)
    for N, D in ((600, 100000), (64, 152064), (600, 100000), (300, 152064)):
        x2 = normal_f16(rng, (N, D), 0, 4)
        assert_close(to_host(mk.softmax(to_dev(x2, dev), workspace=ws)),
                     orc.softmax(x2, nthreads=8), what=f"after fallback [{N},{D}]")


def test_softmax_persistent_graph_replay(mk, orc, dev):
    """The persistent form inside a captured graph, replayed several times
    with eager calls on the same records in between."""
    _case("softmax persistent graph replay [512,152064]")
    import torch
    rng = np.random.default_rng(64)
    x = normal_f16(rng, (512, 152064), 0, 4)
    xd = to_dev(x, dev)
    ws = torch.zeros(mk.softmax_workspace_bytes(512, 152064), dtype=torch.uint8, device=dev)
    y = torch.empty_like(xd)
    ref = to_host(mk.softmax(xd, workspace=ws))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mk.softmax(xd, y=y, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mk.softmax(xd, y=y, workspace=ws)
    for i in range(4):
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        assert_bits_equal(to_host(y), ref, what=f"replay {i}")
        mk.softmax(xd, workspace=ws)
    assert_close(ref, orc.softmax(x, nthreads=8), what="vs oracle")


def _special_logits(rng, N, V):
    x = normal_f16(rng, (N, V), 0, 4)
    x[0, :] = -np.inf                       # nothing eligible: argmax -1
    x[1, 5], x[1, V - 3] = 30.0, 30.0       # a tie across chunks
    if N > 2:
        x[2, ::7] = np.nan                  # NaN never chosen
        x[2, V // 2] = 40.0
    if N > 3:
        x[3, :] = -0.0                      # all equal (signed zeros): the tie order decides
        x[3, 1::2] = 0.0
    return x


@pytest.mark.parametrize("N,V,inplace", [(64, 152064, False), (600, 65544, False),
                                         (5, 40000, False), (64, 152064, True), (7, 1000, False),
                                         (300, 32768, False)])
def test_softmax_argmax_fused(mk, orc, dev, N, V, inplace):
    """Softmax and greedy argmax of the same logits in one pass: probs bit for
    bit those of mi_softmax_ws_f16 (the same kernels' arithmetic), indices
    exactly the oracle's (the reference's tie order), over one-launch split
    rows, the persistent many-row form, and shapes that run the two entry
    points in turn (in place, short rows)."""
    _case(f"softmax+argmax [{N},{V}] inplace={inplace}")
    import torch
    rng = np.random.default_rng(N + V)
    x = _special_logits(rng, N, V)
    xd = to_dev(x, dev)
    ws = torch.zeros(mk.softmax_argmax_workspace_bytes(N, V), dtype=torch.uint8, device=dev)
    ref_idx = orc.greedy_argmax(x)
    sws = torch.zeros(max(16, mk.softmax_workspace_bytes(N, V)), dtype=torch.uint8, device=dev)
    xr = xd.clone()
    ref_p = to_host(mk.softmax(xr, y=xr if inplace else None, workspace=sws))
    for call in range(2):  # the workspace stays valid for the next call
        xin = xd.clone() if inplace else xd
        probs, idx = mk.softmax_argmax(xin, ws, probs=xin if inplace else None)
        assert (to_host(idx) == ref_idx).all(), f"call {call}: argmax"
        assert_bits_equal(to_host(probs), ref_p, what=f"call {call}: probs")
    if not inplace:
        assert_bits_equal(to_host(xd), x, what="logits untouched")


def test_softmax_argmax_forced_fallback(mk, orc, dev):
    """Poll bound 0: every chunk takes the fallback (statistics and the row's
    key from x); results unchanged, and normal calls afterwards still right."""
    _case("softmax+argmax forced fallback")
    import torch
    rng = np.random.default_rng(77)
    N, V = 64, 152064
    x = _special_logits(rng, N, V)
    xd = to_dev(x, dev)
    ws = torch.zeros(mk.softmax_argmax_workspace_bytes(N, V), dtype=torch.uint8, device=dev)
    ref_p = orc.softmax(x, nthreads=8)
    prev = mk.softmax_test_poll_limit(0)
    try:
        probs, idx = mk.softmax_argmax(xd, ws)
        torch.cuda.synchronize()
    finally:
        mk.softmax_test_poll_limit(prev)
    assert (to_host(idx) == orc.greedy_argmax(x)).all()
    ok = np.isfinite(ref_p)
    assert_close(to_host(probs)[ok], ref_p[ok], what="fallback probs")
    x2 = normal_f16(rng, (N, V), 0, 4)
    probs, idx = mk.softmax_argmax(to_dev(x2, dev), ws)
    assert (to_host(idx) == orc.greedy_argmax(x2)).all()
    assert_close(to_host(probs), orc.softmax(x2, nthreads=8), what="after fallback")


def test_softmax_argmax_graph_replay(mk, orc, dev):
    """The fused pass captured in a graph and replayed with eager work in
    between: every replay matches the eager call."""
    _case("softmax+argmax graph replay")
    import torch
    rng = np.random.default_rng(78)
    N, V = 64, 152064
    x = normal_f16(rng, (N, V), 0, 4)
    xd = to_dev(x, dev)
    ws = torch.zeros(mk.softmax_argmax_workspace_bytes(N, V), dtype=torch.uint8, device=dev)
    p_ref, i_ref = (to_host(t) for t in mk.softmax_argmax(xd, ws))
    probs = torch.empty_like(xd)
    idx = torch.empty(N, dtype=torch.int32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mk.softmax_argmax(xd, ws, probs=probs, out=idx)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        mk.softmax_argmax(xd, ws, probs=probs, out=idx, stream=side)
    for i in range(3):
        probs.zero_()
        idx.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_bits_equal(to_host(probs), p_ref, what=f"replay {i}")
        assert (to_host(idx) == i_ref).all(), f"replay {i}"
    del g
