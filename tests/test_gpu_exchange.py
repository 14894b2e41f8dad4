"""GPU: the one-launch kernels' row exchange (csrc/row_exchange.h).

Softmax, greedy argmax and the fused softmax + argmax over split rows publish
each chunk's partial result into the row's slots in the XCD's L2 and into a
device-scope mirror; polls read the L2 copy first.  These tests check that:
  * the mirror-only mode (mi_exchange_test_mode(1)), the path taken when the
    L2 copy does not show every chunk, gives bit-identical results to the
    default mode, on row counts that are and are not multiples of the XCD
    count, one and several rounds per row slot, with a workspace shared
    between the modes;
  * results match the oracle in both modes;
  * the default mode is served by the L2 copy: a call takes far less than
    the L2 phase's 20 us bound (a launch that fell through to the mirror
    would take at least that long);
  * calls on two streams at once, beside a kernel holding CUs, stay correct
    and bounded in time.
"""
import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close, normal_f16, to_dev, to_host

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _run_all(mk, xd, ws_sm, ws_am, ws_fused, N):
    import torch
    y = mk.softmax(xd, workspace=ws_sm)
    idx = mk.greedy_argmax(xd, workspace=ws_am)
    probs, out = mk.softmax_argmax(xd, ws_fused)
    torch.cuda.synchronize()
    return to_host(y), to_host(idx), to_host(probs), to_host(out)


@pytest.mark.parametrize("N,D", [(64, 152064), (5, 152064), (13, 100000), (1, 40000),
                                 (300, 40000), (600, 131072)])
def test_mirror_mode_matches_default(mk, orc, dev, N, D):
    import torch
    _case(f"exchange modes [{N},{D}]")
    rng = np.random.default_rng(N * 7 + D)
    x = normal_f16(rng, (N, D), 0, 4)
    xd = to_dev(x, dev)
    ws_sm = torch.zeros(max(16, mk.softmax_workspace_bytes(N, D)), dtype=torch.uint8, device=dev)
    ws_am = torch.zeros(max(16, mk.greedy_argmax_workspace_bytes(N, D)), dtype=torch.uint8,
                        device=dev)
    ws_fused = torch.zeros(mk.softmax_argmax_workspace_bytes(N, D), dtype=torch.uint8, device=dev)
    base = _run_all(mk, xd, ws_sm, ws_am, ws_fused, N)
    prev = mk.exchange_test_mode(1)
    try:
        assert prev == 0
        mirror = _run_all(mk, xd, ws_sm, ws_am, ws_fused, N)
    finally:
        mk.exchange_test_mode(prev)
    again = _run_all(mk, xd, ws_sm, ws_am, ws_fused, N)  # back on the L2 copy, same workspace
    for name, a, b, c in zip(("softmax", "argmax", "fused probs", "fused argmax"), base, mirror,
                             again):
        assert_bits_equal(b, a, what=f"{name}: mirror vs default")
        assert_bits_equal(c, a, what=f"{name}: default after mirror")
    ref = orc.softmax(x, nthreads=8)
    assert_close(base[0], ref, what="softmax vs oracle")
    assert_bits_equal(base[2], base[0], what="fused probs vs softmax")
    want = orc.greedy_argmax(x)
    np.testing.assert_array_equal(base[1].astype(np.int64), want)
    np.testing.assert_array_equal(base[3].astype(np.int64), want)


def test_default_mode_is_served_by_l2(mk, dev):
    """Average time per call of the one-launch softmax, argmax and fused pass
    at [64, 152064], back-to-back launches replayed from a graph and timed
    with events.  Printed for the log (normally ~7-11 us, well under the 20 us
    the L2 phase may last before polls move to the mirror); asserted only
    against a bound loose enough that a loaded box or lowered clocks cannot
    trip it: 40 us per call, which a call reaches only when its polls run to
    the 50 us fallback bound."""
    import torch
    _case("exchange: L2 phase serves the default mode")
    N, D = 64, 152064
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    x = (torch.randn((N, D), generator=g, device=dev) * 4).half()
    y = torch.empty_like(x)
    out = torch.empty(N, dtype=torch.int32, device=dev)
    ws_sm = torch.zeros(mk.softmax_workspace_bytes(N, D), dtype=torch.uint8, device=dev)
    ws_am = torch.zeros(mk.greedy_argmax_workspace_bytes(N, D), dtype=torch.uint8, device=dev)
    ws_fused = torch.zeros(mk.softmax_argmax_workspace_bytes(N, D), dtype=torch.uint8, device=dev)
    calls = {
        "softmax": lambda: mk.softmax(x, y=y, workspace=ws_sm),
        "argmax": lambda: mk.greedy_argmax(x, out=out, workspace=ws_am),
        "softmax+argmax": lambda: mk.softmax_argmax(x, ws_fused, probs=y, out=out),
    }
    for name, f in calls.items():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(5):
                f()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        n = 50
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(n):
                f()
        graph.replay()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        graph.replay()
        t1.record()
        torch.cuda.synchronize()
        del graph
        us = t0.elapsed_time(t1) * 1e3 / n
        print(f"[case]   {name}: {us:.1f} us per call", flush=True)
        assert us < 40.0, f"{name}: {us:.1f} us per call (polls ran to their bound?)"


def test_one_launch_kernels_on_concurrent_streams(mk, orc, dev):
    """Softmax, argmax and the fused pass on two streams at once, each call
    with its own workspace, next to a large SwiGLU holding CUs: a row's chunk
    workgroups may then not all be resident together, and polls that run out
    take the bounded fallback.  Every result matches the oracle, and the whole
    exchange finishes well inside a wall-clock bound."""
    import time
    import torch
    _case("one-launch kernels on two concurrent streams")
    rng = np.random.default_rng(31)
    shapes = ((64, 152064), (48, 131072))
    xs = [normal_f16(rng, s, 0, 4) for s in shapes]
    xd = [to_dev(x, dev) for x in xs]
    g = (torch.randn((4096, 18944), device=dev) * 2).half()
    u = torch.randn((4096, 18944), device=dev).half()
    act = torch.empty_like(g)
    ws = [(torch.zeros(mk.softmax_workspace_bytes(*s), dtype=torch.uint8, device=dev),
           torch.zeros(mk.greedy_argmax_workspace_bytes(*s), dtype=torch.uint8, device=dev),
           torch.zeros(mk.softmax_argmax_workspace_bytes(*s), dtype=torch.uint8, device=dev))
          for s in shapes]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    t0 = time.time()
    outs = []
    for rep in range(3):
        res = []
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                if i == 0:
                    mk.swiglu(g, u, out=act)
                y = mk.softmax(xd[i], workspace=ws[i][0])
                a = mk.greedy_argmax(xd[i], workspace=ws[i][1])
                p, o = mk.softmax_argmax(xd[i], ws[i][2])
                res.append((y, a, p, o))
        outs.append(res)
    torch.cuda.synchronize()
    wall = time.time() - t0
    for res in outs:
        for i, (y, a, p, o) in enumerate(res):
            x = xs[i]
            want = orc.greedy_argmax(x)
            np.testing.assert_array_equal(to_host(a).astype(np.int64), want)
            np.testing.assert_array_equal(to_host(o).astype(np.int64), want)
            yh = to_host(y)
            assert_bits_equal(to_host(p), yh, what=f"fused probs vs softmax {shapes[i]}")
            assert_close(yh, orc.softmax(x, nthreads=8), what=f"softmax {shapes[i]}")
    # 18 one-launch calls: even every poll of every call running to its 50 us
    # bound would stay far below this
    assert wall < 10.0, f"{wall:.1f} s"
