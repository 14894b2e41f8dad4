"""GPU parity: top-p sampling (mi_top_p_sample_f16 / _batched_f16) against the
oracle's step-by-step restatement of launch_top_p_sample
(src/kernels/sampling_kernel.cu:86-221).

The result is an index, compared exactly.  The probabilities behind it are
fp32 exp/sum values whose last bits differ between implementations (the
reference's fast exp, the GPU's, libm's), so random cases are screened: no
running sum of the ordered candidate probabilities within 1e-4 of p, and no
two different candidate probabilities within 1e-5 (relative) of each other.
Equal logits give equal probabilities in every implementation, so exact ties
are kept and must resolve to the lower index.  Above 30000 logits the result
is the greedy argmax, compared with the oracle's simulation of the
reference's greedy kernel (Qwen2.5's 152064-entry rows included).
"""
import numpy as np
import pytest

from helpers import normal_f16, to_dev, to_host

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _safe(x, p, T):
    """Whether a row's outcome is far from every rounding boundary."""
    xf = x.astype(np.float64) / T
    e = np.exp(xf - xf.max())
    q = np.exp(xf[::128] - xf.max()) / e.sum()
    qs = np.sort(q)[::-1]
    cum = np.cumsum(qs)
    if np.min(np.abs(cum - p)) < 1e-4:
        return False
    d = np.diff(qs)
    close = (np.abs(d) < 1e-5 * np.maximum(qs[1:], 1e-30)) & (d != 0)
    return not close.any()


def _rows(rng, B, V, p, T):
    """B rows with most of the mass on a few candidate indices, screened."""
    rows = []
    while len(rows) < B:
        x = normal_f16(rng, (V,), 0, 2)
        nc = (V + 127) // 128
        hot = rng.choice(np.arange(0, V, 128), size=min(int(rng.integers(1, 9)), nc),
                         replace=False)
        x[hot] = (rng.random(hot.size) * 8 + 4).astype(np.float16)
        if rng.random() < 0.25 and hot.size > 1:
            x[hot[1]] = x[hot[0]]  # an exact tie between candidates
        if _safe(x, p, T):
            rows.append(x)
    return np.stack(rows)


@pytest.mark.parametrize("V", [100, 129, 1000, 4096, 30000])
@pytest.mark.parametrize("B", [1, 5, 64])
def test_top_p_vs_oracle(mk, orc, dev, V, B):
    rng = np.random.default_rng(V * 7 + B)
    for p, T in ((0.5, 1.0), (0.9, 0.7), (0.95, 1.3)):
        _case(f"top-p B={B} V={V} p={p} T={T}")
        x = _rows(rng, B, V, p, T)
        seed = int(rng.integers(0, 1 << 62))
        got = to_host(mk.top_p_sample(to_dev(x, dev), p, T, seed))
        want = orc.top_p_sample(x, p, T, seed)
        np.testing.assert_array_equal(got, want)
        if B == 1:  # the single-row entry point draws with the same seed
            out = to_dev(np.zeros(1, np.int32), dev)
            st = mk.load_library().mi_top_p_sample_f16(
                mk._ptr(to_dev(x[0], dev)), V, p, T, seed, mk._ptr(out), None)
            assert st == 0
            assert int(to_host(out)[0]) == int(want[0])


@pytest.mark.parametrize("V", [1000, 30000])
def test_top_p_large_logits_small_temperature(mk, orc, dev, V):
    """Logits far from zero (1e3 .. 6e4) at temperatures 0.1-0.5, where x / T
    reaches ~6e5 and its fp32 rounding is ~0.03: the normaliser and the
    candidate numerators must be formed consistently, or q moves by a few
    percent and the nucleus crossing with it.  Candidates sit a few fp16 ulps
    below the maximum (ties included), the rest 40 ulps below; p is placed
    1-3% away from a running sum (as q is exact to ~1e-6 in every consistent
    implementation, the screen still holds)."""
    rng = np.random.default_rng(V + 17)
    for base, T in ((1000.0, 0.5), (20000.0, 0.25), (60000.0, 0.1), (-30000.0, 0.2)):
        ulp = float(np.spacing(np.float16(abs(base))))
        for p in (0.32, 0.65, 0.9):
            _case(f"top-p large logits V={V} base={base} T={T} p={p}")
            rows = []
            while len(rows) < 8:
                x = np.full(V, base - 40 * ulp, dtype=np.float32)
                n = int(rng.integers(2, 6))
                hot = rng.choice(np.arange(0, V, 128), size=n, replace=False)
                x[hot] = base - ulp * rng.integers(0, 3, n)
                x = x.astype(np.float16)
                if _safe(x, p, T):
                    rows.append(x)
            x = np.stack(rows)
            seed = int(rng.integers(0, 1 << 62))
            got = to_host(mk.top_p_sample(to_dev(x, dev), p, T, seed))
            want = orc.top_p_sample(x, p, T, seed)
            np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("V", [128, 1000, 30000])
def test_top_p_unaligned_rows(mk, orc, dev, V):
    """Rows starting 0..7 halves past a 16-byte boundary: the kernel reads
    each row through an aligned window and masks the elements outside it."""
    import torch
    rng = np.random.default_rng(V + 3)
    B = 3
    x = _rows(rng, B, V, 0.9, 1.0)
    flat = torch.empty(B * V + 16, dtype=torch.float16, device=dev)
    want = orc.top_p_sample(x, 0.9, 1.0, 11)
    for off in range(8):
        _case(f"top-p V={V} rows at +{off} halves")
        flat.fill_(60.0)  # neighbours far above every logit: a stray read would win
        xs = flat[off:off + B * V].view(B, V)
        xs.copy_(torch.from_numpy(x).to(dev))
        got = to_host(mk.top_p_sample(xs, 0.9, 1.0, 11))
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("V", [1000, 30000])  # serial walk; double prefix + walk
@pytest.mark.parametrize("k", [3, 7])
def test_top_p_p_on_a_running_sum(mk, orc, dev, k, V):
    """p equal to (or one ulp either side of) the fp32 running sum at each
    position: within the kernel's error bound of its double prefix, so the
    in-order fp32 sum decides.  k equal candidates and every other logit at
    fp16's lowest value make q = fl(1/k) exactly on every implementation (exp
    of 0 is 1, the others underflow to 0), so no screening is needed."""
    _case(f"top-p: p on the running sums of {k} equal candidates, V={V}")
    x = np.full((1, V), np.finfo(np.float16).min, dtype=np.float16)
    x[0, np.arange(k) * 128] = 0.0
    q = np.float32(1.0) / np.float32(k)
    cums, c = [], np.float32(0.0)
    for _ in range(k):
        c = np.float32(c + q)
        cums.append(c)
    ps = set()
    for c in cums:
        ps.update((float(c), float(np.nextafter(c, np.float32(0))),
                   float(np.nextafter(c, np.float32(2)))))
    xd = to_dev(x, dev)
    for p in sorted(ps):
        for seed in (1, 99):
            got = to_host(mk.top_p_sample(xd, p, 1.0, seed))
            np.testing.assert_array_equal(got, orc.top_p_sample(x, p, 1.0, seed),
                                          err_msg=f"p={p!r} seed={seed}")


def test_top_p_nucleus_not_reached_and_ties(mk, orc, dev):
    _case("top-p: -1 when the candidates cannot reach p; exact ties")
    x = np.zeros((3, 1000), dtype=np.float16)
    x[0, 385] = 20            # the mass sits off the candidates: -1
    x[1, ::128] = 8           # eight equal candidates, ~all of the mass
    x[2, [0, 256]] = 10       # two equal candidates, p below either one
    for p, seed in ((0.5, 1), (0.9, 2), (0.3, 3)):
        got = to_host(mk.top_p_sample(to_dev(x, dev), p, 1.0, seed))
        np.testing.assert_array_equal(got, orc.top_p_sample(x, p, 1.0, seed))
    assert to_host(mk.top_p_sample(to_dev(x, dev), 0.5, 1.0, 1))[0] == -1


@pytest.mark.parametrize("V", [30001, 152064])
def test_top_p_above_30000_is_greedy(mk, orc, dev, V):
    _case(f"top-p V={V}: greedy")
    rng = np.random.default_rng(V)
    x = normal_f16(rng, (8, V), 0, 4)
    x[3, 17] = x[3, 9000] = 30  # a tie, resolved by the reference's tree order
    got = to_host(mk.top_p_sample(to_dev(x, dev), 0.9, 0.8, 5))
    np.testing.assert_array_equal(got, orc.greedy_argmax(x))
    np.testing.assert_array_equal(got, orc.top_p_sample(x, 0.9, 0.8, 5))


def test_top_p_empty_rows_and_refusals(mk, dev):
    import torch
    _case("top-p: empty rows, refusals")
    out = torch.full((3,), 7, dtype=torch.int32, device=dev)
    lib = mk.load_library()
    # vocab 0: the reference's kernel finds no candidate and returns -1
    assert lib.mi_top_p_sample_batched_f16(None, 3, 0, 0.9, 1.0, 1, mk._ptr(out), None) == 0
    assert to_host(out).tolist() == [-1, -1, -1]
    # B = 0: nothing written; negative sizes refused
    assert lib.mi_top_p_sample_batched_f16(None, 0, 10, 0.9, 1.0, 1, mk._ptr(out), None) == 0
    assert lib.mi_top_p_sample_batched_f16(None, -1, 10, 0.9, 1.0, 1, mk._ptr(out), None) == -1


def test_top_p_in_a_graph(mk, orc, dev):
    """Captured once, replayed several times with eager work between the
    replays; every replay matches the oracle (the launch allocates nothing
    and clears nothing)."""
    import torch
    _case("top-p: graph replays")
    rng = np.random.default_rng(77)
    x = _rows(rng, 16, 4096, 0.9, 1.0)
    xd = to_dev(x, dev)
    out = torch.empty(16, dtype=torch.int32, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mk.top_p_sample(xd, 0.9, 1.0, 123, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        mk.top_p_sample(xd, 0.9, 1.0, 123, out=out)
    want = orc.top_p_sample(x, 0.9, 1.0, 123)
    for _ in range(4):
        out.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_host(out), want)
    del graph
