"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something it does not share code
with: the golden vectors of the reference's own test cases (outputs computed
by torch, tests/golden/make_golden.py), library routines (numpy's IEEE fp16
cast, torch's rms_norm / softmax / silu / gelu, libm powf), closed forms and
invariants, and brute force.  A dropped term, wrong sign, swapped half or
transposed operand in the oracle fails at least one of these.
"""
import ctypes
import ctypes.util
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import normal_f16, ulp_diff

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "ref_cases.npz")


def _wide_floats(n, seed):
    rng = np.random.default_rng(seed)
    mant = rng.standard_normal(n).astype(np.float64)
    expo = rng.integers(-30, 18, n)
    x = (mant * np.power(2.0, expo)).astype(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504, 65519.99, 65520, -65520,
                         6.1035156e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-9,
                         1.0 + 2**-11, 1.0 + 3 * 2**-11, 1.0 + 2**-11 + 2**-20],
                        dtype=np.float32)
    return np.concatenate([x, specials])


# ---------------------------------------------------------------------------
# conversions and generators
# ---------------------------------------------------------------------------

def test_f32_to_f16_is_ieee_rne():
    x = _wide_floats(400_000, 0)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    ours = O.f32_to_f16(x)
    same = (ours.view(np.uint16) == ref.view(np.uint16)) | (np.isnan(ours) & np.isnan(ref))
    assert same.all()


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    ours = O.f16_to_f32(h)
    ref = h.astype(np.float32)
    same = (ours.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(ours) & np.isnan(ref))
    assert same.all()


def test_reftest_converter_quirks():
    """The reference tests' converter equals IEEE RNE except where its two
    documented quirks apply: in the normal range it truncates instead of
    rounding up when the kept LSB is even; below 2^-14 it over-shifts."""
    x = _wide_floats(200_000, 1)
    x = x[np.isfinite(x) & (np.abs(x) < 65504)]
    with np.errstate(over="ignore"):
        rne = x.astype(np.float16)
    trunc = x.astype(np.float32)  # truncation toward zero to 10 mantissa bits
    tb = (trunc.view(np.uint32) & np.uint32(0xFFFFE000)).view(np.float32)
    with np.errstate(over="ignore"):
        trunc16 = tb.astype(np.float16)
    ours = O.reftest_f32_to_f16(x)
    normal = np.abs(x) >= 2.0 ** -14
    kept_lsb_odd = ((x.view(np.uint32) >> 13) & 1).astype(bool)
    # odd kept LSB: identical to RNE
    m = normal & kept_lsb_odd
    assert (ours[m].view(np.uint16) == rne[m].view(np.uint16)).all()
    # even kept LSB: truncation
    m = normal & ~kept_lsb_odd
    assert (ours[m].view(np.uint16) == trunc16[m].view(np.uint16)).all()
    # it does differ from RNE somewhere (so the quirk is real)
    assert (ours[normal].view(np.uint16) != rne[normal].view(np.uint16)).any()


def test_xorshift32_known_answer():
    # Marsaglia xorshift32 (13, 17, 5) from state 1 yields 270369 first.
    v = O.fill_uniform(1, 1.0, 1)[0]
    assert v == np.float32((270369 >> 1) / 2.0 ** 31 * 2.0 - 1.0)
    # seed 0 falls back to the golden-ratio constant (tests/test_helpers.h:50)
    assert (O.fill_uniform(4, 1.0, 0) == O.fill_uniform(4, 1.0, 0x9E3779B9)).all()


def test_xorshift32_brute_force_sequence():
    s = 42
    ref = []
    for _ in range(1000):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        # fp32 arithmetic throughout, as tests/test_helpers.h:53-55 writes it
        q = np.float32((s >> 1) & 0x7FFFFFFF) / np.float32(2.0 ** 31)
        ref.append((q * np.float32(2.0) - np.float32(1.0)) * np.float32(3.0))
    assert (O.fill_uniform(1000, 3.0, 42) == np.array(ref, dtype=np.float32)).all()


def test_uniform_int64_range():
    v = O.fill_uniform_int64(10_000, 2024, 0, 4096)
    assert v.min() >= 0 and v.max() <= 4096
    assert len(np.unique(v)) > 3000


# ---------------------------------------------------------------------------
# RMSNorm family
# ---------------------------------------------------------------------------

def test_rmsnorm_golden():
    y = O.rmsnorm(GOLD["rms_x"], GOLD["rms_w"], 1e-6)
    np.testing.assert_allclose(y, GOLD["rms_y"], rtol=1e-5, atol=1e-6)
    y = O.rmsnorm(GOLD["rms_x"], GOLD["rms_w"], 1e-6, add_one=True)
    np.testing.assert_allclose(y, GOLD["rms_y_gemma"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("shape", [(16, 3584), (7, 128), (3, 1000)])
def test_rmsnorm_vs_torch_rms_norm(shape):
    rng = np.random.default_rng(5)
    x = normal_f16(rng, shape)
    w = normal_f16(rng, shape[1:], 1.0, 0.1)
    ref = F.rms_norm(torch.from_numpy(x.astype(np.float32)), (shape[1],),
                     torch.from_numpy(w.astype(np.float32)), eps=1e-6).numpy()
    np.testing.assert_allclose(O.rmsnorm(x, w, 1e-6), ref, rtol=2e-6, atol=1e-6)


def test_rmsnorm_constant_row_and_gemma_identity():
    D = 256
    w = normal_f16(np.random.default_rng(1), (D,))
    x = np.full((2, D), 3.0, dtype=np.float16)
    x[1] = -0.5
    y = O.rmsnorm(x, w, eps=0.0)
    wf = w.astype(np.float32)
    np.testing.assert_allclose(y[0], wf, rtol=1e-6)
    np.testing.assert_allclose(y[1], -wf, rtol=1e-6)
    # Gemma variant == standard variant with weight 1 + w (fp32)
    yg = O.rmsnorm(x, w, eps=0.0, add_one=True)
    np.testing.assert_allclose(yg[0], 1.0 + wf, rtol=1e-6)


def test_fused_add_rmsnorm_composition():
    rng = np.random.default_rng(2)
    x = normal_f16(rng, (9, 384))
    r = normal_f16(rng, (9, 384))
    w = normal_f16(rng, (384,), 1.0, 0.1)
    new_r, y = O.fused_add_rmsnorm(x, r, w, 1e-6)
    # fp16 sum: numpy's IEEE cast of the fp32 sum, and the direct rounding of
    # the exact (float64) sum -- equal because fp32 keeps >= 2*11+2 bits.
    s32 = (x.astype(np.float32) + r.astype(np.float32)).astype(np.float16)
    s64 = (x.astype(np.float64) + r.astype(np.float64)).astype(np.float16)
    assert (new_r.view(np.uint16) == s32.view(np.uint16)).all()
    assert (new_r.view(np.uint16) == s64.view(np.uint16)).all()
    np.testing.assert_allclose(y, O.rmsnorm(s32, w, 1e-6), rtol=0, atol=0)


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def test_inv_freq_matches_libm_powf_and_closed_form():
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    libm.powf.restype = ctypes.c_float
    for hd in (64, 128, 256):
        inv = O.rope_inv_freq(hd, 1e6)
        ref = np.array([np.float32(1.0) / np.float32(libm.powf(1e6, float(np.float32(2.0 * i)
                                                                          / np.float32(hd))))
                        for i in range(hd // 2)], dtype=np.float32)
        assert (inv == ref).all()
        exact = 1e6 ** (-2.0 * np.arange(hd // 2) / hd)
        np.testing.assert_allclose(inv, exact, rtol=1e-6)
        assert inv[0] == 1.0 and (np.diff(inv) < 0).all()


def test_rope_tables_definition():
    inv = O.rope_inv_freq(128, 1e6)
    pos = np.array([0, 1, 7, 4095, 27999, 31999], dtype=np.int64)
    c, s = O.rope_tables(inv, pos)
    ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float32)
    assert (c == np.cos(ang.astype(np.float64)).astype(np.float32).astype(np.float16)).all()
    assert (s == np.sin(ang.astype(np.float64)).astype(np.float32).astype(np.float16)).all()
    assert (c[0] == 1).all() and (s[0] == 0).all()


def test_rope_golden():
    B, S, H, D = GOLD["rope_x"].shape
    c, s = O.rope_tables(GOLD["rope_inv_freq"], np.tile(GOLD["rope_pos"], B))
    assert (c[:S] == GOLD["rope_cos"]).all() and (s[:S] == GOLD["rope_sin"]).all()
    y = O.rope_neox(GOLD["rope_x"], c, s)
    np.testing.assert_allclose(y, GOLD["rope_y"], rtol=0, atol=0)


def test_rope_complex_formulation_and_invariants():
    """NeoX rotation == complex multiply of (x1 + i x2) by (c + i s)."""
    rng = np.random.default_rng(3)
    T, H, hd = 5, 3, 16
    x = normal_f16(rng, (T, H, hd))
    pos = np.array([0, 3, 100, 5000, 31000], dtype=np.int64)
    c, s = O.rope_tables(O.rope_inv_freq(hd, 1e6), pos)
    y = O.rope_neox(x, c, s)
    xf = x.astype(np.float64)
    z = (xf[..., :hd // 2] + 1j * xf[..., hd // 2:]) * (
        c.astype(np.float64) + 1j * s.astype(np.float64))[:, None, :]
    np.testing.assert_allclose(y[..., :hd // 2], z.real, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(y[..., hd // 2:], z.imag, rtol=1e-6, atol=1e-6)
    assert (y[0] == x[0].astype(np.float32)).all()  # position 0 is the identity
    n_in = xf[1:, :, :hd // 2] ** 2 + xf[1:, :, hd // 2:] ** 2
    n_out = y[1:, :, :hd // 2].astype(np.float64) ** 2 + y[1:, :, hd // 2:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=2e-3, atol=1e-6)  # fp16 cos/sin -> ~1e-3


# ---------------------------------------------------------------------------
# Activations, elementwise, softmax, gather
# ---------------------------------------------------------------------------

def test_swiglu_gelu_softmax_golden():
    np.testing.assert_allclose(O.swiglu(GOLD["swiglu_g"], GOLD["swiglu_u"]), GOLD["swiglu_y"],
                               rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(O.gelu_tanh(GOLD["gelu_x"]), GOLD["gelu_y"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(O.softmax(GOLD["softmax_x"]), GOLD["softmax_y"], rtol=1e-5,
                               atol=1e-8)


def test_activations_vs_torch_wide_range():
    rng = np.random.default_rng(4)
    g = normal_f16(rng, (100_000,), 0.0, 6.0)
    u = normal_f16(rng, (100_000,))
    gt, ut = torch.from_numpy(g.astype(np.float32)), torch.from_numpy(u.astype(np.float32))
    np.testing.assert_allclose(O.swiglu(g, u), (F.silu(gt) * ut).numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(O.gelu_tanh(g), F.gelu(gt, approximate="tanh").numpy(),
                               rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(O.geglu(g, u), (F.gelu(gt, approximate="tanh") * ut).numpy(),
                               rtol=1e-6, atol=1e-6)
    assert O.swiglu(np.zeros(3, np.float16), np.ones(3, np.float16)).tolist() == [0, 0, 0]
    assert O.gelu_tanh(np.zeros(3, np.float16)).tolist() == [0, 0, 0]


def test_geglu_composed_within_one_ulp_of_fused():
    rng = np.random.default_rng(6)
    g = normal_f16(rng, (50_000,))
    u = normal_f16(rng, (50_000,))
    fused = O.geglu(g, u).astype(np.float16)
    comp = O.geglu_composed(g, u)
    assert (ulp_diff(fused, comp) <= 1).all()


def test_elementwise_bit_exact_vs_numpy():
    rng = np.random.default_rng(7)
    a = normal_f16(rng, (10_000,), 0, 100)
    b = normal_f16(rng, (10_000,), 0, 100)
    assert (O.add(a, b) == (a.astype(np.float32) + b.astype(np.float32)).astype(np.float16)).all()
    with np.errstate(over="ignore"):
        assert (O.mul(a, b).view(np.uint16) ==
                (a.astype(np.float32) * b.astype(np.float32)).astype(np.float16).view(np.uint16)).all()
    s = np.float32(np.sqrt(3584.0))
    with np.errstate(over="ignore"):
        assert (O.scale(a, s).view(np.uint16) ==
                (a.astype(np.float32) * s).astype(np.float16).view(np.uint16)).all()


def test_add_bias_brute_force_and_numpy_broadcast():
    """mio_add_bias (model_utils_kernel.cu:11-28): numpy's broadcast add with an
    IEEE cast on a whole-batch layout; a strided layout (batch_stride > M*N)
    leaves the gaps untouched; batch_stride below M*N (no batch) and M == 0 do
    nothing; a bias of -0 keeps every bit."""
    rng = np.random.default_rng(17)
    M, N = 37, 24
    y = normal_f16(rng, (3, M, N), 0, 50)
    bias = normal_f16(rng, (N,), 0, 50)
    want = (y.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    got = O.add_bias(y.reshape(-1), bias, M, N, M * N)
    assert (got[: M * N] == want[0].reshape(-1)).all()
    assert (got[M * N:] == y.reshape(-1)[M * N:]).all()  # batch_stride = M*N: one batch
    got3 = O.add_bias(y.reshape(-1), bias, M, N // 2, M * (N // 2) * 2)  # 2 batches of half rows
    flat = y.reshape(-1).astype(np.float32)
    exp3 = flat.copy()
    for b in range(2):
        for m in range(M):
            for n in range(N // 2):
                i = b * M * (N // 2) * 2 + m * (N // 2) + n
                exp3[i] = flat[i] + np.float32(bias[n])
    exp3 = np.where(np.isin(np.arange(flat.size), [b * M * N + m * (N // 2) + n for b in range(2)
                                                   for m in range(M) for n in range(N // 2)]),
                    exp3.astype(np.float16), y.reshape(-1))
    assert (got3.view(np.uint16) == exp3.astype(np.float16).view(np.uint16)).all()
    assert (O.add_bias(y.reshape(-1), bias, M, N, M * N - 1) == y.reshape(-1)).all()
    assert (O.add_bias(y.reshape(-1), bias, 0, N, 0) == y.reshape(-1)).all()
    z = np.full(N, -0.0, dtype=np.float16)
    assert (O.add_bias(y.reshape(-1), z, M, N, M * N).view(np.uint16)[: M * N] ==
            y.reshape(-1).view(np.uint16)[: M * N]).all()


def test_softmax_vs_torch_and_invariants():
    rng = np.random.default_rng(8)
    x = normal_f16(rng, (4, 5000), 0, 4)
    y = O.softmax(x)
    np.testing.assert_allclose(y, torch.softmax(torch.from_numpy(x.astype(np.float32)), -1).numpy(),
                               rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(y.sum(-1), 1.0, rtol=1e-6)
    # shift invariance on a grid where the shift is exact in fp16
    # (multiples of 2^-6 in [-8, 8) plus 8 need at most 10 significant bits)
    g = (rng.integers(-512, 512, (3, 700)) / 64.0).astype(np.float16)
    y1 = O.softmax(g)
    y2 = O.softmax((g.astype(np.float32) + 8.0).astype(np.float16))
    np.testing.assert_allclose(y2, y1, rtol=1e-6, atol=1e-12)


def test_embedding_gather_brute_force():
    rng = np.random.default_rng(9)
    table = normal_f16(rng, (1000, 72), 0, 0.02)
    ids = rng.integers(0, 1000, (3, 11))
    out = O.embedding_gather(ids, table, nthreads=4)
    assert (out.view(np.uint16) == table[ids].view(np.uint16)).all()
    bad = np.array([0, -1, 1000, 999], dtype=np.int64)
    out = O.embedding_gather(bad, table)
    assert (out[1] == 0).all() and (out[2] == 0).all()
    assert (out[3] == table[999]).all()


def test_threaded_matches_single_thread():
    rng = np.random.default_rng(10)
    x = normal_f16(rng, (64, 512))
    w = normal_f16(rng, (512,), 1.0, 0.1)
    assert (O.rmsnorm(x, w, nthreads=1) == O.rmsnorm(x, w, nthreads=8)).all()
    assert (O.softmax(x, nthreads=1) == O.softmax(x, nthreads=8)).all()


# ---------------------------------------------------------------------------
# Paged KV scatter and greedy argmax (the steps either side of the chain)
# ---------------------------------------------------------------------------

def _bitrev8(u):
    return int(f"{u:08b}"[::-1], 2)


def _argmax_rule(row):
    """The reference kernel's result stated as a rule: among entries equal to
    the maximum (NaN ignored, -0 == +0, only values above -inf), the one whose
    thread u = i mod 256 has the smallest 8-bit bit reversal (the tree keeps
    the lower slot, so u's low bits decide first), then the smallest i; -1 if
    none."""
    v = row.astype(np.float32)
    ok = ~np.isnan(v) & (v > -np.inf)
    if not ok.any():
        return -1
    m = v[ok].max()
    idx = np.nonzero(ok & (v == m))[0]
    return int(min(idx, key=lambda i: (_bitrev8(i % 256), i)))


def test_greedy_argmax_simulation_matches_rule_and_numpy():
    rng = np.random.default_rng(11)
    # distinct maxima: plain argmax
    x = normal_f16(rng, (6, 5000), 0, 4)
    x[np.arange(6), rng.integers(0, 5000, 6)] = 60.0
    assert (O.greedy_argmax(x) == np.argmax(x.astype(np.float32), axis=1)).all()
    # heavy ties: values on a coarse grid
    t = (rng.integers(-3, 4, (20, 3000))).astype(np.float16)
    got = O.greedy_argmax(t)
    assert [int(g) for g in got] == [_argmax_rule(r) for r in t]
    # ties where the smaller index is not the answer: thread 128 (reversed 1)
    # beats thread 1 (reversed 128); i = 300 (thread 44 = 0b00101100,
    # reversed 52) beats i = 100 (thread 100 = 0b01100100, reversed 38)? no:
    # 38 < 52, so 100 wins there
    r = np.zeros(1500, dtype=np.float16)
    r[1281] = 5; r[128] = 5
    assert O.greedy_argmax(r)[0] == 128 == _argmax_rule(r)
    r = np.zeros(1000, dtype=np.float16)
    r[100] = 5; r[300] = 5
    assert O.greedy_argmax(r)[0] == 100 == _argmax_rule(r)
    r = np.zeros(1000, dtype=np.float16)
    r[2] = 5; r[257] = 5  # thread 2 (reversed 64) vs thread 1 (reversed 128)
    assert O.greedy_argmax(r)[0] == 2 == _argmax_rule(r)
    # NaN never chosen, -0 == +0, all -inf -> -1
    r = np.array([np.nan, -0.0, 0.0, -1.0], dtype=np.float16)
    assert O.greedy_argmax(r)[0] == 2 == _argmax_rule(r)  # -0 ties +0; thread 2 beats 1
    assert O.greedy_argmax(np.full(10, -np.inf, dtype=np.float16))[0] == -1


def test_paged_kv_scatter_brute_force():
    rng = np.random.default_rng(12)
    B, S, H, D, bs, L, NB, MB = 3, 9, 2, 16, 4, 2, 20, 5
    src = normal_f16(rng, (B, S, H, D))
    cache = normal_f16(rng, (L, NB, H, bs, D))
    bt = rng.permutation(NB)[:B * MB].reshape(B, MB).astype(np.int32)
    bt[2, 3] = -1                     # an unallocated block: skipped
    start = np.array([0, 5, 8], dtype=np.int32)
    seq = np.array([9, 12, 20], dtype=np.int32)  # b=1 keeps s < 7
    out = O.paged_kv_scatter(src, cache, bt, seq, start, layer=1, block_size=bs)
    ref = cache.copy()
    for b in range(B):
        for s in range(S):
            p = start[b] + s
            if p >= seq[b] or p // bs >= MB or bt[b, p // bs] < 0:
                continue
            ref[1, bt[b, p // bs], :, p % bs, :] = src[b, s]
    assert (out.view(np.uint16) == ref.view(np.uint16)).all()
    assert (out[0].view(np.uint16) == cache[0].view(np.uint16)).all()  # other layer untouched


# --- top-p sampling (launch_top_p_sample, sampling_kernel.cu:86-221) ---------

_M64 = (1 << 64) - 1


def _fmix64_inverse(h):
    """The published inverse of MurmurHash3's fmix64 (its own constants)."""
    h ^= h >> 33
    h = (h * 0x9CB4B2F8129337DB) & _M64
    h ^= h >> 33
    h = (h * 0x4F74430C22A54005) & _M64
    h ^= h >> 33
    return h


def test_fmix64_known_answer_and_inverse():
    # fmix64(1) is MurmurHash3's widely quoted value; the inverse, built from
    # different constants, undoes it only if both multipliers and all shifts
    # are right
    assert O.fmix64(1) == 0xB456BCFC34C2CB2C
    assert O.fmix64(0) == 0
    rng = np.random.default_rng(5)
    for v in [int(a) for a in rng.integers(0, 1 << 63, 200, dtype=np.int64)] + [_M64, 1 << 63]:
        assert _fmix64_inverse(O.fmix64(v)) == v


def _top_p_by_sorting(x, p, T, seed):
    """The rule restated as a sort (not the reference's K selection rounds):
    candidates at multiples of 128 in (q descending, index ascending) order,
    the fp32 running sum, the fmix64 slot."""
    xf = x.astype(np.float32) / np.float32(T)
    m = xf.max()
    e = np.exp((xf - m).astype(np.float64))
    S = np.float32(e.sum())
    idx = np.arange(0, x.size, 128)
    q = (np.exp((xf[idx] - m)).astype(np.float32) / S).astype(np.float32)
    order = np.lexsort((idx, -q))
    cum = np.float32(0)
    for i, o in enumerate(order):
        cum = np.float32(cum + q[o])
        if cum >= np.float32(p):
            h = O.fmix64(seed ^ (int(idx[o]) << 32))
            u = np.float32(h & 0xFFFFFF) / np.float32(1 << 24)
            slot = min(max(int(np.float32(u * np.float32(i + 1))), 0), i)
            return int(idx[order[slot]])
    return -1


def test_top_p_rules():
    rng = np.random.default_rng(21)
    # above 30000 logits: the greedy argmax
    x = normal_f16(rng, (3, 30001), 0, 3)
    assert (O.top_p_sample(x, 0.9, 0.8, 7) == O.greedy_argmax(x)).all()
    # a dominant candidate: the running sum passes p at the first slot
    x = normal_f16(rng, (1000,), 0, 1)
    x[384] = 30
    assert O.top_p_sample(x, 0.9, 1.0, 3)[0] == 384
    # a dominant logit that is not a candidate: the sum never reaches p
    x[384] = 0
    x[385] = 30
    assert O.top_p_sample(x, 0.5, 1.0, 3)[0] == -1
    # nothing but candidates can be returned; equal logits order by index
    x = np.zeros(640, dtype=np.float16)
    x[::128] = 8  # five equal candidates holding 95.9% of the mass
    seen = set()
    for seed in range(20):
        got = O.top_p_sample(x, 0.9, 1.0, seed)[0]
        assert got == _top_p_by_sorting(x, 0.9, 1.0, seed) and got >= 0 and got % 128 == 0
        seen.add(int(got))
    assert len(seen) > 1  # the draw spreads over the nucleus


@pytest.mark.parametrize("V", [129, 1000, 4096, 30000])
def test_top_p_selection_rounds_match_a_sort(V):
    rng = np.random.default_rng(V)
    for trial in range(12):
        x = normal_f16(rng, (V,), 0, 2)
        hot = rng.choice(np.arange(0, V, 128), size=min(6, (V + 127) // 128), replace=False)
        x[hot] = (rng.random(hot.size) * 6 + 6).astype(np.float16)  # mass on candidates
        p, T, seed = float(rng.choice([0.3, 0.6, 0.9])), float(rng.choice([0.7, 1.0])), trial
        assert O.top_p_sample(x, p, T, seed)[0] == _top_p_by_sorting(x, p, T, seed)
    # rows of a batch draw with seed + row
    xb = normal_f16(rng, (4, V), 0, 2)
    xb[:, 0] = 12
    xb[:, 128 % V] = 12
    got = O.top_p_sample(xb, 0.95, 1.0, 100)
    assert [int(g) for g in got] == [_top_p_by_sorting(xb[b], 0.95, 1.0, 100 + b)
                                     for b in range(4)]
