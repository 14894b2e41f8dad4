"""GPU parity: SwiGLU, GeGLU, gelu_tanh and the in-place add / mul / scale.

Tolerances: activations within rtol = atol = 1e-3 of the fp32 oracle
(tests/verify/verify.py:142); add / mul / scale are one fp32 operation
rounded to fp16, so they are bit-exact.  GeGLU is additionally held within
the reference's two-kernel composition (gelu rounded to fp16, then mul).
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close, normal_f16, to_dev, to_host, ulp_diff

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).resolve().parent / "golden" / "ref_cases.npz")


def _case(msg):
    print(f"[case] {msg}", flush=True)


def test_reference_cases(mk, orc, dev):
    """tests/test_swiglu/main.cpp:63-68 and tests/test_gelu/main.cpp:64-67."""
    _case("swiglu/gelu reference n=4096")
    g, u = GOLD["swiglu_g"], GOLD["swiglu_u"]
    y = to_host(mk.swiglu(to_dev(g, dev), to_dev(u, dev)))
    assert_close(y, GOLD["swiglu_y"], what="swiglu vs golden")
    assert_close(y, orc.swiglu(g, u), what="swiglu vs oracle")
    gx = GOLD["gelu_x"]
    y = to_host(mk.gelu_tanh(to_dev(gx, dev)))
    assert_close(y, GOLD["gelu_y"], what="gelu vs golden")
    assert_close(y, orc.gelu_tanh(gx), what="gelu vs oracle")


def test_config4_swiglu_full(mk, orc, dev):
    """The SwiGLU workload: gate/up [4096, 18944] ~N(0,1)."""
    _case("swiglu [4096,18944]")
    rng = np.random.default_rng(41)
    g = normal_f16(rng, (4096, 18944))
    u = normal_f16(rng, (4096, 18944))
    y = to_host(mk.swiglu(to_dev(g, dev), to_dev(u, dev)))
    assert_close(y, orc.swiglu(g, u, nthreads=8), what="swiglu cfg4a")


def test_config4_geglu_full(mk, orc, dev):
    """The GeGLU workload: gate/up [4096, 14336] ~N(0,1)."""
    _case("geglu [4096,14336]")
    rng = np.random.default_rng(42)
    g = normal_f16(rng, (4096, 14336))
    u = normal_f16(rng, (4096, 14336))
    y = to_host(mk.geglu(to_dev(g, dev), to_dev(u, dev)))
    assert_close(y, orc.geglu(g, u, nthreads=8), what="geglu cfg4b")


def test_geglu_vs_reference_composition(mk, orc, dev):
    """The fused GeGLU rounds gelu(g) to fp16 before the multiply, as the
    reference's gelu_tanh + mul_inplace pair does (src/layers/mlp.cpp:282-291):
    it equals this library's own two-launch composition bit for bit, and the
    oracle's composition wherever the device and host gelu round to the same
    fp16 value."""
    _case("geglu vs gelu+mul composition")
    rng = np.random.default_rng(43)
    g = normal_f16(rng, (300_000,), 0, 3)
    u = normal_f16(rng, (300_000,))
    gd, ud = to_dev(g, dev), to_dev(u, dev)
    y = to_host(mk.geglu(gd, ud))
    a = mk.gelu_tanh(gd)
    gelu_dev = to_host(a)
    mk.mul_inplace(a, ud)
    assert_bits_equal(y, to_host(a), what="fused geglu vs gelu_tanh + mul_inplace")
    comp = orc.geglu_composed(g, u)
    same_gelu = gelu_dev.view(np.uint16) == orc.f32_to_f16(orc.gelu_tanh(g)).view(np.uint16)
    # below g = -3 the oracle's 0.5 x (1 + tanhf(u)) cancels in fp32 (the
    # reference formula, gelu_kernel.cuh:11) and its gelu is off by many ulps
    core = np.abs(g.astype(np.float32)) <= 3.0
    assert same_gelu[core].mean() > 0.999
    assert_bits_equal(y[same_gelu], comp[same_gelu], what="geglu vs oracle composition")
    assert_close(y, comp.astype(np.float32), what="geglu vs composition")


@pytest.mark.parametrize("n", [1, 7, 8, 9, 255, 8192, 8193, 1_000_003])
def test_odd_sizes(mk, orc, dev, n):
    _case(f"elementwise n={n}")
    rng = np.random.default_rng(n)
    g = normal_f16(rng, (n,), 0, 4)
    u = normal_f16(rng, (n,))
    gd, ud = to_dev(g, dev), to_dev(u, dev)
    assert_close(to_host(mk.swiglu(gd, ud)), orc.swiglu(g, u), what="swiglu")
    assert_close(to_host(mk.geglu(gd, ud)), orc.geglu(g, u), what="geglu")
    assert_close(to_host(mk.gelu_tanh(gd)), orc.gelu_tanh(g), what="gelu")


def test_extreme_inputs(mk, orc, dev):
    _case("activations at extremes")
    g = np.array([0, -0.0, 1e-7, -1e-7, 10, -10, 20, -20, 88, -88, 1000, -1000, 65504, -65504,
                  3.0, -3.0], dtype=np.float16)
    u = np.ones_like(g)
    gd, ud = to_dev(g, dev), to_dev(u, dev)
    assert_close(to_host(mk.swiglu(gd, ud)), orc.swiglu(g, u), what="swiglu")
    assert_close(to_host(mk.gelu_tanh(gd)), orc.gelu_tanh(g), what="gelu")


def test_unaligned(mk, orc, dev):
    _case("elementwise unaligned")
    import torch
    rng = np.random.default_rng(44)
    n = 5000
    g = normal_f16(rng, (n,))
    u = normal_f16(rng, (n,))
    buf = torch.empty(n + 1, dtype=torch.float16, device=dev)
    gv = buf[1:]
    gv.copy_(to_dev(g, dev))
    assert_close(to_host(mk.swiglu(gv, to_dev(u, dev))), orc.swiglu(g, u), what="swiglu")


def test_add_mul_scale_bit_exact(mk, orc, dev):
    _case("add/mul/scale")
    rng = np.random.default_rng(45)
    n = 1_000_001
    a = normal_f16(rng, (n,), 0, 50)
    b = normal_f16(rng, (n,), 0, 50)
    bd = to_dev(b, dev)
    y = to_dev(a, dev); mk.add_inplace(y, bd)
    assert_bits_equal(to_host(y), orc.add(a, b), what="add")
    y = to_dev(a, dev); mk.mul_inplace(y, bd)
    assert_bits_equal(to_host(y), orc.mul(a, b), what="mul")
    s = float(np.float32(np.sqrt(3584.0)))
    y = to_dev(a, dev); mk.scale_inplace(y, s)
    assert_bits_equal(to_host(y), orc.scale(a, s), what="scale")


def test_in_place_activation(mk, orc, dev):
    _case("swiglu out == gate")
    rng = np.random.default_rng(46)
    g = normal_f16(rng, (4096,))
    u = normal_f16(rng, (4096,))
    gd = to_dev(g, dev)
    mk.swiglu(gd, to_dev(u, dev), out=gd)
    assert_close(to_host(gd), orc.swiglu(g, u), what="in place")


@pytest.mark.parametrize("M,N,batches,gap,offset", [
    (6064, 3584, 1, 0, 0),    # Qwen2.5 q_proj bias at T = 6064 (vector path)
    (6064, 512, 1, 0, 0),     # k_proj / v_proj
    (37, 24, 3, 16, 0),       # three batches with gaps between them
    (5, 7, 2, 3, 0),          # N % 8 != 0: scalar path
    (33, 64, 1, 0, 1),        # unaligned y: scalar path
])
def test_add_bias_bit_exact(mk, orc, dev, M, N, batches, gap, offset):
    """launch_add_bias (model_utils_kernel.cu:11-28): every batch of M rows
    gets bias [N] added with one fp16 rounding; elements between batches are
    left alone."""
    _case(f"add_bias M={M} N={N} batches={batches} gap={gap} offset={offset}")
    import torch
    rng = np.random.default_rng(M * 7 + N + batches)
    stride = M * N + gap
    total = (batches - 1) * stride + M * N
    y = normal_f16(rng, (total,), 0, 30)
    bias = normal_f16(rng, (N,), 0, 30)
    buf = torch.empty(total + offset, dtype=torch.float16, device=dev)
    yd = buf[offset:]
    yd.copy_(to_dev(y, dev))
    mk.add_bias(yd, to_dev(bias, dev), M, N, stride)
    assert_bits_equal(to_host(yd), orc.add_bias(y, bias, M, N, stride), what="add_bias")


def test_add_bias_argument_errors(mk, dev):
    import torch
    y = torch.zeros(64, dtype=torch.float16, device=dev)
    b = torch.zeros(8, dtype=torch.float16, device=dev)
    mk.add_bias(y, b, 0, 8, 0)  # M == 0: nothing to do, as in the reference
    with pytest.raises(RuntimeError):
        mk.add_bias(y, b, 8, 8, 63)  # no whole batch
    with pytest.raises(RuntimeError):
        mk.add_bias(y, y[:8], 8, 8, 64)  # bias inside y
