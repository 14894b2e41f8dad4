"""GPU parity: RMSNorm, Gemma RMSNorm, Q/K RMSNorm and residual-add + RMSNorm
(HIP kernels through the C ABI vs the CPU oracle, same seeded inputs).

Tolerance: fp16 outputs within rtol = atol = 1e-3 of the fp32 oracle
(tests/verify/verify.py:142); the updated residual of the fused kernel is
bit-exact (it is the rounding of one fp32 add, src/kernels/model_utils_kernel.cu:34).
"""
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_bits_equal, assert_close, normal_f16, to_dev, to_host

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).resolve().parent / "golden" / "ref_cases.npz")


def _case(msg):
    print(f"[case] {msg}", flush=True)


def test_reference_case_std_and_gemma(mk, orc, dev):
    """tests/test_rmsnorm/main.cpp:83-124: x [4,4096] seed 42, w seed 7 x0.5."""
    _case("rmsnorm reference [4,4096]")
    x, w = GOLD["rms_x"], GOLD["rms_w"]
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    y = to_host(mk.rmsnorm(xd, wd, eps=1e-6))
    yg = to_host(mk.rmsnorm(xd, wd, eps=1e-6, add_one=True))
    assert_close(y, GOLD["rms_y"], what="std vs golden")
    assert_close(yg, GOLD["rms_y_gemma"], what="gemma vs golden")
    assert_close(y, orc.rmsnorm(x, w, 1e-6), what="std vs oracle")
    assert (y.view(np.uint16) != yg.view(np.uint16)).any()
    assert np.isfinite(y).all() and np.isfinite(yg).all()


def test_config1_16x3584(mk, orc, dev):
    """The small RMSNorm workload: x [16,3584] ~N(0,1), w ~N(1,0.1), eps 1e-6."""
    _case("rmsnorm [16,3584]")
    rng = np.random.default_rng(1)
    x = normal_f16(rng, (16, 3584))
    w = normal_f16(rng, (3584,), 1.0, 0.1)
    y = to_host(mk.rmsnorm(to_dev(x, dev), to_dev(w, dev), eps=1e-6))
    assert_close(y, orc.rmsnorm(x, w, 1e-6), what="cfg1")


@pytest.mark.parametrize("N,D", [(5, 8), (33, 16), (17, 64), (100, 128), (9, 136), (31, 320),
                                 (8, 512), (8, 520), (3, 1000), (7, 4096), (4, 8192),
                                 (2, 16384), (2, 16392), (2, 40000), (2, 70000), (3, 3583),
                                 (6, 7), (1, 3584), (17, 3584), (32, 3584), (33, 3584)])
@pytest.mark.parametrize("add_one", [False, True])
def test_shapes(mk, orc, dev, N, D, add_one):
    _case(f"rmsnorm [{N},{D}] add_one={add_one}")
    rng = np.random.default_rng(N * 7919 + D)
    x = normal_f16(rng, (N, D))
    w = normal_f16(rng, (D,), 0.0 if add_one else 1.0, 0.1)
    y = to_host(mk.rmsnorm(to_dev(x, dev), to_dev(w, dev), eps=1e-6, add_one=add_one))
    assert_close(y, orc.rmsnorm(x, w, 1e-6, add_one), what=f"[{N},{D}]")


def test_unaligned_scalar_path(mk, orc, dev):
    """A view 2 bytes into a buffer defeats 16-byte vectors: scalar kernel."""
    _case("rmsnorm unaligned")
    import torch
    rng = np.random.default_rng(3)
    x = normal_f16(rng, (12, 256))
    w = normal_f16(rng, (256,), 1.0, 0.1)
    buf = torch.empty(12 * 256 + 1, dtype=torch.float16, device=dev)
    xv = buf[1:].view(12, 256)
    xv.copy_(to_dev(x, dev))
    y = to_host(mk.rmsnorm(xv, to_dev(w, dev)))
    assert_close(y, orc.rmsnorm(x, w, 1e-6), what="unaligned")


def test_in_place(mk, orc, dev):
    _case("rmsnorm in place")
    rng = np.random.default_rng(4)
    for D in (128, 3584, 3583):
        x = normal_f16(rng, (64, D))
        w = normal_f16(rng, (D,), 1.0, 0.1)
        xd = to_dev(x, dev)
        mk.rmsnorm(xd, to_dev(w, dev), y=xd)
        assert_close(to_host(xd), orc.rmsnorm(x, w, 1e-6), what=f"in place D={D}")


def test_qk_norm_chain_shape(mk, orc, dev):
    """Q/K RMSNorm at the chain config: [6064*28, 128] and [6064*4, 128], in
    place, add_one = 0 (src/layers/attention.cpp:754-768)."""
    _case("qk-norm [169792,128] + [24256,128]")
    rng = np.random.default_rng(5)
    for rows in (6064 * 28, 6064 * 4):
        x = normal_f16(rng, (rows, 128))
        w = normal_f16(rng, (128,), 1.0, 0.1)
        xd = to_dev(x, dev)
        mk.rmsnorm(xd, to_dev(w, dev), y=xd, eps=1e-6)
        assert_close(to_host(xd), orc.rmsnorm(x, w, 1e-6, nthreads=8), what=f"qk rows={rows}")


@pytest.mark.parametrize("N,D", [(8192, 3584), (6064, 3584), (37, 128), (5, 3583), (3, 20000),
                                 (9, 3584), (31, 4096)])
def test_fused_add_rmsnorm(mk, orc, dev, N, D):
    """The headline workload ([8192,3584]) and the chain's residual+norm ([6064,3584])."""
    _case(f"fused add+rmsnorm [{N},{D}]")
    rng = np.random.default_rng(N + D)
    x = normal_f16(rng, (N, D))
    r = normal_f16(rng, (N, D))
    w = normal_f16(rng, (D,), 1.0, 0.1)
    xd, rd = to_dev(x, dev), to_dev(r, dev)
    y = to_host(mk.fused_add_rmsnorm(xd, rd, to_dev(w, dev), eps=1e-6))
    r_ref, y_ref = orc.fused_add_rmsnorm(x, r, w, 1e-6, nthreads=8)
    assert_bits_equal(to_host(rd), r_ref, what="residual")
    assert_close(y, y_ref, what="normed")


def test_fused_output_into_x(mk, orc, dev):
    _case("fused add+rmsnorm y == x")
    rng = np.random.default_rng(6)
    x = normal_f16(rng, (40, 3584))
    r = normal_f16(rng, (40, 3584))
    w = normal_f16(rng, (3584,), 1.0, 0.1)
    xd, rd = to_dev(x, dev), to_dev(r, dev)
    mk.fused_add_rmsnorm(xd, rd, to_dev(w, dev), y=xd)
    r_ref, y_ref = orc.fused_add_rmsnorm(x, r, w, 1e-6)
    assert_bits_equal(to_host(rd), r_ref, what="residual")
    assert_close(to_host(xd), y_ref, what="normed in x")


def test_argument_errors(mk, dev):
    import torch
    buf = torch.zeros(4 * 64 + 8, dtype=torch.float16, device=dev)
    x = buf[:256].view(4, 64)
    y = buf[8:].view(4, 64)  # overlaps x without being x
    w = torch.zeros(64, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError, match="status -3"):
        mk.fused_add_rmsnorm(x, x, w)  # residual aliases x
    with pytest.raises(RuntimeError, match="status -3"):
        mk.rmsnorm(x, w, y=y)


@pytest.mark.parametrize("N,D", [(64, 128), (16, 3584), (5, 3583)])
def test_signed_zero_weights(mk, orc, dev, N, D):
    """Weights of -0 and +0 give zero outputs whose sign is that of
    x * rrms * w, as the reference computes it (rmsnorm_kernel.cu:61-65):
    the Gemma bias is only added when add_one is set.  Small-row, long-row
    and scalar kernels, plain and fused."""
    _case(f"rmsnorm signed-zero weights [{N},{D}]")
    rng = np.random.default_rng(D)
    x = normal_f16(rng, (N, D))
    r = normal_f16(rng, (N, D))
    w = normal_f16(rng, (D,), 1.0, 0.1)
    w[0::4] = np.float16(-0.0)
    w[1::4] = np.float16(0.0)
    zero = np.zeros((N, D), bool)
    zero[:, 0::4] = zero[:, 1::4] = True
    y = to_host(mk.rmsnorm(to_dev(x, dev), to_dev(w, dev)))
    ref = orc.f32_to_f16(orc.rmsnorm(x, w))
    assert_bits_equal(y[zero], ref[zero], what="signed zeros, plain")
    assert_close(y, orc.rmsnorm(x, w), what="plain")
    yf = to_host(mk.fused_add_rmsnorm(to_dev(x, dev), to_dev(r, dev), to_dev(w, dev)))
    reff = orc.f32_to_f16(orc.fused_add_rmsnorm(x, r, w)[1])
    assert_bits_equal(yf[zero], reff[zero], what="signed zeros, fused")


@pytest.mark.parametrize("T,Hq,Hkv,hd,add_one,offset", [
    (6064, 28, 4, 128, False, 0),   # the chain config, one launch for Q and K
    (333, 8, 2, 64, True, 0),       # Gemma (1 + w), rows straddling workgroups at the Q/K seam
    (17, 4, 1, 256, False, 0),
    (9, 0, 3, 128, False, 0),       # K only
    (11, 5, 0, 128, False, 0),      # Q only
    (7, 3, 2, 128, False, 1),       # unaligned: two general launches
])
def test_qk_rmsnorm_one_launch(mk, orc, dev, T, Hq, Hkv, hd, add_one, offset):
    """mi_qk_rmsnorm_f16: the Gemma-3 Q-norm and K-norm pair in one launch,
    against the oracle (1e-3) and bit for bit against two mi_rmsnorm_f16 calls."""
    _case(f"qk rmsnorm one launch T={T} Hq={Hq} Hkv={Hkv} hd={hd}")
    import torch
    rng = np.random.default_rng(T + Hq + 7 * Hkv + hd)
    q = normal_f16(rng, (T, Hq, hd))
    k = normal_f16(rng, (T, Hkv, hd))
    wq, wk = normal_f16(rng, (hd,), 1.0, 0.1), normal_f16(rng, (hd,), 0.0 if add_one else 1.0, 0.1)

    def dev_buf(a):
        buf = torch.empty(a.size + offset, dtype=torch.float16, device=dev)
        t = buf[offset:].view(a.shape)
        t.copy_(to_dev(a, dev))
        return t
    qd, kd = dev_buf(q), dev_buf(k)
    mk.qk_rmsnorm(qd if Hq else kd, (kd if Hkv else None) if Hq else None,
                  to_dev(wq if Hq else wk, dev), to_dev(wk, dev) if Hq and Hkv else None,
                  eps=1e-6, add_one=add_one)
    for name, x, w, got in (("q", q, wq, qd), ("k", k, wk, kd)):
        if x.shape[1] == 0:
            continue
        rows = x.reshape(-1, hd)
        assert_close(to_host(got).reshape(-1, hd), orc.rmsnorm(rows, w, 1e-6, add_one, nthreads=8),
                     what=f"{name} vs oracle")
        if offset == 0:  # the same kernel arithmetic as one aligned mi_rmsnorm_f16 call
            two = to_dev(rows, dev)
            mk.rmsnorm(two, to_dev(w, dev), y=two, eps=1e-6, add_one=add_one)
            assert_bits_equal(to_host(got).reshape(-1, hd), to_host(two),
                              what=f"{name} vs mi_rmsnorm_f16")
