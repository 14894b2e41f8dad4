"""Regenerates tests/golden/ref_cases.npz: the reference's own kernel-test
cases with expected outputs computed by torch on the CPU.

The reference keeps no golden files: each of its kernel tests rebuilds its
inputs from an xorshift32 seed (tests/test_helpers.h:46-68), converts them to
fp16 with its own host converter (tests/test_rmsnorm/main.cpp:40-67), runs
the kernel and checks the result against torch on the CPU through
tests/verify/verify.py (allclose rtol = atol = 1e-3).  This script rebuilds
the same inputs (oracle.reftest_input) and computes the expected outputs with
the torch operations verify.py names, written out here (verify.py itself is
not imported):
  rmsnorm   verify.py:32-44   x * rsqrt(mean(x^2) + eps) * w   (and 1 + w)
  rope      verify.py:47-66   tables as tests/test_rope/main.cpp:89-100
  softmax   verify.py:69-73   torch.softmax
  swiglu    verify.py:76-82   F.silu(g) * u
  gelu_tanh verify.py:85-91   F.gelu(x, approximate="tanh")
Cases (shapes, seeds, scales) are the reference tests':
  tests/test_rmsnorm/main.cpp:83-103, tests/test_rope/main.cpp:63-80,
  tests/test_swiglu/main.cpp:63-68, tests/test_gelu/main.cpp:64-67,
  tests/test_softmax/main.cpp:63-66.

Run from the repository root:  python tests/golden/make_golden.py
"""
import ctypes
import ctypes.util
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
import oracle  # noqa: E402


def t32(a):
    return torch.from_numpy(np.asarray(a).astype(np.float32))


def main():
    out = {}
    # rmsnorm: x [4, 4096] seed 42 x1.0, w [4096] seed 7 x0.5, eps 1e-6
    x = oracle.reftest_input((4, 4096), 1.0, 42)
    w = oracle.reftest_input((4096,), 0.5, 7)
    xf, wf = t32(x), t32(w)
    rrms = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    out.update(rms_x=x, rms_w=w, rms_y=(xf * rrms * wf).numpy(),
               rms_y_gemma=(xf * rrms * (1.0 + wf)).numpy())

    # rope: x [2, 16, 4, 64] seed 101, positions [16] seed 2024 in [0, 4096],
    # theta 1e6; the layer replicates positions across the batch
    # (src/layers/rope.cpp:66-71).  Tables: fp32 angle, fp16 cos/sin (RNE,
    # the kernel's __float2half) from the double cosine rounded to fp32.
    B, S, H, D = 2, 16, 4, 64
    half = D // 2
    xr = oracle.reftest_input((B, S, H, D), 1.0, 101)
    pos = oracle.fill_uniform_int64(S, 2024, 0, 4096)
    # inv_freq[i] = 1 / powf(theta, 2i/D) in fp32, as src/layers/rope.cpp:20-28
    # computes it with std::pow(float, float), i.e. the C library's powf.
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    libm.powf.restype = ctypes.c_float
    inv = np.array([np.float32(1.0) / np.float32(libm.powf(1e6, float(np.float32(2.0 * i)
                                                                      / np.float32(D))))
                    for i in range(half)], dtype=np.float32)
    ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float32)
    cos_t = np.cos(ang.astype(np.float64)).astype(np.float32).astype(np.float16)
    sin_t = np.sin(ang.astype(np.float64)).astype(np.float32).astype(np.float16)
    xt = t32(xr)
    c = t32(cos_t).reshape(1, S, 1, half)
    s = t32(sin_t).reshape(1, S, 1, half)
    x1, x2 = xt[..., :half], xt[..., half:]
    y = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)
    out.update(rope_x=xr, rope_pos=pos, rope_inv_freq=inv, rope_cos=cos_t, rope_sin=sin_t,
               rope_y=y.numpy())

    # swiglu: n = 4096, gate seed 11 x2, up seed 22 x2
    g = oracle.reftest_input((4096,), 2.0, 11)
    u = oracle.reftest_input((4096,), 2.0, 22)
    out.update(swiglu_g=g, swiglu_u=u, swiglu_y=(F.silu(t32(g)) * t32(u)).numpy())

    # gelu_tanh: n = 4096, seed 13 x2
    gx = oracle.reftest_input((4096,), 2.0, 13)
    out.update(gelu_x=gx, gelu_y=F.gelu(t32(gx), approximate="tanh").numpy())

    # softmax: [8, 1024], seed 555 x4
    sx = oracle.reftest_input((8, 1024), 4.0, 555)
    out.update(softmax_x=sx, softmax_y=torch.softmax(t32(sx), dim=-1).numpy())

    dst = Path(__file__).resolve().parent / "ref_cases.npz"
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({dst.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
