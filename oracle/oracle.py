"""numpy front end of the CPU oracle (oracle/libmi_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product path never imports
this module.

Arrays of fp16 values are numpy float16 arrays (passed to C as their uint16
bit patterns); results documented as fp32 are numpy float32 arrays.  Each
function names the C function and, through it, the reference lines it
restates (see mi_oracle.h).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmi_oracle.so"

_lib = None


def build() -> None:
    """Compile libmi_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-B", "-C", str(HERE)], check=True, capture_output=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I64, F, I, U32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_uint32
        sig = {
            "mio_f32_to_f16": ([F], ctypes.c_uint16),
            "mio_reftest_f32_to_f16": ([F], ctypes.c_uint16),
            "mio_f16_to_f32": ([ctypes.c_uint16], F),
            "mio_f32_to_f16_array": ([P, P, I64], None),
            "mio_reftest_f32_to_f16_array": ([P, P, I64], None),
            "mio_f16_to_f32_array": ([P, P, I64], None),
            "mio_fill_uniform": ([P, I64, F, U32], None),
            "mio_fill_uniform_int64": ([P, I64, U32, I64, I64], None),
            "mio_rmsnorm": ([P, P, P, I64, I64, F, I, I], None),
            "mio_fused_add_rmsnorm": ([P, P, P, P, I64, I64, F, I, I], None),
            "mio_rope_inv_freq": ([P, I, F], None),
            "mio_rope_tables": ([P, P, P, P, I64, I], None),
            "mio_rope_neox": ([P, P, P, P, I64, I, I, I], None),
            "mio_swiglu": ([P, P, P, I64, I], None),
            "mio_gelu_tanh": ([P, P, I64, I], None),
            "mio_geglu": ([P, P, P, I64, I], None),
            "mio_geglu_composed": ([P, P, P, I64], None),
            "mio_add_inplace": ([P, P, I64], None),
            "mio_add_bias": ([P, P, I64, I64, I64], None),
            "mio_mul_inplace": ([P, P, I64], None),
            "mio_scale_inplace": ([P, F, I64], None),
            "mio_softmax": ([P, P, I64, I64, I], None),
            "mio_embedding_gather": ([P, P, P, I64, I64, I64, I], None),
            "mio_paged_kv_scatter": ([P, P, P, P, P] + [I64] * 8, None),
            "mio_greedy_argmax": ([P, I64, I64, P], None),
            "mio_fmix64": ([ctypes.c_uint64], ctypes.c_uint64),
            "mio_top_p_sample": ([P, I64, I64, F, F, ctypes.c_uint64, P], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def _h(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float16))


# --- conversions and generators (tests/test_helpers.h, test_*/main.cpp) ---

def f32_to_f16(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    out = np.empty(a.shape, dtype=np.float16)
    lib().mio_f32_to_f16_array(_p(a), _p(out), a.size)
    return out


def reftest_f32_to_f16(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    out = np.empty(a.shape, dtype=np.float16)
    lib().mio_reftest_f32_to_f16_array(_p(a), _p(out), a.size)
    return out


def f16_to_f32(a) -> np.ndarray:
    a = _h(a)
    out = np.empty(a.shape, dtype=np.float32)
    lib().mio_f16_to_f32_array(_p(a), _p(out), a.size)
    return out


def fill_uniform(n: int, scale: float, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().mio_fill_uniform(_p(out), n, scale, seed)
    return out


def fill_uniform_int64(n: int, seed: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int64)
    lib().mio_fill_uniform_int64(_p(out), n, seed, lo, hi)
    return out


def reftest_input(shape, scale: float, seed: int) -> np.ndarray:
    """fp16 input exactly as a reference kernel test builds it."""
    n = int(np.prod(shape))
    return reftest_f32_to_f16(fill_uniform(n, scale, seed)).reshape(shape)


# --- kernels ---

def rmsnorm(x, w, eps=1e-6, add_one=False, nthreads=1) -> np.ndarray:
    x = _h(x); w = _h(w)
    N, D = x.shape
    y = np.empty((N, D), dtype=np.float32)
    lib().mio_rmsnorm(_p(x), _p(w), _p(y), N, D, eps, int(add_one), nthreads)
    return y


def fused_add_rmsnorm(x, residual, w, eps=1e-6, add_one=False, nthreads=1):
    """Returns (new residual fp16, y fp32); inputs are not modified."""
    x = _h(x); r = _h(residual).copy(); w = _h(w)
    N, D = x.shape
    y = np.empty((N, D), dtype=np.float32)
    lib().mio_fused_add_rmsnorm(_p(x), _p(r), _p(w), _p(y), N, D, eps, int(add_one), nthreads)
    return r, y


def rope_inv_freq(head_dim: int, theta: float = 1e6) -> np.ndarray:
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().mio_rope_inv_freq(_p(out), head_dim, theta)
    return out


def rope_tables(inv_freq, positions):
    inv = np.ascontiguousarray(np.asarray(inv_freq, dtype=np.float32))
    pos = np.ascontiguousarray(np.asarray(positions, dtype=np.int64))
    half = inv.size
    c = np.empty((pos.size, half), dtype=np.float16)
    s = np.empty((pos.size, half), dtype=np.float16)
    lib().mio_rope_tables(_p(inv), _p(pos), _p(c), _p(s), pos.size, half)
    return c, s


def rope_neox(x, cos_t, sin_t, nthreads=1) -> np.ndarray:
    """x: [T, H, hd] (or [B, S, H, hd]); tables [T, hd/2]; fp32 result."""
    x = _h(x); c = _h(cos_t); s = _h(sin_t)
    hd = x.shape[-1]
    H = x.shape[-2]
    T = x.size // (H * hd)
    y = np.empty(x.shape, dtype=np.float32)
    lib().mio_rope_neox(_p(x), _p(c), _p(s), _p(y), T, H, hd, nthreads)
    return y


def _ew(name, a, b=None, nthreads=1):
    a = _h(a)
    out = np.empty(a.shape, dtype=np.float32)
    if b is None:
        getattr(lib(), name)(_p(a), _p(out), a.size, nthreads)
    else:
        b = _h(b)
        getattr(lib(), name)(_p(a), _p(b), _p(out), a.size, nthreads)
    return out


def swiglu(g, u, nthreads=1):
    return _ew("mio_swiglu", g, u, nthreads)


def gelu_tanh(x, nthreads=1):
    return _ew("mio_gelu_tanh", x, None, nthreads)


def geglu(g, u, nthreads=1):
    return _ew("mio_geglu", g, u, nthreads)


def geglu_composed(g, u) -> np.ndarray:
    g = _h(g); u = _h(u)
    out = np.empty(g.shape, dtype=np.float16)
    lib().mio_geglu_composed(_p(g), _p(u), _p(out), g.size)
    return out


def add(y, x) -> np.ndarray:
    y = _h(y).copy(); x = _h(x)
    lib().mio_add_inplace(_p(y), _p(x), y.size)
    return y


def add_bias(y, bias, M: int, N: int, batch_stride: int) -> np.ndarray:
    """y (flat fp16, at least (batches - 1) * batch_stride + M * N elements)
    with bias [N] added to each of the M rows of every batch."""
    y = _h(y).copy(); bias = _h(bias)
    lib().mio_add_bias(_p(y), _p(bias), M, N, batch_stride)
    return y


def mul(y, x) -> np.ndarray:
    y = _h(y).copy(); x = _h(x)
    lib().mio_mul_inplace(_p(y), _p(x), y.size)
    return y


def scale(y, s: float) -> np.ndarray:
    y = _h(y).copy()
    lib().mio_scale_inplace(_p(y), s, y.size)
    return y


def softmax(x, nthreads=1) -> np.ndarray:
    x = _h(x)
    N, D = x.shape
    y = np.empty((N, D), dtype=np.float32)
    lib().mio_softmax(_p(x), _p(y), N, D, nthreads)
    return y


def embedding_gather(ids, table, vocab=None, nthreads=1) -> np.ndarray:
    ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int64))
    table = _h(table)
    V, H = table.shape
    out = np.empty((*ids.shape, H), dtype=np.float16)
    lib().mio_embedding_gather(_p(ids), _p(table), _p(out), ids.size, H,
                               V if vocab is None else vocab, nthreads)
    return out


def paged_kv_scatter(src, cache, block_table, seq_len, start_pos, layer, block_size):
    """src [B, S, H_kv, D] fp16; cache [L, num_blocks, H_kv, bs, D] fp16 (copied
    and returned); block_table int32 [B, max_blocks]; seq_len, start_pos int32 [B]."""
    src = _h(src); out = _h(cache).copy()
    bt = np.ascontiguousarray(np.asarray(block_table, dtype=np.int32))
    sl = np.ascontiguousarray(np.asarray(seq_len, dtype=np.int32))
    sp = np.ascontiguousarray(np.asarray(start_pos, dtype=np.int32))
    B, S, H, D = src.shape
    L, NB = out.shape[0], out.shape[1]
    assert out.shape == (L, NB, H, block_size, D)
    lib().mio_paged_kv_scatter(_p(src), _p(out), _p(bt), _p(sl), _p(sp), B, S, layer, NB, H, D,
                               block_size, bt.shape[1])
    return out


def greedy_argmax(logits) -> np.ndarray:
    x = _h(logits)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    B, V = x.shape
    out = np.empty(B, dtype=np.int32)
    lib().mio_greedy_argmax(_p(x), B, V, _p(out))
    return out


def fmix64(v: int) -> int:
    return int(lib().mio_fmix64(v & 0xFFFFFFFFFFFFFFFF))


def top_p_sample(logits, p: float, temperature: float, seed: int) -> np.ndarray:
    """logits [V] or [B, V] fp16; int32 [B] (row b with seed + b)."""
    x = _h(logits)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    B, V = x.shape
    out = np.empty(B, dtype=np.int32)
    lib().mio_top_p_sample(_p(x), B, V, p, temperature, seed & 0xFFFFFFFFFFFFFFFF, _p(out))
    return out
