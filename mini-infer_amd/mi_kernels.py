"""ctypes binding of libmi_kernels.so (the C ABI in include/mi_kernels.h).

PyTorch is used here only for device memory and streams: every function takes
torch CUDA (HIP) tensors, checks dtype / contiguity / shape on the host, and
enqueues the HIP kernel on the current torch stream through the C ABI.  There
is no fallback: if the shared library is missing, or the call's status is not
0, a RuntimeError is raised.

The functions mirror the reference's ``mini_infer::kernels::launch_*`` entry
points (src/kernels/<name>_kernel.cuh in the reference tree); the two fused
ops (``fused_add_rmsnorm``, ``geglu``) and the positions-driven
``rope_neox_qk`` are additions named after what they fuse.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libmi_kernels.so"

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int

# name -> argtypes (restype is int for every entry point)
SIGNATURES = {
    "mi_rmsnorm_f16": [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32, _int, _c_void_p],
    "mi_fused_add_rmsnorm_f16": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32,
                                 _int, _c_void_p],
    "mi_rope_neox_f16": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
                         _c_void_p],
    "mi_rope_tables_f16": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "mi_rope_neox_qk_f16": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
                            _c_void_p],
    "mi_qk_rmsnorm_f16": [_c_void_p] * 4 + [_i64] * 4 + [_f32, _int, _c_void_p],
    "mi_qk_norm_rope_f16": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                            _i64, _i64, _i64, _i64, _f32, _int, _c_void_p],
    "mi_swiglu_f16": [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p],
    "mi_gelu_tanh_f16": [_c_void_p, _c_void_p, _i64, _c_void_p],
    "mi_geglu_f16": [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p],
    "mi_add_inplace_f16": [_c_void_p, _c_void_p, _i64, _c_void_p],
    "mi_mul_inplace_f16": [_c_void_p, _c_void_p, _i64, _c_void_p],
    "mi_scale_inplace_f16": [_c_void_p, _f32, _i64, _c_void_p],
    "mi_add_bias_f16": [_c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p],
    "mi_bias_rope_neox_qk_f16": [_c_void_p] * 5 + [_c_void_p, _i64, _i64, _i64, _i64, _c_void_p],
    "mi_paged_kv_scatter_kv_bias_f16": [_c_void_p] * 9 + [_i64] * 8 + [_c_void_p],
    "mi_rope_kv_scatter_f16": [_c_void_p] * 8 + [_i64] * 4 + [_c_void_p, _c_void_p] + [_i64] * 3
                              + [_c_void_p, _int, _c_void_p],
    "mi_qk_norm_rope_kv_scatter_f16": [_c_void_p] * 6 + [_c_void_p] + [_i64] * 4 + [_f32, _int]
                                      + [_c_void_p, _c_void_p] + [_i64] * 3
                                      + [_c_void_p, _int, _c_void_p],
    "mi_top_p_sample_f16": [_c_void_p, _i64, _f32, _f32, ctypes.c_uint64, _c_void_p, _c_void_p],
    "mi_top_p_sample_batched_f16": [_c_void_p, _i64, _i64, _f32, _f32, ctypes.c_uint64,
                                    _c_void_p, _c_void_p],
    "mi_softmax_f16": [_c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "mi_embedding_gather_f16": [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p],
    "mi_embedding_rmsnorm_f16": [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                 _i64, _i64, _f32, _f32, _int, _c_void_p],
    "mi_softmax_ws_f16": [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i64, _c_void_p],
    "mi_softmax_noalloc_f16": [_c_void_p, _c_void_p, _i64, _i64, _c_void_p],
    "mi_softmax_argmax_ws_f16": [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i64,
                                 _c_void_p],
    "mi_paged_kv_scatter_f16": [_c_void_p] * 5 + [_i64] * 8 + [_c_void_p],
    "mi_paged_kv_scatter_kv_f16": [_c_void_p] * 7 + [_i64] * 8 + [_c_void_p],
    "mi_greedy_argmax_f16": [_c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "mi_greedy_argmax_ws_f16": [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64, _c_void_p],
    "mi_softmax_test_poll_limit": [_int],
    "mi_greedy_argmax_test_poll_limit": [_int],
    "mi_exchange_test_mode": [_int],
    "mi_abi_version": [],
}

_lib = None


def load_library(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load (once) and type the kernel library; raise if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is not built; run __graft_entry__.build() (or `make -C mini-infer_amd`)")
    lib = ctypes.CDLL(str(p))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _int
    lib.mi_greedy_argmax_workspace_bytes.argtypes = [_i64, _i64]
    lib.mi_greedy_argmax_workspace_bytes.restype = _i64
    lib.mi_softmax_workspace_bytes.argtypes = [_i64, _i64]
    lib.mi_softmax_workspace_bytes.restype = _i64
    lib.mi_softmax_argmax_workspace_bytes.argtypes = [_i64, _i64]
    lib.mi_softmax_argmax_workspace_bytes.restype = _i64
    lib.mi_status_string.argtypes = [_int]
    lib.mi_status_string.restype = ctypes.c_char_p
    if path is None:
        _lib = lib
    return lib


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = load_library().mi_status_string(status).decode()
        raise RuntimeError(f"{what} failed: status {status} ({msg})")


def _torch():
    import torch  # noqa: PLC0415  (imported lazily so CPU-only users can load the ABI)
    return torch


def _stream(stream):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _need(t, dtype, name: str) -> None:
    torch = _torch()
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU, got {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _f16():
    return _torch().float16


# ---------------------------------------------------------------------------
# RMSNorm family (reference: launch_rmsnorm, src/kernels/rmsnorm_kernel.cuh:19)
# ---------------------------------------------------------------------------

def rmsnorm(x, weight, y=None, eps: float = 1e-6, add_one: bool = False, stream=None):
    """y = x * rsqrt(mean(x^2) + eps) * (1 + w if add_one else w); x: [N, D]."""
    _need(x, _f16(), "x"); _need(weight, _f16(), "weight")
    if x.dim() != 2:
        raise ValueError("x must be 2-D [N, D]")
    N, D = x.shape
    if weight.numel() != D:
        raise ValueError("weight size must equal D")
    if y is None:
        y = _torch().empty_like(x)
    _need(y, _f16(), "y")
    if y.shape != x.shape:
        raise ValueError("y must have x's shape")
    _check(load_library().mi_rmsnorm_f16(_ptr(x), _ptr(weight), _ptr(y), N, D, eps,
                                         int(bool(add_one)), _stream(stream)), "mi_rmsnorm_f16")
    return y


def fused_add_rmsnorm(x, residual, weight, y=None, eps: float = 1e-6, add_one: bool = False,
                      stream=None):
    """residual <- half(residual + x); y = rmsnorm(residual).  Returns y."""
    _need(x, _f16(), "x"); _need(residual, _f16(), "residual"); _need(weight, _f16(), "weight")
    if x.dim() != 2 or residual.shape != x.shape:
        raise ValueError("x and residual must be 2-D [N, D] of the same shape")
    N, D = x.shape
    if weight.numel() != D:
        raise ValueError("weight size must equal D")
    if y is None:
        y = _torch().empty_like(x)
    _need(y, _f16(), "y")
    if y.shape != x.shape:
        raise ValueError("y must have x's shape")
    _check(load_library().mi_fused_add_rmsnorm_f16(_ptr(x), _ptr(residual), _ptr(weight), _ptr(y),
                                                   N, D, eps, int(bool(add_one)),
                                                   _stream(stream)), "mi_fused_add_rmsnorm_f16")
    return y


# ---------------------------------------------------------------------------
# RoPE (reference: launch_rope / launch_rope_precompute*, rope_kernel.cuh:11-28)
# ---------------------------------------------------------------------------

def _inv_freq_buffer(inv_freq):
    """inv_freq as a host float32 ctypes array (the ABI reads it on the host)."""
    import numpy as np  # noqa: PLC0415
    a = np.ascontiguousarray(np.asarray(inv_freq, dtype=np.float32))
    return a, a.ctypes.data_as(ctypes.c_void_p)


def rope_neox(x, cos_t, sin_t, y=None, stream=None):
    """Table-driven NeoX RoPE; x: [B, S, H, D], tables [B*S, D/2]; y may be x."""
    _need(x, _f16(), "x"); _need(cos_t, _f16(), "cos_t"); _need(sin_t, _f16(), "sin_t")
    if x.dim() != 4:
        raise ValueError("x must be 4-D [B, S, H, D]")
    B, S, H, D = x.shape
    if cos_t.numel() != B * S * (D // 2) or sin_t.numel() != B * S * (D // 2):
        raise ValueError("cos/sin tables must be [B*S, D/2]")
    if y is None:
        y = _torch().empty_like(x)
    _need(y, _f16(), "y")
    _check(load_library().mi_rope_neox_f16(_ptr(x), _ptr(cos_t), _ptr(sin_t), _ptr(y), B, S, H, D,
                                           _stream(stream)), "mi_rope_neox_f16")
    return y


def rope_inv_freq(head_dim: int, theta: float = 1e6):
    """inv_freq[i] = 1 / powf(theta, 2i/head_dim) in fp32, computed on the host
    with the C library's powf, as RoPE::recompute_inv_freq_ does
    (src/layers/rope.cpp:20-28)."""
    import ctypes.util  # noqa: PLC0415
    import numpy as np  # noqa: PLC0415
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    libm.powf.restype = ctypes.c_float
    hd = np.float32(head_dim)
    return np.array([np.float32(1.0) / np.float32(libm.powf(theta, float(np.float32(2.0 * i) / hd)))
                     for i in range(head_dim // 2)], dtype=np.float32)


def rope_tables(inv_freq, positions, cos_t=None, sin_t=None, stream=None):
    """fp16 cos/sin tables [N, half] for device int64 positions [N]."""
    torch = _torch()
    _need(positions, torch.int64, "positions")
    arr, p = _inv_freq_buffer(inv_freq)
    half = arr.size
    N = positions.numel()
    if cos_t is None:
        cos_t = torch.empty((N, half), dtype=torch.float16, device=positions.device)
    if sin_t is None:
        sin_t = torch.empty((N, half), dtype=torch.float16, device=positions.device)
    _need(cos_t, _f16(), "cos_t"); _need(sin_t, _f16(), "sin_t")
    if cos_t.numel() != N * half or sin_t.numel() != N * half:
        raise ValueError("tables must hold N * half elements")
    _check(load_library().mi_rope_tables_f16(p, _ptr(positions), _ptr(cos_t), _ptr(sin_t), N, half,
                                             _stream(stream)), "mi_rope_tables_f16")
    return cos_t, sin_t


def rope_neox_qk(q, k, positions, inv_freq, stream=None):
    """In-place NeoX RoPE of q [T, Hq, hd] and k [T, Hkv, hd] (k may be None)."""
    torch = _torch()
    _need(q, _f16(), "q"); _need(positions, torch.int64, "positions")
    if q.dim() != 3:
        raise ValueError("q must be 3-D [T, Hq, hd]")
    T, Hq, hd = q.shape
    Hkv = 0
    if k is not None:
        _need(k, _f16(), "k")
        if k.dim() != 3 or k.shape[0] != T or k.shape[2] != hd:
            raise ValueError("k must be [T, Hkv, hd]")
        Hkv = k.shape[1]
    if positions.numel() != T:
        raise ValueError("positions must hold T entries")
    arr, p = _inv_freq_buffer(inv_freq)
    if arr.size != hd // 2:
        raise ValueError("inv_freq must hold head_dim/2 entries")
    kp = _ptr(k) if k is not None else ctypes.c_void_p(0)
    _check(load_library().mi_rope_neox_qk_f16(_ptr(q), kp, _ptr(positions), p, T, Hq, Hkv, hd,
                                              _stream(stream)), "mi_rope_neox_qk_f16")
    return q, k


def bias_rope_neox_qk(q, k, q_bias, k_bias, positions, inv_freq, stream=None):
    """In place: q = rope(half(q + q_bias)), k = rope(half(k + k_bias)) for
    q [T, Hq, hd], k [T, Hkv, hd] (k may be None), biases [Hq * hd] / [Hkv * hd]."""
    torch = _torch()
    _need(q, _f16(), "q"); _need(q_bias, _f16(), "q_bias"); _need(positions, torch.int64, "positions")
    if q.dim() != 3:
        raise ValueError("q must be 3-D [T, Hq, hd]")
    T, Hq, hd = q.shape
    if q_bias.numel() != Hq * hd:
        raise ValueError("q_bias must hold Hq * hd entries")
    Hkv = 0
    if k is not None:
        _need(k, _f16(), "k"); _need(k_bias, _f16(), "k_bias")
        if k.dim() != 3 or k.shape[0] != T or k.shape[2] != hd:
            raise ValueError("k must be [T, Hkv, hd]")
        Hkv = k.shape[1]
        if k_bias.numel() != Hkv * hd:
            raise ValueError("k_bias must hold Hkv * hd entries")
    if positions.numel() != T:
        raise ValueError("positions must hold T entries")
    arr, p = _inv_freq_buffer(inv_freq)
    if arr.size != hd // 2:
        raise ValueError("inv_freq must hold head_dim/2 entries")
    null = ctypes.c_void_p(0)
    _check(load_library().mi_bias_rope_neox_qk_f16(
        _ptr(q), _ptr(k) if k is not None else null, _ptr(q_bias),
        _ptr(k_bias) if k is not None else null, _ptr(positions), p, T, Hq, Hkv, hd,
        _stream(stream)), "mi_bias_rope_neox_qk_f16")
    return q, k


class KvSegment(ctypes.Structure):
    """mi_kv_segment: tokens [token_offset, token_offset + B*S) of a step in
    the [B, S] scatter layout, with int32 device block_table / seq_len /
    start_pos."""
    _fields_ = [("token_offset", _i64), ("B", _i64), ("S", _i64), ("block_table", _c_void_p),
                ("seq_len", _c_void_p), ("start_pos", _c_void_p), ("max_blocks_per_seq", _i64)]


def _rope_kv_checks(q, k, v, positions, k_cache, v_cache, layer, block_size):
    torch = _torch()
    _need(q, _f16(), "q"); _need(k, _f16(), "k"); _need(v, _f16(), "v")
    _need(positions, torch.int64, "positions")
    _need(k_cache, _f16(), "k_cache"); _need(v_cache, _f16(), "v_cache")
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise ValueError("q must be [T, Hq, hd], k and v [T, Hkv, hd]")
    T, Hq, hd = q.shape
    Hkv = k.shape[1]
    if k.shape[0] != T or k.shape[2] != hd or positions.numel() != T:
        raise ValueError("k / positions do not match q")
    if k_cache.dim() != 5 or v_cache.shape != k_cache.shape:
        raise ValueError("caches must be [L, num_blocks, Hkv, bs, hd], equal shapes")
    L, NB, Hc, bs, Dc = k_cache.shape
    if Hc != Hkv or Dc != hd or bs != block_size or not 0 <= layer < L:
        raise ValueError("cache shape does not match k / block_size / layer")
    return T, Hq, Hkv, hd, NB


def _kv_segments(segments):
    """ctypes mi_kv_segment array from segment dicts (token_offset, S, and int32
    device block_table [B, max_blocks], seq_len [B], start_pos [B])."""
    torch = _torch()
    segs = (KvSegment * max(1, len(segments)))()
    for i, g in enumerate(segments):
        bt = g["block_table"]
        for t, n in ((bt, "block_table"), (g["seq_len"], "seq_len"),
                     (g["start_pos"], "start_pos")):
            _need(t, torch.int32, n)
        if bt.dim() != 2 or g["seq_len"].numel() != bt.shape[0] or \
                g["start_pos"].numel() != bt.shape[0]:
            raise ValueError("segment: block_table [B, max_blocks], seq_len and start_pos [B]")
        segs[i].token_offset = g["token_offset"]
        segs[i].B = bt.shape[0]
        segs[i].S = g["S"]
        segs[i].block_table = _ptr(bt).value
        segs[i].seq_len = _ptr(g["seq_len"]).value
        segs[i].start_pos = _ptr(g["start_pos"]).value
        segs[i].max_blocks_per_seq = bt.shape[1]
    return segs


def rope_kv_scatter(q, k, v, positions, inv_freq, k_cache, v_cache, layer: int, block_size: int,
                    segments, q_bias=None, k_bias=None, v_bias=None, stream=None):
    """One launch: NeoX RoPE of q [T, Hq, hd] and k [T, Hkv, hd] in place and
    the rotated K and V [T, Hkv, hd] rows written into k_cache / v_cache
    [L, num_blocks, Hkv, bs, hd] for the tokens of `segments` (dicts with
    token_offset, S, block_table [B, max_blocks], seq_len [B], start_pos [B]).
    With q_bias / k_bias / v_bias (all three) the biases are added first."""
    T, Hq, Hkv, hd, NB = _rope_kv_checks(q, k, v, positions, k_cache, v_cache, layer,
                                         block_size)
    biases = (q_bias, k_bias, v_bias)
    if any(b is not None for b in biases):
        for b, n, h in zip(biases, ("q_bias", "k_bias", "v_bias"), (Hq, Hkv, Hkv)):
            if b is None:
                raise ValueError("set q_bias, k_bias and v_bias together")
            _need(b, _f16(), n)
            if b.numel() != h * hd:
                raise ValueError(f"{n} must hold {h} * head_dim entries")
    segs = _kv_segments(segments)
    arr, p = _inv_freq_buffer(inv_freq)
    if arr.size != hd // 2:
        raise ValueError("inv_freq must hold head_dim/2 entries")
    null = ctypes.c_void_p(0)
    bp = [_ptr(b) if b is not None else null for b in biases]
    _check(load_library().mi_rope_kv_scatter_f16(
        _ptr(q), _ptr(k), _ptr(v), bp[0], bp[1], bp[2], _ptr(positions), p, T, Hq, Hkv, hd,
        _ptr(k_cache), _ptr(v_cache), layer, NB, block_size, segs, len(segments),
        _stream(stream)), "mi_rope_kv_scatter_f16")
    return q, k


def qk_norm_rope_kv_scatter(q, k, v, q_weight, k_weight, positions, inv_freq, k_cache, v_cache,
                            layer: int, block_size: int, segments, eps: float = 1e-6,
                            add_one: bool = False, stream=None):
    """rope_kv_scatter with the per-head Q/K RMSNorm (q_weight / k_weight
    [hd]) applied first, as qk_norm_rope does."""
    T, Hq, Hkv, hd, NB = _rope_kv_checks(q, k, v, positions, k_cache, v_cache, layer,
                                         block_size)
    _need(q_weight, _f16(), "q_weight"); _need(k_weight, _f16(), "k_weight")
    if q_weight.numel() != hd or k_weight.numel() != hd:
        raise ValueError("q_weight / k_weight must hold head_dim entries")
    segs = _kv_segments(segments)
    arr, p = _inv_freq_buffer(inv_freq)
    if arr.size != hd // 2:
        raise ValueError("inv_freq must hold head_dim/2 entries")
    _check(load_library().mi_qk_norm_rope_kv_scatter_f16(
        _ptr(q), _ptr(k), _ptr(v), _ptr(q_weight), _ptr(k_weight), _ptr(positions), p, T, Hq,
        Hkv, hd, float(eps), int(add_one), _ptr(k_cache), _ptr(v_cache), layer, NB, block_size,
        segs, len(segments), _stream(stream)), "mi_qk_norm_rope_kv_scatter_f16")
    return q, k


def qk_rmsnorm(q, k, q_weight, k_weight, eps: float = 1e-6, add_one: bool = False, stream=None):
    """In place, one launch: per-head RMSNorm of q [T, Hq, hd] with q_weight
    and of k [T, Hkv, hd] (may be None) with k_weight [hd]."""
    _need(q, _f16(), "q"); _need(q_weight, _f16(), "q_weight")
    if q.dim() != 3:
        raise ValueError("q must be 3-D [T, Hq, hd]")
    T, Hq, hd = q.shape
    Hkv = 0
    if k is not None:
        _need(k, _f16(), "k"); _need(k_weight, _f16(), "k_weight")
        if k.dim() != 3 or k.shape[0] != T or k.shape[2] != hd:
            raise ValueError("k must be [T, Hkv, hd]")
        Hkv = k.shape[1]
    if q_weight.numel() != hd or (k is not None and k_weight.numel() != hd):
        raise ValueError("weights must hold head_dim entries")
    null = ctypes.c_void_p(0)
    _check(load_library().mi_qk_rmsnorm_f16(
        _ptr(q), _ptr(k) if k is not None else null, _ptr(q_weight),
        _ptr(k_weight) if k is not None else null, T, Hq, Hkv, hd, float(eps), int(add_one),
        _stream(stream)), "mi_qk_rmsnorm_f16")
    return q, k


def qk_norm_rope(q, k, q_weight, k_weight, positions, inv_freq, eps: float = 1e-6,
                 add_one: bool = False, stream=None):
    """In place: per-head RMSNorm of q [T, Hq, hd] / k [T, Hkv, hd] (k may be
    None) with q_weight / k_weight [hd], then NeoX RoPE at device positions."""
    torch = _torch()
    _need(q, _f16(), "q"); _need(q_weight, _f16(), "q_weight")
    _need(positions, torch.int64, "positions")
    if q.dim() != 3:
        raise ValueError("q must be 3-D [T, Hq, hd]")
    T, Hq, hd = q.shape
    if q_weight.numel() != hd:
        raise ValueError("q_weight must hold head_dim entries")
    Hkv = 0
    if k is not None:
        _need(k, _f16(), "k"); _need(k_weight, _f16(), "k_weight")
        if k.dim() != 3 or k.shape[0] != T or k.shape[2] != hd or k_weight.numel() != hd:
            raise ValueError("k must be [T, Hkv, hd] with k_weight [hd]")
        Hkv = k.shape[1]
    if positions.numel() != T:
        raise ValueError("positions must hold T entries")
    arr, p = _inv_freq_buffer(inv_freq)
    if arr.size != hd // 2:
        raise ValueError("inv_freq must hold head_dim/2 entries")
    kp = _ptr(k) if k is not None else ctypes.c_void_p(0)
    kw = _ptr(k_weight) if k is not None else ctypes.c_void_p(0)
    _check(load_library().mi_qk_norm_rope_f16(_ptr(q), kp, _ptr(q_weight), kw, _ptr(positions), p,
                                              T, Hq, Hkv, hd, eps, int(bool(add_one)),
                                              _stream(stream)), "mi_qk_norm_rope_f16")
    return q, k


# ---------------------------------------------------------------------------
# Elementwise (reference: swiglu_kernel.cuh:9, gelu_kernel.cuh:15,
# model_utils_kernel.cuh:12-29)
# ---------------------------------------------------------------------------

def _binary(fn_name, a, b, out, stream):
    _need(a, _f16(), "a"); _need(b, _f16(), "b")
    if a.numel() != b.numel():
        raise ValueError("operands must have the same number of elements")
    if out is None:
        out = _torch().empty_like(a)
    _need(out, _f16(), "out")
    if out.numel() != a.numel():
        raise ValueError("out must have the operands' size")
    _check(getattr(load_library(), fn_name)(_ptr(a), _ptr(b), _ptr(out), a.numel(),
                                            _stream(stream)), fn_name)
    return out


def swiglu(gate, up, out=None, stream=None):
    return _binary("mi_swiglu_f16", gate, up, out, stream)


def geglu(gate, up, out=None, stream=None):
    return _binary("mi_geglu_f16", gate, up, out, stream)


def gelu_tanh(x, y=None, stream=None):
    _need(x, _f16(), "x")
    if y is None:
        y = _torch().empty_like(x)
    _need(y, _f16(), "y")
    if y.numel() != x.numel():
        raise ValueError("y must have x's size")
    _check(load_library().mi_gelu_tanh_f16(_ptr(x), _ptr(y), x.numel(), _stream(stream)),
           "mi_gelu_tanh_f16")
    return y


def add_inplace(y, x, stream=None):
    _need(y, _f16(), "y"); _need(x, _f16(), "x")
    if y.numel() != x.numel():
        raise ValueError("size mismatch")
    _check(load_library().mi_add_inplace_f16(_ptr(y), _ptr(x), y.numel(), _stream(stream)),
           "mi_add_inplace_f16")
    return y


def add_bias(y, bias, M: int, N: int, batch_stride: int, stream=None):
    """y[b * batch_stride + m * N + n] += bias[n] (fp16 rounding) for
    b < batch_stride // (M * N), m < M, n < N; y is any fp16 GPU tensor."""
    _need(y, _f16(), "y"); _need(bias, _f16(), "bias")
    if bias.numel() < N:
        raise ValueError("bias must hold N entries")
    if M > 0 and N > 0 and batch_stride >= M * N:
        batches = batch_stride // (M * N)
        if y.numel() < (batches - 1) * batch_stride + M * N:
            raise ValueError("y is smaller than the batches it names")
    _check(load_library().mi_add_bias_f16(_ptr(y), _ptr(bias), M, N, batch_stride,
                                          _stream(stream)), "mi_add_bias_f16")
    return y


def mul_inplace(y, x, stream=None):
    _need(y, _f16(), "y"); _need(x, _f16(), "x")
    if y.numel() != x.numel():
        raise ValueError("size mismatch")
    _check(load_library().mi_mul_inplace_f16(_ptr(y), _ptr(x), y.numel(), _stream(stream)),
           "mi_mul_inplace_f16")
    return y


def scale_inplace(y, scale: float, stream=None):
    _need(y, _f16(), "y")
    _check(load_library().mi_scale_inplace_f16(_ptr(y), float(scale), y.numel(),
                                               _stream(stream)), "mi_scale_inplace_f16")
    return y


# ---------------------------------------------------------------------------
# Softmax (reference: launch_softmax, softmax_kernel.cuh:12)
# ---------------------------------------------------------------------------

def softmax_workspace_bytes(N: int, D: int) -> int:
    return int(load_library().mi_softmax_workspace_bytes(N, D))


def softmax(x, y=None, workspace=None, stream=None):
    """Row softmax of x [N, D].  With `workspace` (a device tensor of at least
    softmax_workspace_bytes(N, D) bytes, zero before its first use and kept
    for softmax calls only) nothing is allocated per call, and out-of-place
    split rows run in one launch.  Without it, split rows run in one launch on
    stream 0 (row records held by the library) and in two launches with a
    per-call workspace on other streams."""
    _need(x, _f16(), "x")
    if x.dim() != 2:
        raise ValueError("x must be 2-D [N, D]")
    if y is None:
        y = _torch().empty_like(x)
    _need(y, _f16(), "y")
    if y.shape != x.shape:
        raise ValueError("y must have x's shape")
    if workspace is None:
        _check(load_library().mi_softmax_f16(_ptr(x), _ptr(y), x.shape[0], x.shape[1],
                                             _stream(stream)), "mi_softmax_f16")
        return y
    if workspace.device.type != "cuda" or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous GPU tensor")
    nbytes = workspace.numel() * workspace.element_size()
    _check(load_library().mi_softmax_ws_f16(_ptr(x), _ptr(y), x.shape[0], x.shape[1],
                                            _ptr(workspace), nbytes, _stream(stream)),
           "mi_softmax_ws_f16")
    return y


def softmax_argmax_workspace_bytes(N: int, V: int) -> int:
    return int(load_library().mi_softmax_argmax_workspace_bytes(N, V))


def softmax_argmax(logits, workspace, probs=None, out=None, stream=None):
    """probs = softmax(logits) and out = greedy argmax(logits) in one pass over
    logits [N, V]; `workspace` (softmax_argmax_workspace_bytes bytes) must be
    zero before its first use and kept for this function.  Returns (probs, out)."""
    torch = _torch()
    _need(logits, _f16(), "logits")
    if logits.dim() != 2:
        raise ValueError("logits must be 2-D [N, V]")
    N, V = logits.shape
    if probs is None:
        probs = torch.empty_like(logits)
    if out is None:
        out = torch.empty(N, dtype=torch.int32, device=logits.device)
    _need(probs, _f16(), "probs"); _need(out, torch.int32, "out")
    if probs.shape != logits.shape or out.numel() != N:
        raise ValueError("probs must match logits and out hold N entries")
    nbytes = workspace.numel() * workspace.element_size()
    _check(load_library().mi_softmax_argmax_ws_f16(_ptr(logits), _ptr(probs), _ptr(out), N, V,
                                                   _ptr(workspace), nbytes, _stream(stream)),
           "mi_softmax_argmax_ws_f16")
    return probs, out


def softmax_noalloc(x, y=None, stream=None):
    """Row softmax through the allocation-free entry point
    (mi_softmax_noalloc_f16): its workspace is a device array the library
    holds, shared by every call on the GPU."""
    torch = _torch()
    _need(x, _f16(), "x")
    x2 = x if x.dim() == 2 else x.view(-1, x.shape[-1])
    N, D = x2.shape
    if y is None:
        y = torch.empty_like(x)
    _need(y, _f16(), "y")
    if y.numel() != x.numel():
        raise ValueError("y must match x")
    _check(load_library().mi_softmax_noalloc_f16(_ptr(x2), _ptr(y), N, D, _stream(stream)),
           "mi_softmax_noalloc_f16")
    return y


def softmax_test_poll_limit(limit: int) -> int:
    """Test hook: bound on one-pass softmax polling (0 forces the fallback that
    computes each row's statistics from x); returns the previous bound."""
    prev = int(load_library().mi_softmax_test_poll_limit(int(limit)))
    if prev < 0:
        raise ValueError("limit must be >= 0")
    return prev


def exchange_test_mode(mode: int) -> int:
    """Test hook: how the one-launch softmax / argmax / softmax + argmax
    kernels read their row records -- 0 (default) the XCD-local L2 copy first,
    then the device-scope mirror; 1 the mirror only.  Returns the previous mode."""
    prev = int(load_library().mi_exchange_test_mode(int(mode)))
    if prev < 0:
        raise ValueError("mode must be 0 or 1")
    return prev


# ---------------------------------------------------------------------------
# Embedding gather (reference: launch_embedding_gather, model_utils_kernel.cuh:14)
# ---------------------------------------------------------------------------

def embedding_gather(ids, table, out=None, check_range: bool = True, stream=None):
    """out[t] = table[ids[t]]; ids int64 (any shape), table [V, H]."""
    torch = _torch()
    _need(ids, torch.int64, "ids"); _need(table, _f16(), "table")
    if table.dim() != 2:
        raise ValueError("table must be 2-D [V, H]")
    V, H = table.shape
    T = ids.numel()
    if out is None:
        out = torch.empty((*ids.shape, H), dtype=torch.float16, device=table.device)
    _need(out, _f16(), "out")
    if out.numel() != T * H:
        raise ValueError("out must hold T * H elements")
    vocab = V if check_range else 0
    _check(load_library().mi_embedding_gather_f16(_ptr(ids), _ptr(table), _ptr(out), T, H, vocab,
                                                  _stream(stream)), "mi_embedding_gather_f16")
    return out


def embedding_rmsnorm(ids, table, weight, hidden=None, y=None, scale: float = 1.0,
                      eps: float = 1e-6, add_one: bool = False, check_range: bool = True,
                      stream=None):
    """hidden[t] = half(table[ids[t]] * scale), y = rmsnorm(hidden) in one pass;
    returns (hidden, y), each [*ids.shape, D]."""
    torch = _torch()
    _need(ids, torch.int64, "ids"); _need(table, _f16(), "table"); _need(weight, _f16(), "weight")
    if table.dim() != 2:
        raise ValueError("table must be 2-D [V, D]")
    V, D = table.shape
    T = ids.numel()
    if weight.numel() != D:
        raise ValueError("weight must hold D elements")
    if hidden is None:
        hidden = torch.empty((*ids.shape, D), dtype=torch.float16, device=table.device)
    if y is None:
        y = torch.empty((*ids.shape, D), dtype=torch.float16, device=table.device)
    for t, n in ((hidden, "hidden"), (y, "y")):
        _need(t, _f16(), n)
        if t.numel() != T * D:
            raise ValueError(f"{n} must hold T * D elements")
    _check(load_library().mi_embedding_rmsnorm_f16(
        _ptr(ids), _ptr(table), _ptr(hidden), _ptr(weight), _ptr(y), T, D,
        V if check_range else 0, float(scale), float(eps), int(add_one), _stream(stream)),
        "mi_embedding_rmsnorm_f16")
    return hidden, y


# ---------------------------------------------------------------------------
# Paged KV scatter (reference: launch_paged_kv_scatter, model_utils_kernel.cuh:55)
# ---------------------------------------------------------------------------

def paged_kv_scatter(src, cache, block_table, seq_len, start_pos, layer: int, block_size: int,
                     v_src=None, v_cache=None, stream=None, k_bias=None, v_bias=None):
    """Scatter src [B, S, H_kv, D] into cache [L, num_blocks, H_kv, bs, D] (and
    v_src into v_cache in the same launch when given).  k_bias / v_bias
    ([H_kv * D], with v_src): the caches receive half(src + bias)."""
    torch = _torch()
    _need(src, _f16(), "src"); _need(cache, _f16(), "cache")
    for t, n in ((block_table, "block_table"), (seq_len, "seq_len"), (start_pos, "start_pos")):
        _need(t, torch.int32, n)
    if src.dim() != 4 or cache.dim() != 5:
        raise ValueError("src must be [B, S, H_kv, D] and cache [L, num_blocks, H_kv, bs, D]")
    B, S, H, D = src.shape
    L, NB, Hc, bs, Dc = cache.shape
    if Hc != H or Dc != D or bs != block_size or not 0 <= layer < L:
        raise ValueError("cache shape does not match src / block_size / layer")
    if block_table.dim() != 2 or block_table.shape[0] != B or seq_len.numel() != B or \
            start_pos.numel() != B:
        raise ValueError("block_table must be [B, max_blocks]; seq_len, start_pos [B]")
    mb = block_table.shape[1]
    lib = load_library()
    if v_src is None:
        _check(lib.mi_paged_kv_scatter_f16(_ptr(src), _ptr(cache), _ptr(block_table), _ptr(seq_len),
                                           _ptr(start_pos), B, S, layer, NB, H, D, block_size, mb,
                                           _stream(stream)), "mi_paged_kv_scatter_f16")
    elif k_bias is not None or v_bias is not None:
        _need(v_src, _f16(), "v_src"); _need(v_cache, _f16(), "v_cache")
        if v_src.shape != src.shape or v_cache.shape != cache.shape:
            raise ValueError("v_src / v_cache must match src / cache")
        for bz, n in ((k_bias, "k_bias"), (v_bias, "v_bias")):
            if bz is not None:
                _need(bz, _f16(), n)
                if bz.numel() != H * D:
                    raise ValueError(f"{n} must hold H_kv * D entries")
        null = ctypes.c_void_p(0)
        _check(lib.mi_paged_kv_scatter_kv_bias_f16(
            _ptr(src), _ptr(v_src), _ptr(cache), _ptr(v_cache),
            _ptr(k_bias) if k_bias is not None else null,
            _ptr(v_bias) if v_bias is not None else null, _ptr(block_table), _ptr(seq_len),
            _ptr(start_pos), B, S, layer, NB, H, D, block_size, mb, _stream(stream)),
            "mi_paged_kv_scatter_kv_bias_f16")
    else:
        _need(v_src, _f16(), "v_src"); _need(v_cache, _f16(), "v_cache")
        if v_src.shape != src.shape or v_cache.shape != cache.shape:
            raise ValueError("v_src / v_cache must match src / cache")
        _check(lib.mi_paged_kv_scatter_kv_f16(_ptr(src), _ptr(v_src), _ptr(cache), _ptr(v_cache),
                                              _ptr(block_table), _ptr(seq_len), _ptr(start_pos),
                                              B, S, layer, NB, H, D, block_size, mb,
                                              _stream(stream)), "mi_paged_kv_scatter_kv_f16")
    return cache


# ---------------------------------------------------------------------------
# Greedy sampling (reference: launch_greedy_sample[_batched], sampling_kernel.cuh:17-30)
# ---------------------------------------------------------------------------

def greedy_argmax_workspace_bytes(B: int, V: int) -> int:
    return int(load_library().mi_greedy_argmax_workspace_bytes(B, V))


def greedy_argmax_test_poll_limit(limit: int) -> int:
    """Test hook: bound on one-launch argmax polling (0 forces chunk 0 to scan
    its whole row); returns the previous bound."""
    prev = int(load_library().mi_greedy_argmax_test_poll_limit(int(limit)))
    if prev < 0:
        raise ValueError("limit must be >= 0")
    return prev


def top_p_sample(logits, p: float, temperature: float, seed: int, out=None, stream=None):
    """int32 [B] top-p samples of logits [B, V] (or [V]) with the reference's
    rule (greedy above 30000 logits); row b draws with seed + b."""
    torch = _torch()
    _need(logits, _f16(), "logits")
    x = logits if logits.dim() == 2 else logits.view(1, -1)
    B, V = x.shape
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    _need(out, torch.int32, "out")
    if out.numel() != B:
        raise ValueError("out must hold B entries")
    _check(load_library().mi_top_p_sample_batched_f16(
        _ptr(x), B, V, float(p), float(temperature), int(seed) & 0xFFFFFFFFFFFFFFFF, _ptr(out),
        _stream(stream)), "mi_top_p_sample_batched_f16")
    return out


def greedy_argmax(logits, out=None, workspace=None, stream=None):
    """int32 [B] argmax of logits [B, V] (or [V]) with the reference's tie rule.
    `workspace` (greedy_argmax_workspace_bytes bytes) must be zero before its
    first use and kept for argmax calls only; split rows then run in one
    launch."""
    torch = _torch()
    _need(logits, _f16(), "logits")
    x = logits if logits.dim() == 2 else logits.view(1, -1)
    B, V = x.shape
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    _need(out, torch.int32, "out")
    if out.numel() != B:
        raise ValueError("out must hold B entries")
    lib = load_library()
    if workspace is None:
        _check(lib.mi_greedy_argmax_f16(_ptr(x), B, V, _ptr(out), _stream(stream)),
               "mi_greedy_argmax_f16")
    else:
        nbytes = workspace.numel() * workspace.element_size()
        _check(lib.mi_greedy_argmax_ws_f16(_ptr(x), B, V, _ptr(out), _ptr(workspace), nbytes,
                                           _stream(stream)), "mi_greedy_argmax_ws_f16")
    return out
