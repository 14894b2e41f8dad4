"""CPU checks of the C ABI library and the Python binding (no kernel runs).

The library must load without a GPU, export every entry point that
include/mi_kernels.h declares, and reject bad arguments on the host before
touching the HIP runtime.
"""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import mi_kernels

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mi_kernels.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return mi_kernels.load_library()


def test_library_exports_every_declared_symbol(lib):
    names = declared_symbols()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), f"{n} declared in mi_kernels.h but not exported"


def test_binding_covers_header():
    names = set(declared_symbols()) - {"mi_status_string", "mi_softmax_workspace_bytes",
                                       "mi_softmax_argmax_workspace_bytes",
                                       "mi_greedy_argmax_workspace_bytes"}
    assert names == set(mi_kernels.SIGNATURES), names ^ set(mi_kernels.SIGNATURES)


def test_abi_version_and_status_strings(lib):
    m = re.search(r"#define MI_KERNELS_ABI_VERSION (\d+)", HEADER.read_text())
    assert lib.mi_abi_version() == int(m.group(1))
    assert lib.mi_status_string(0) == b"ok"
    for code in (-1, -2, -3):
        assert lib.mi_status_string(code)
    assert lib.mi_status_string(-99) == b"unknown status"


def P(v):
    return ctypes.c_void_p(v)


def test_host_side_argument_rejection(lib):
    """Every check here returns before any HIP call (fake pointers)."""
    a, b, c, r = P(0x10000), P(0x20000), P(0x30000), P(0x40000)
    # negative sizes
    assert lib.mi_rmsnorm_f16(a, b, c, -1, 64, 1e-6, 0, None) == -1
    assert lib.mi_swiglu_f16(a, b, c, -5, None) == -1
    assert lib.mi_softmax_f16(a, c, 4, -1, None) == -1
    assert lib.mi_embedding_gather_f16(a, b, c, -1, 8, 0, None) == -1
    # zero sizes are successful no-ops
    assert lib.mi_rmsnorm_f16(a, b, c, 0, 64, 1e-6, 0, None) == 0
    assert lib.mi_swiglu_f16(a, b, c, 0, None) == 0
    assert lib.mi_rope_neox_qk_f16(a, b, c, None, 0, 28, 4, 128, None) == 0
    # null pointers
    assert lib.mi_rmsnorm_f16(None, b, c, 4, 64, 1e-6, 0, None) == -1
    assert lib.mi_geglu_f16(a, None, c, 16, None) == -1
    assert lib.mi_fused_add_rmsnorm_f16(a, None, b, c, 4, 64, 1e-6, 0, None) == -1
    # overlap rules
    assert lib.mi_rmsnorm_f16(a, b, P(0x10000 + 8), 4, 64, 1e-6, 0, None) == -3
    assert lib.mi_fused_add_rmsnorm_f16(a, a, b, c, 4, 64, 1e-6, 0, None) == -3
    assert lib.mi_fused_add_rmsnorm_f16(a, c, b, c, 4, 64, 1e-6, 0, None) == -3
    assert lib.mi_swiglu_f16(a, b, P(0x10000 + 2), 64, None) == -3
    assert lib.mi_rope_neox_f16(a, b, c, P(0x10000 + 2), 1, 2, 4, 64, None) == -3
    # unsupported shapes
    inv = (ctypes.c_float * 512)()
    assert lib.mi_rope_neox_qk_f16(a, r, c, inv, 4, 1, 1, 1024, None) == -2  # head_dim > 512
    assert lib.mi_rope_neox_qk_f16(a, r, c, inv, 4, 1, 1, 7, None) == -2     # odd head_dim
    assert lib.mi_rope_neox_qk_f16(a, r, c, None, 4, 1, 1, 64, None) == -1   # no inv_freq
    assert lib.mi_rope_tables_f16(None, a, b, c, 4, 32, None) == -1


def test_size_products_that_overflow_are_rejected(lib):
    """Sizes whose byte counts would overflow int64 are argument errors,
    decided before any HIP call (fake pointers)."""
    a, b, c, d, e = (P(0x10000 * i) for i in range(1, 6))
    big = 1 << 40
    assert lib.mi_rmsnorm_f16(a, b, c, 1 << 30, big, 1e-6, 0, None) == -1
    assert lib.mi_softmax_f16(a, c, 1 << 30, big, None) == -1
    assert lib.mi_swiglu_f16(a, b, c, 1 << 62, None) == -1
    assert lib.mi_embedding_gather_f16(a, b, c, 1 << 30, big, 0, None) == -1
    assert lib.mi_add_bias_f16(a, b, big, big, big, None) == -1
    # B * S past int64 (and a layer whose + 1 would overflow)
    assert lib.mi_paged_kv_scatter_f16(a, b, c, d, e, 1 << 40, 1 << 40, 0, 8, 4, 128, 16, 4,
                                       None) == -1
    assert lib.mi_paged_kv_scatter_f16(a, b, c, d, e, 1, 1, (1 << 63) - 1, 8, 4, 128, 16, 4,
                                       None) == -1
    # a segment of the one-launch RoPE + KV scatter whose B * S would overflow
    import mi_kernels
    inv = (ctypes.c_float * 64)()
    seg = (mi_kernels.KvSegment * 1)()
    seg[0].token_offset, seg[0].B, seg[0].S = 0, 1 << 40, 1 << 40
    seg[0].block_table, seg[0].seq_len, seg[0].start_pos = 0x60000, 0x70000, 0x80000
    seg[0].max_blocks_per_seq = 4
    q, k, v, kc, vc = (P(0x1000000 * i) for i in range(1, 6))
    assert lib.mi_rope_kv_scatter_f16(q, k, v, None, None, None, P(0x90000), inv, 100, 28, 4,
                                      128, kc, vc, 0, 8, 16, seg, 1, None) == -1
    # overlapping token ranges: unsupported (the separate scatters write such a
    # token once per segment); refused before any launch
    two = (mi_kernels.KvSegment * 2)()
    for i, off in enumerate((0, 30)):
        two[i].token_offset, two[i].B, two[i].S = off, 2, 20
        two[i].block_table, two[i].seq_len, two[i].start_pos = 0x60000, 0x70000, 0x80000
        two[i].max_blocks_per_seq = 4
    assert lib.mi_rope_kv_scatter_f16(q, k, v, None, None, None, P(0x90000), inv, 100, 28, 4,
                                      128, kc, vc, 0, 8, 16, two, 2, None) == -2
    # fp16 logits at an odd address, on the nucleus and the greedy path
    assert lib.mi_top_p_sample_f16(P(0x10001), 100, 0.9, 1.0, 1, P(0x20000), None) == -1
    assert lib.mi_top_p_sample_f16(P(0x10001), 40000, 0.9, 1.0, 1, P(0x20000), None) == -1
    seg[0].B, seg[0].S = 0, 1 << 62  # an empty segment is fine; nothing launched for T = 0
    assert lib.mi_rope_kv_scatter_f16(q, k, v, None, None, None, P(0x90000), inv, 0, 28, 4,
                                      128, kc, vc, 0, 8, 16, seg, 1, None) == 0


def test_binding_validates_on_host():
    import torch
    x = torch.zeros(4, 8, dtype=torch.float16)
    w = torch.zeros(8, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        mi_kernels.rmsnorm(x, w)
    with pytest.raises(TypeError):
        mi_kernels.rmsnorm(np.zeros((4, 8)), w)


def test_product_path_has_no_oracle_dependency():
    """The shipped package must not import, link or load the oracle."""
    pkg = ROOT / "mini-infer_amd"
    files = [f for ext in ("*.py", "*.hip", "*.cpp", "*.h", "Makefile") for f in pkg.rglob(ext)]
    assert files
    for f in files:
        text = f.read_text()
        for needle in ("import oracle", "libmi_oracle", "mi_oracle.h", "mio_"):
            assert needle not in text, f"{f} references the oracle ({needle})"


def test_softmax_workspace_sizes(lib):
    lib.mi_softmax_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int64]
    lib.mi_softmax_workspace_bytes.restype = ctypes.c_int64
    # Row records: 512 rows x 4224 B (128 B header, two sets of 64 slot pairs
    # and their mirror).
    # 64 rows of 152064: the records, then for the two-launch form chunks of
    # one 4096-element tile (the whole number of tiles nearest 152064 / 32),
    # 38 per row, one (max, sum) pair each
    rec = 512 * 4224
    assert lib.mi_softmax_workspace_bytes(64, 152064) == rec + 64 * 38 * 8
    # 512 rows or more (256 or more up to 65536) longer than 32768: the
    # records only (persistent one-launch form; a workgroup per row when a
    # call cannot use them)
    assert lib.mi_softmax_workspace_bytes(512, 152064) == rec
    assert lib.mi_softmax_workspace_bytes(4096, 32769) == rec
    assert lib.mi_softmax_workspace_bytes(256, 65536) == rec
    assert lib.mi_softmax_workspace_bytes(512, 32768) == 0
    assert lib.mi_softmax_workspace_bytes(256, 32768) == 0
    assert lib.mi_softmax_workspace_bytes(512, 600000) == 0  # more than 64 chunks per row
    assert lib.mi_softmax_workspace_bytes(57344, 512) == 0
    assert lib.mi_softmax_workspace_bytes(8, 1024) == 0
    assert lib.mi_softmax_workspace_bytes(0, 5) == 0
    assert 0 < lib.mi_softmax_workspace_bytes(511, 10**6) <= rec + 256 * 1024


def test_argmax_workspace_sizes(lib):
    lib.mi_greedy_argmax_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int64]
    lib.mi_greedy_argmax_workspace_bytes.restype = ctypes.c_int64
    # split rows: the one-launch records (512 rows x 2176 B: 128 B header, 64
    # slots and their mirror), then one key per
    # chunk for the two-launch form (4096- or 2048-element chunks)
    assert lib.mi_greedy_argmax_workspace_bytes(64, 152064) == 512 * 2176 + 64 * 38 * 8
    assert lib.mi_greedy_argmax_workspace_bytes(1, 152064) == 512 * 2176 + 75 * 8
    assert lib.mi_greedy_argmax_workspace_bytes(512, 152064) == 0           # one workgroup per row
    assert lib.mi_greedy_argmax_workspace_bytes(64, 4096) == 0
    assert 0 < lib.mi_greedy_argmax_workspace_bytes(511, 10**6) <= 512 * 2176 + 256 * 1024
