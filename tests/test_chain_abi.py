"""CPU checks of the decoder-chain ABI (include/mi_chain.h, libmini_infer.so):
the ctypes mirror of mi_chain_desc matches the C layout field for field, the
library exports what the header declares, and a descriptor that misses a
buffer a requested stage needs is refused on the host, before any HIP call.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

import mi_chain

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mi_chain.h"


@pytest.fixture(scope="module")
def lib():
    return mi_chain.load_library()


def test_exports_every_declared_symbol(lib):
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))
    assert names == ["mi_decoder_chain_last_error", "mi_decoder_chain_run"]
    for n in names:
        assert hasattr(lib, n)


def test_stage_numbers_match_header():
    text = HEADER.read_text()
    for name in ("EMBED", "INPUT_NORM", "QK_ROPE", "KV_SCATTER", "POST_ATTN_NORM", "ACTIVATION",
                 "FINAL_NORM", "SAMPLE"):
        m = re.search(rf"MI_CHAIN_{name} = (\d+)", text)
        assert m and int(m.group(1)) == getattr(mi_chain.Stage, name), name


def test_struct_layout_matches_c(tmp_path):
    """Offsets and sizes of every field, from a C program compiled against
    the header, against the ctypes Structures."""
    fields = [n for n, _ in mi_chain.ChainDesc._fields_]
    seg = [n for n, _ in mi_chain.KvSegment._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", '#include "mi_chain.h"', "int main(void) {",
           'printf("desc %zu\\n", sizeof(mi_chain_desc));',
           'printf("seg %zu\\n", sizeof(mi_chain_kv_segment));']
    src += [f'printf("{n} %zu\\n", offsetof(mi_chain_desc, {n}));' for n in fields]
    src += [f'printf("seg.{n} %zu\\n", offsetof(mi_chain_kv_segment, {n}));' for n in seg]
    src += ["return 0; }"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(c), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                      check=True).stdout.splitlines())
    assert int(out["desc"]) == ctypes.sizeof(mi_chain.ChainDesc)
    assert int(out["seg"]) == ctypes.sizeof(mi_chain.KvSegment)
    for n in fields:
        assert int(out[n]) == getattr(mi_chain.ChainDesc, n).offset, n
    for n in seg:
        assert int(out[f"seg.{n}"]) == getattr(mi_chain.KvSegment, n).offset, n


def _desc(**kw):
    d = mi_chain.ChainDesc()
    base = dict(mi_chain.QWEN25_7B, T=4, logit_rows=1, layer=0, num_layers=1, num_blocks=4,
                block_size=16)
    base.update(kw)
    for k, v in base.items():
        setattr(d, k, v)
    fake = 0x100000
    for n in ("embed", "ids", "hidden"):
        setattr(d, n, fake)
    return d


def test_refuses_missing_buffers_on_host(lib):
    run = lib.mi_decoder_chain_run
    assert run(None, 8, None) == -1
    assert b"null" in lib.mi_decoder_chain_last_error()
    d = _desc()
    for stage, msg in ((0, b"last_stage"), (9, b"last_stage"), (2, b"input norm"),
                       (3, b"input norm")):
        assert run(ctypes.byref(d), stage, None) == -1
        assert msg in lib.mi_decoder_chain_last_error(), lib.mi_decoder_chain_last_error()
    d2 = _desc(act=2)
    assert run(ctypes.byref(d2), 1, None) == -1
    assert b"act" in lib.mi_decoder_chain_last_error()
    d3 = _desc(head_dim=127)
    assert run(ctypes.byref(d3), 1, None) == -1
    d4 = _desc(hidden_size=0)
    assert run(ctypes.byref(d4), 1, None) == -1


def test_refuses_partial_qkv_bias(lib):
    """Qwen2's QKV bias comes as q_bias, k_bias and v_bias together."""
    d = _desc()
    d.q_bias = 0x200000
    assert lib.mi_decoder_chain_run(ctypes.byref(d), 1, None) == -1
    assert b"qkv bias" in lib.mi_decoder_chain_last_error(), lib.mi_decoder_chain_last_error()
