"""CPU build check of the write-through store (st8_stream_wt in
mini-infer_amd/csrc/mi_device.h): its inline asm hides the store from the
compiler's hazard pass, so the asm must carry the wait states a wide store
needs before VALU code may overwrite its data registers.

For every MI_WT_FORM a small kernel that stores and then overwrites the
stored registers is compiled for gfx950; each inline-asm block must be
exactly the form's store followed by `s_nop 1`.  The default build of the
kernels that use the store (rope.hip, rmsnorm.hip) is checked the same way.
"""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "mini-infer_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"
FORMS = {0: "nt sc1", 1: "sc1", 2: "sc0 sc1", 3: "sc0 sc1 nt", 4: "sc0 nt"}
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         f"-I{ROOT / 'include'}", f"-I{CSRC}"]

PROBE = """
#include "mi_device.h"
__global__ void probe(mi::half_t* p, float s) {
    mi::h8 v;
    for (int k = 0; k < 8; ++k) v[k] = (mi::half_t)(s * (threadIdx.x + k));
    mi::st8_stream_wt(p + threadIdx.x * 8, v);
    for (int k = 0; k < 8; ++k) v[k] = (mi::half_t)(s + k);  // reuses the registers
    mi::st8_stream_wt(p + 4096 + threadIdx.x * 8, v);
}
"""


def _asm_blocks(asm: str):
    """The non-empty inline-asm blocks (the empty ones are fp32_rounded's
    register pins)."""
    blocks = [b.strip() for b in re.findall(r";;#ASMSTART\n(.*?);;#ASMEND", asm, flags=re.S)]
    return [b for b in blocks if b]


def _check(blocks, bits):
    assert blocks, "no inline-asm store found"
    for b in blocks:
        lines = [ln.strip() for ln in b.splitlines() if ln.strip()]
        assert len(lines) == 2, b
        assert re.fullmatch(r"global_store_dwordx4 v\[\d+:\d+\], v\[\d+:\d+\], off " + bits,
                            lines[0]), lines[0]
        assert lines[1] == "s_nop 1", b


@pytest.mark.parametrize("form", sorted(FORMS))
def test_every_form_carries_its_wait_states(tmp_path, form):
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    out = tmp_path / "probe.s"
    subprocess.run([HIPCC, *FLAGS, f"-DMI_WT_FORM={form}", str(src), "-o", str(out)], check=True,
                   capture_output=True)
    _check(_asm_blocks(out.read_text()), FORMS[form])


def test_other_forms_do_not_build(tmp_path):
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    r = subprocess.run([HIPCC, *FLAGS, "-DMI_WT_FORM=5", str(src), "-o", str(tmp_path / "x.s")],
                       capture_output=True, text=True)
    assert r.returncode != 0 and "MI_WT_FORM must be 0-4" in r.stderr


@pytest.mark.parametrize("name", ["rope.hip", "rmsnorm.hip"])
def test_library_build_stores(tmp_path, name):
    out = tmp_path / "k.s"
    subprocess.run([HIPCC, *FLAGS, str(CSRC / name), "-o", str(out)], check=True,
                   capture_output=True)
    blocks = _asm_blocks(out.read_text())
    # rope.hip's other inline asm: the inverse-frequency load from the
    # kernel-argument block and the explicit waits for it
    other = [b for b in blocks if "global_store" not in b]
    for b in other:
        assert re.fullmatch(r"global_load_dword v\d+, v\[\d+:\d+\], off|s_waitcnt vmcnt\(\d+\)", b), b
    _check([b for b in blocks if "global_store" in b], FORMS[0])
