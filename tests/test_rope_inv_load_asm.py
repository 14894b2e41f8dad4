"""CPU build check of the RoPE kernels' inverse-frequency load (rope.hip).

The kernels read each lane's inverse frequency from the kernel-argument block
with an inline-asm vector load issued ahead of the token data, then wait with
an inline-asm `s_waitcnt vmcnt(N)` that lets the N data loads issued after it
stay in flight.  Vector loads complete in issue order, so that wait is only
right if at least N vector loads are issued, unconditionally, between the
asm load and the asm wait.  A compiler that reordered or predicated those
loads would make the wait pass too early and the rotation read a stale
register, with no error: this test checks the built code for it.
"""
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "mini-infer_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         f"-I{ROOT / 'include'}", f"-I{CSRC}", f"-I{ROOT / 'mini-infer_amd' / 'host'}"]
VLOAD = ("global_load", "buffer_load", "flat_load")


def _functions(asm: str):
    for part in re.split(r"\n(?=_Z\S+:)", asm):
        m = re.match(r"(_Z\S+):", part)
        if m:
            yield m.group(1), [ln.strip() for ln in part.splitlines()]


def _checks(lines):
    """(loads issued after each asm inverse-frequency load up to its asm
    wait, the wait's N, vector loads under a branch in between)."""
    out = []
    for i, ln in enumerate(lines):
        if ln != ";;#ASMSTART" or i + 1 >= len(lines) or not lines[i + 1].startswith("global_load_dword "):
            continue
        loads, wait, skipped, target = 0, None, 0, None
        for k in range(i + 3, len(lines)):
            t = lines[k]
            if t == ";;#ASMSTART" and lines[k + 1].startswith("s_waitcnt vmcnt"):
                wait = int(re.search(r"vmcnt\((\d+)\)", lines[k + 1]).group(1))
                break
            if target and t.startswith(target + ":"):
                target = None
            m = re.match(r"s_cbranch_\w+ (\.LBB\w+)", t)
            if m and target is None:
                target = m.group(1)
            if t.startswith(VLOAD):
                loads += 1
                if target:
                    skipped += 1
        out.append((loads, wait, skipped))
    return out


def test_inverse_frequency_waits_cover_the_data_loads(tmp_path):
    out = tmp_path / "rope.s"
    subprocess.run([HIPCC, *FLAGS, str(CSRC / "rope.hip"), "-o", str(out)], check=True,
                   capture_output=True)
    seen = 0
    for name, lines in _functions(out.read_text()):
        for loads, wait, skipped in _checks(lines):
            seen += 1
            assert wait is not None, f"{name}: no asm wait after the inverse-frequency load"
            assert skipped == 0, f"{name}: {skipped} vector loads under a branch before the wait"
            assert loads >= wait, f"{name}: {loads} loads after the inverse-frequency load, vmcnt({wait})"
    # the rows kernel and the one-token kernels (plain, bias, norm) all use it
    assert seen >= 40, seen
