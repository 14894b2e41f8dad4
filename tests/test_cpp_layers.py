"""Runs the C++ host-layer parity program (tests/cpp/test_layers.cpp) and the
host check of the RoPE sin/cos header (tests/cpp/test_rope_sincos.cpp).

CPU: the host-side Tensor checks (`--cpu`).  GPU: RMSNorm / RoPE / gated
activation layers and the reference-named launchers against the oracle.
"""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
EXE = ROOT / "tests" / "cpp" / "test_layers"


def _ensure_built():
    if not EXE.exists():
        subprocess.run(["make", "-j8", "-C", str(ROOT / "mini-infer_amd")], check=True,
                       capture_output=True)
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
        subprocess.run(["make", "-C", str(ROOT / "tests" / "cpp")], check=True,
                       capture_output=True)


def test_cpp_tensor_host_side():
    _ensure_built()
    r = subprocess.run([str(EXE), "--cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout


@pytest.mark.gpu
def test_cpp_layers_on_gpu(dev):
    _ensure_built()
    print("[case] C++ layer parity program", flush=True)
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout


SINCOS = ROOT / "tests" / "cpp" / "test_rope_sincos"


def test_rope_sincos_header_on_cpu():
    """The RoPE kernels' sin/cos (rope_sincos.h) built for the host: the guard
    interval holds RN32(exact) and the table value equals half(RN32(exact))
    over a strided sweep of fp32 angles and every real RoPE angle for
    positions < 65536 (tests/cpp/test_rope_sincos.cpp)."""
    if not SINCOS.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
        subprocess.run(["make", "-C", str(ROOT / "tests" / "cpp"), "test_rope_sincos"],
                       check=True, capture_output=True)
    r = subprocess.run([str(SINCOS)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout
