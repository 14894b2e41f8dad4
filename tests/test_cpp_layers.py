"""Runs the C++ host-layer parity program (tests/cpp/test_layers.cpp).

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
