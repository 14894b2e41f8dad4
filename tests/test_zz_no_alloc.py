"""GPU check of the allocation-free softmax entry point (mi_softmax_noalloc_f16):
through the C ABI it gives the same bits as mi_softmax_ws_f16 (the entry
point whose kernels it shares) on two calls in a row, the second smaller,
for each plan that uses the library's device array -- one-launch split rows
(row records), the two-launch form (in place: (max, sum) pairs) and the
persistent many-row form -- and for a shape that needs no workspace.  Run
after the other tests, and alone in a fresh process (the array is looked up
on the device's first call and is zero from the library's load); a fresh
process whose first call is captured in a graph is checked as well."""
import numpy as np
import pytest

from helpers import assert_bits_equal, normal_f16, to_dev, to_host

pytestmark = pytest.mark.gpu


def _ws_softmax(mk, x, inplace):
    """The existing entry point with a fresh zeroed workspace."""
    import torch
    N, D = x.shape
    ws = torch.zeros(max(16, mk.softmax_workspace_bytes(N, D)), dtype=torch.uint8,
                     device=x.device)
    xd = x.clone()
    return to_host(mk.softmax(xd, y=xd if inplace else None, workspace=ws))


@pytest.mark.parametrize("shapes,inplace", [
    (((64, 152064), (8, 40000)), False),   # one launch, row records
    (((64, 152064), (3, 65536)), True),    # two launches, (max, sum) pairs
    (((1024, 65600), (600, 40000)), False),  # persistent many rows, several rounds
    (((4096, 512), (7, 1000)), False),     # whole rows in registers, no workspace
])
def test_noalloc_matches_workspace_entry(mk, dev, shapes, inplace):
    print(f"[case] softmax noalloc {shapes} inplace={inplace}", flush=True)
    rng = np.random.default_rng(sum(n * d for n, d in shapes) % 10007)
    for N, D in shapes:  # two calls in a row, the second smaller
        x = normal_f16(rng, (N, D), 0, 4)
        x[0, :: max(1, D // 7)] = -np.inf
        xd = to_dev(x, dev)
        ref = _ws_softmax(mk, xd, inplace)
        if inplace:
            y = mk.softmax_noalloc(xd, y=xd)
        else:
            y = mk.softmax_noalloc(xd)
            assert_bits_equal(to_host(xd), x, what="input untouched")
        assert_bits_equal(to_host(y), ref, what=f"noalloc vs ws entry [{N},{D}]")


def test_noalloc_argument_errors(mk):
    lib = mk.load_library()
    assert lib.mi_softmax_noalloc_f16(None, None, -1, 5, None) == -1
    assert lib.mi_softmax_noalloc_f16(None, None, 4, 5, None) == -1
    assert lib.mi_softmax_noalloc_f16(None, None, 0, 5, None) == 0


_CAPTURED_FIRST = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
import mi_kernels as mk
mk.load_library()
dev = torch.device("cuda:0")
rng = np.random.default_rng(5)
x = torch.from_numpy((rng.standard_normal((64, 152064), dtype=np.float32) * 4).astype(np.float16)).to(dev)
ws = torch.zeros(mk.softmax_workspace_bytes(64, 152064), dtype=torch.uint8, device=dev)
y_graph = torch.empty_like(x)
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        mk.softmax_noalloc(x, y=y_graph)   # the process's first call: captured
torch.cuda.current_stream().wait_stream(side)
torch.cuda.synchronize()
ref = mk.softmax(x.clone(), workspace=ws)
torch.cuda.synchronize()
ref_bits = ref.cpu().numpy().view(np.uint16)
bad = 0
for rep in range(3):
    y_graph.zero_()
    graph.replay()
    torch.cuda.synchronize()
    bad += int((y_graph.cpu().numpy().view(np.uint16) != ref_bits).sum())
    y_eager = mk.softmax_noalloc(x)  # eager calls between the replays
    torch.cuda.synchronize()
    bad += int((y_eager.cpu().numpy().view(np.uint16) != ref_bits).sum())
print("MISMATCHES", bad, flush=True)
"""


def test_noalloc_first_call_captured(dev):
    """In a fresh process, the first allocation-free call is captured in a HIP
    graph (nothing but the softmax is recorded: the array is zero from load);
    three replays, each followed by an eager call, all equal the workspace
    entry point bit for bit."""
    import subprocess
    import sys
    from pathlib import Path
    print("[case] softmax noalloc: first call captured, replays + eager calls", flush=True)
    pkg = str(Path(__file__).resolve().parent.parent / "mini-infer_amd")
    r = subprocess.run([sys.executable, "-c", _CAPTURED_FIRST, pkg], capture_output=True,
                       text=True, timeout=110)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "MISMATCHES 0" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
