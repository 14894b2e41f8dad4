"""GPU check of the allocation-free softmax entry point (mi_softmax_noalloc_f16):
through the C ABI it gives the same bits as mi_softmax_ws_f16 (the entry
point whose kernels it shares) on two calls in a row, the second smaller,
for each plan that uses the library's device array -- one-launch split rows
(row records), the two-launch form (in place: (max, sum) pairs) and the
persistent many-row form -- and for a shape that needs no workspace.  Run
after the other tests, and alone in a fresh process (the array is looked up
and zeroed on the device's first call)."""
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
