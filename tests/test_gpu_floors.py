"""The benchmark's calibration streams (mini-infer_amd/bench/floors.hip) move
the bytes they claim to: every form of the copy reproduces its source, the
in-place stream changes every word and a second call restores it, and the
read stream leaves its never-taken store untouched.  A floor that skipped
bytes would flatter every kernel set beside it."""
import pytest
import torch

import bench

pytestmark = pytest.mark.gpu

NBYTES = 3 * (1 << 20) + 4096  # not a multiple of any tile


@pytest.fixture(scope="module")
def lib():
    return bench.floors_lib()


def _forms():
    return bench.FLOOR_FORMS


@pytest.mark.parametrize("form", _forms(), ids=lambda f: "v%d_p%d_pl%d_s%d" % f)
def test_copy_and_inplace_forms(lib, form):
    vpl, pers, plain, serial = form
    code = vpl | (16 if pers else 0) | (32 if plain else 0) | (64 if serial else 0)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(vpl * 8 + pers * 4 + plain * 2 + serial)
    src = torch.randint(0, 256, (NBYTES,), dtype=torch.uint8, device=dev, generator=g)
    dst = torch.zeros_like(src)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.mi_floor_copy(src.data_ptr(), dst.data_ptr(), NBYTES, code, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(src, dst)

    buf = src.clone()
    assert lib.mi_floor_inplace(buf.data_ptr(), NBYTES, code, st) == 0
    torch.cuda.synchronize()
    words = buf.view(torch.int32) ^ src.view(torch.int32)
    assert bool((words == 0x3C003C00).all())
    assert lib.mi_floor_inplace(buf.data_ptr(), NBYTES, code, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(buf, src)


@pytest.mark.parametrize("vpl", [1, 2, 4, 8])
@pytest.mark.parametrize("pers", [0, 1])
def test_read_form_never_stores(lib, vpl, pers):
    dev = torch.device("cuda:0")
    src = torch.full((NBYTES,), 1, dtype=torch.uint8, device=dev)
    sink = torch.full((1 << 20,), 7, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    code = vpl | (16 if pers else 0)
    assert lib.mi_floor_read(src.data_ptr(), NBYTES, code, sink.data_ptr(), sink.numel(), st) == 0
    torch.cuda.synchronize()
    assert bool((sink == 7).all())


def test_rejects_bad_arguments(lib):
    dev = torch.device("cuda:0")
    a = torch.zeros(64, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.mi_floor_copy(a.data_ptr(), a.data_ptr() + 32, 24, 1, st) == -1  # not 16-byte sized
    assert lib.mi_floor_copy(a.data_ptr() + 8, a.data_ptr() + 32, 16, 1, st) == -1  # misaligned
    assert lib.mi_floor_copy(a.data_ptr(), a.data_ptr() + 32, 16, 3, st) == -1  # vpl 3
