"""Test helpers: seeded inputs, host<->device copies, tolerance checks."""
import numpy as np

RTOL = 1e-3  # tests/verify/verify.py:142 (torch.allclose rtol=1e-3, atol=1e-3)
ATOL = 1e-3


def normal_f16(rng, shape, mean=0.0, std=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
            + np.float32(mean)).astype(np.float16)


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def assert_close(ours_f16, ref_f32, rtol=RTOL, atol=ATOL, what=""):
    """allclose(ours, ref) as verify.py checks it, with a useful message."""
    ours = np.asarray(ours_f16).astype(np.float32)
    ref = np.asarray(ref_f32, dtype=np.float32)
    assert ours.shape == ref.shape, f"{what}: shape {ours.shape} vs {ref.shape}"
    diff = np.abs(ours - ref)
    bad = diff > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.unravel_index(np.argmax(diff - (atol + rtol * np.abs(ref))), diff.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside rtol={rtol} atol={atol}; "
            f"worst at {i}: ours={ours[i]} ref={ref[i]} max_abs={diff.max():.3e}")


def assert_bits_equal(a, b, what=""):
    a = np.ascontiguousarray(a); b = np.ascontiguousarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    av = a.view(np.uint16 if a.dtype.itemsize == 2 else np.uint8)
    bv = b.view(np.uint16 if b.dtype.itemsize == 2 else np.uint8)
    ne = av != bv
    if ne.any():
        i = np.argwhere(ne)[0]
        raise AssertionError(f"{what}: {int(ne.sum())} of {ne.size} differ; first at {tuple(i)}: "
                             f"{a[tuple(i)]} vs {b[tuple(i)]}")


def ulp_diff(a, b):
    """Distance in fp16 units in the last place (+0 and -0 coincide)."""
    def ordered(x):
        v = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16).astype(np.int32)
        return np.where(v & 0x8000, -(v & 0x7FFF), v)
    return np.abs(ordered(a) - ordered(b))


def qk_norm_rope_ref(orc, x, w, pos, inv, eps=1e-6, add_one=False):
    """Reference composition: per-head RMSNorm written as fp16, then RoPE."""
    T, H, hd = x.shape
    n = orc.rmsnorm(x.reshape(T * H, hd), w, eps, add_one, nthreads=8)
    n16 = orc.f32_to_f16(n).reshape(T, H, hd)
    c, s = orc.rope_tables(inv, pos)
    return orc.rope_neox(n16, c, s, nthreads=8), n16


def _ulp16(v):
    return np.spacing(np.abs(np.asarray(v, np.float32)).astype(np.float16)).astype(np.float32)


def assert_norm_rope_close(ours, ref, n16, what):
    """rtol = atol = 1e-3, except at elements whose fp16 normalised input sits
    on a rounding boundary.  The oracle's statistics are exact (double sum of
    squares, double 1/sqrt); a GPU kernel -- the reference's included --
    sums in an fp32 tree and uses an fp32 reciprocal square root, so the fp16
    value it hands to the rotation can be one ulp away there.  RoPE then
    carries that ulp into an output that may be much smaller (x1 c - x2 s
    cancels).  Such elements must be rare (at most 1e-5 of the
    tensor, or 2 in a smaller one) and within one ulp of each rotated operand
    plus one output ulp."""
    ours = np.asarray(ours).astype(np.float32)
    ref = np.asarray(ref, np.float32)
    diff = np.abs(ours - ref)
    out = diff > ATOL + RTOL * np.abs(ref)
    if not out.any():
        return
    half = n16.shape[-1] // 2
    partner = np.concatenate([n16[..., half:], n16[..., :half]], axis=-1)
    bound = _ulp16(n16) + _ulp16(partner) + _ulp16(ref)
    worst = np.unravel_index(np.argmax(diff - bound), diff.shape)
    assert (diff[out] <= bound[out]).all(), (
        f"{what}: error beyond one ulp of the normalised operands at {worst}: "
        f"ours={ours[worst]} ref={ref[worst]} bound={bound[worst]}")
    # rare: at most 1 in 10^5 of the tensor, or 2 elements in a small one
    # (where one boundary case alone exceeds the fraction)
    assert out.sum() <= max(2, 1e-5 * out.size), (
        f"{what}: {int(out.sum())} of {out.size} outside tolerance")
