#!/usr/bin/env python3
"""Benchmark of the MI355X layer kernels (one GPU).

Headline (the JSON line's `value`): achieved HBM bandwidth of the fused
residual-add + RMSNorm kernel at Qwen2.5-7B prefill, x / residual fp16
[8192, 3584] (Qwen2.5-7B prefill).  One step = one launch over that batch;
inputs are resident in HBM before the timed region.  Buffer sets are rotated
so the working set of consecutive launches exceeds the 256 MB Infinity Cache
and every launch streams from HBM.

Also reported, under "kernels": every benchmark workload, each kernel timed the
same way (average over back-to-back launches with HIP events on the launch
stream), as algorithmic GB/s, fraction of the 8 TB/s HBM peak and tokens/s.

`cpu_baseline` times the CPU oracle (a C restatement of the reference's
test arithmetic, oracle/libmi_oracle.so) on the host, on a bounded sample of
the same workload.  The oracle is the checker, never the thing measured on
the GPU.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-kernels] [--no-cpu] [--no-chain]
       [--shapes]
"""
import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "mini-infer_amd"))

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
MALL_BYTES = 256 << 20     # Infinity Cache
METRIC = "achieved HBM GB/s (% of 8 TB/s peak) per layer kernel at Qwen2.5-7B shapes"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def rotations(set_bytes, min_sets=2, max_sets=64):
    """Enough buffer sets that a full rotation is >= 3x the Infinity Cache."""
    return int(min(max_sets, max(min_sets, math.ceil(3 * MALL_BYTES / max(set_bytes, 1)))))


EAGER = False  # --eager: plain launches (for counter collection), no graph
KERNEL_ITERS = 100  # launches per kernel-table row (at least)
CHAIN_ITERS = 40    # decoder-chain steps per chain row (at least)


def time_launches(launch, nsets, iters, warmup):
    """Average seconds per launch over `iters` back-to-back launches cycling
    through `nsets` buffer sets.  The launches are captured into one HIP
    graph and replayed, so host-side launch cost (Python, ctypes) is not in
    the figure; events on the replay stream bracket the timed replay."""
    import torch
    if EAGER:
        for i in range(warmup):
            launch(i % nsets)
        torch.cuda.synchronize()
        s = torch.cuda.current_stream()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(s)
        for i in range(iters):
            launch(i % nsets)
        t1.record(s)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) * 1e-3 / iters
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(warmup):
            launch(i % nsets)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            launch(i % nsets)
    graph.replay()  # untimed replay: first-replay setup cost
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(s)
    graph.replay()
    t1.record(s)
    torch.cuda.synchronize()
    del graph
    return t0.elapsed_time(t1) * 1e-3 / iters


def copy_calibration(dev, iters=50):
    """HBM bandwidth of a plain device-to-device copy of 1 GiB (read + write
    counted), for context: the practical ceiling of a streaming kernel."""
    import torch
    n = 1 << 29
    a = torch.empty(n, dtype=torch.float16, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    sec = time_launches(lambda i: b.copy_(a), 1, iters, 5)
    del a, b
    return 2 * n * 2 / sec / 1e9


def randn16(shape, gen, dev, mean=0.0, std=1.0):
    import torch
    return (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32) * std + mean).half()


# ---------------------------------------------------------------------------
# Floors: calibration streams that move the same bytes and do nothing else
# (mini-infer_amd/bench/floors.hip -> libmi_floors.so), timed like the
# kernels (graph replay, buffers rotated past the Infinity Cache).  Each floor
# is the fastest of a few plain forms (16-byte vectors per lane per step
# 1/2/4/8, one workgroup per tile or a resident grid-stride grid,
# non-temporal or plain loads, stores issued back to back or each waiting for
# the one before it -- the latter is faster at 40 MB), so it is the time a
# no-work kernel of this library's style needs for those bytes.
# ---------------------------------------------------------------------------

FLOOR_FORMS = ([(v, p, n, 0) for v in (1, 2, 4, 8) for p in (0, 1) for n in (0, 1)] +
               [(v, p, 0, 1) for v in (1, 2, 4, 8) for p in (0, 1)])
_FLOORS_LIB = None
_FLOOR = {}


def floors_lib():
    import ctypes
    global _FLOORS_LIB
    if _FLOORS_LIB is None:
        path = ROOT / "mini-infer_amd" / "libmi_floors.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run `make -C mini-infer_amd`")
        lib = ctypes.CDLL(str(path))
        i64, vp, ci = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
        lib.mi_floor_copy.argtypes = [vp, vp, i64, ci, vp]
        lib.mi_floor_inplace.argtypes = [vp, i64, ci, vp]
        lib.mi_floor_read.argtypes = [vp, i64, ci, vp, i64, vp]
        lib.mi_floor_empty.argtypes = [vp]
        lib.mi_floor_rope_inplace.argtypes = [vp, vp, i64, i64, i64, i64, ci, vp]
        lib.mi_floor_gather2.argtypes = [vp, vp, vp, vp, i64, i64, vp]
        lib.mi_floor_read_rows.argtypes = [vp, i64, i64, ci, vp, i64, vp]
        _FLOORS_LIB = lib
    return _FLOORS_LIB


def _floor_launcher(kind, bufs, sink, nbytes, vpl, persistent, plain, serial):
    import torch
    lib = floors_lib()
    form = vpl | (16 if persistent else 0) | (32 if plain else 0) | (64 if serial else 0)

    def go(i):
        st = torch.cuda.current_stream().cuda_stream
        if kind == "copy":
            rc = lib.mi_floor_copy(bufs[i][0].data_ptr(), bufs[i][1].data_ptr(), nbytes, form, st)
        elif kind == "inplace":
            rc = lib.mi_floor_inplace(bufs[i][0].data_ptr(), nbytes, form, st)
        else:
            rc = lib.mi_floor_read(bufs[i][0].data_ptr(), nbytes, form, sink.data_ptr(),
                                   sink.numel(), st)
        if rc != 0:
            raise RuntimeError(f"floor {kind} failed: {rc}")
    return go


def floor_time(dev, kind, nbytes, iters=40, warmup=5, forms=None):
    """Fastest time of the `kind` stream ("copy": read nbytes + write nbytes
    elsewhere; "inplace": read and rewrite nbytes; "read": read nbytes) over
    FLOOR_FORMS; returns (seconds, {form: seconds})."""
    import torch
    nbytes = max(16, (int(nbytes) + 15) // 16 * 16)
    key = (kind, nbytes)
    if key in _FLOOR and forms is None:
        return _FLOOR[key]
    nb = nbytes // 2
    ns = rotations(2 * nbytes if kind == "copy" else nbytes)
    bufs = [(torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1),
             torch.empty(nbytes, dtype=torch.uint8, device=dev) if kind == "copy" else None)
            for _ in range(ns)]
    sink = torch.zeros(1 << 20, dtype=torch.int32, device=dev)
    per = {}
    for vpl, pers, plain, serial in (forms or FLOOR_FORMS):
        if serial and kind == "read":
            continue  # no stores
        per[(vpl, pers, plain, serial)] = time_launches(
            _floor_launcher(kind, bufs, sink, nbytes, vpl, pers, plain, serial), ns, iters, warmup)
    del bufs, nb
    best = min(per.values())
    if forms is None:
        _FLOOR[key] = (best, per)
    return best, per


def rope_floor_time(dev, T, Hq, Hkv, hd, form, iters=100, warmup=10):
    """The in-place RoPE access pattern with no arithmetic (mi_floor_rope_inplace):
    form 32 = the contiguous-row kernel's (lane j on vectors j, j + 256 of a
    token's [Q | K] row, its tokens per workgroup, paced stores), 1 = one token
    per workgroup, lane (head, slice) on both half-head vectors, write-through
    stores (the one-token kernel's)."""
    import torch
    lib = floors_lib()
    ns = rotations(T * (Hq + Hkv) * hd * 2)
    bufs = [(torch.zeros((T, Hq, hd), dtype=torch.float16, device=dev),
             torch.zeros((T, Hkv, hd), dtype=torch.float16, device=dev)) for _ in range(ns)]

    def go(i):
        rc = lib.mi_floor_rope_inplace(bufs[i][0].data_ptr(), bufs[i][1].data_ptr(), T, Hq, Hkv,
                                       hd, form, torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"rope floor failed: {rc}")
    sec = time_launches(go, ns, iters, warmup)
    del bufs
    return sec


def empty_launch_time(iters=400, warmup=20):
    """Average time per launch of an empty one-workgroup kernel, replayed
    back to back like the kernel rows: the launch floor of a tiny kernel."""
    import torch
    lib = floors_lib()

    def go(i):
        if lib.mi_floor_empty(torch.cuda.current_stream().cuda_stream) != 0:
            raise RuntimeError("empty launch failed")
    return time_launches(go, 1, iters, warmup)


# Which floors apply to a kernel row: (read bytes, written bytes) -> the
# out-of-place copy and the in-place stream of half the row's bytes each
# (every row), and the read stream for rows that write next to nothing.
def attach_floors(dev, row, read_only=False):
    half = row["bytes"] // 2
    oop, _ = floor_time(dev, "copy", half)
    inp, _ = floor_time(dev, "inplace", half)
    row["oop_floor_us"] = round(oop * 1e6, 3)
    row["inplace_floor_us"] = round(inp * 1e6, 3)
    if read_only:
        rd, _ = floor_time(dev, "read", row["bytes"])
        row["read_floor_us"] = round(rd * 1e6, 3)
        row["frac_of_floor"] = round(rd / (row["us"] * 1e-6), 4)
        row["floor_kind"] = "read"
    else:
        kind = row.get("floor_kind", "copy")
        f = inp if kind == "inplace" else oop
        row["frac_of_floor"] = round(f / (row["us"] * 1e-6), 4)
        row["floor_kind"] = kind


def floor_sweep(dev, sizes_mb=(8, 20, 40, 67, 100, 174, 235, 465)):
    """--floors: every form of every stream at a range of sizes (us and % of
    HBM peak of the bytes moved), to compare the forms with each other."""
    rows = []
    for mb in sizes_mb:
        nbytes = int(mb * 1e6) // 2 // 16 * 16
        for kind in ("copy", "inplace", "read"):
            moved = nbytes if kind == "read" else 2 * nbytes
            n = moved if kind == "read" else nbytes
            _, per = floor_time(dev, kind, n, forms=FLOOR_FORMS)
            for (v, p, pl, se), sec in per.items():
                rows.append({"kind": kind, "moved_bytes": moved, "vpl": v, "persistent": p,
                             "plain_loads": pl, "serial_stores": se, "us": round(sec * 1e6, 3),
                             "frac": round(moved / sec / HBM_PEAK, 4)})
                log(f"[floors] {kind:<8} {moved / 1e6:8.1f} MB vpl={v} persistent={p} "
                    f"plain_loads={pl} serial_stores={se} {sec * 1e6:9.2f} us "
                    f"{100 * moved / sec / HBM_PEAK:6.1f}%")
    return rows


def report(name, cfg, nbytes, seconds, tokens, floor_kind=None):
    r = {
        "kernel": name,
        "config": cfg,
        "bytes": int(nbytes),
        "us": round(seconds * 1e6, 3),
        "GBps": round(nbytes / seconds / 1e9, 1),
        "frac": round(nbytes / seconds / HBM_PEAK, 4),
        "tokens_per_s": round(tokens / seconds, 1),
    }
    if floor_kind:
        r["floor_kind"] = floor_kind
    return r


# ---------------------------------------------------------------------------
# Headline: fused residual-add + RMSNorm [8192, 3584]
# ---------------------------------------------------------------------------

def fused_sets(mk, dev, gen, T, D, nsets):
    w = randn16((D,), gen, dev, 1.0, 0.1)
    sets = [(randn16((T, D), gen, dev), randn16((T, D), gen, dev),
             __import__("torch").empty((T, D), dtype=__import__("torch").float16, device=dev))
            for _ in range(nsets)]
    return w, sets


def headline(mk, dev, steps, warmup):
    import torch
    gen = torch.Generator(device=dev).manual_seed(0)
    T, D = 8192, 3584
    nbytes = 4 * T * D * 2 + D * 2
    nsets = rotations(3 * T * D * 2)
    w, sets = fused_sets(mk, dev, gen, T, D, nsets)

    def launch(i):
        x, r, y = sets[i]
        mk.fused_add_rmsnorm(x, r, w, y=y, eps=1e-6)

    sec = time_launches(launch, nsets, steps, warmup)
    return T, D, nbytes, sec


# ---------------------------------------------------------------------------
# Every benchmark workload
# ---------------------------------------------------------------------------

def config3_positions(gen_np, total, nseq, max_start):
    import numpy as np
    cuts = np.sort(gen_np.choice(np.arange(1, total), nseq - 1, replace=False))
    lengths = np.diff(np.concatenate([[0], cuts, [total]]))
    starts = gen_np.integers(0, max_start, nseq)
    return np.concatenate([s + np.arange(n) for s, n in zip(starts, lengths)]).astype(np.int64)


def chain_positions(gen_np):
    """64 decode tokens at random offsets, then two 3000-token prefills."""
    import numpy as np
    dec = gen_np.integers(0, 28000, 64)
    pre = [s + np.arange(3000) for s in gen_np.integers(0, 28000, 2)]
    return np.concatenate([dec] + pre).astype(np.int64)


def _floor_ok(rc):
    if rc != 0:
        raise RuntimeError(f"floor kernel failed: {rc}")


def attach_rope_floors(dev, row, T, Hq, Hkv, hd):
    """RoPE rows: the time of their own access pattern with no arithmetic."""
    row["rope_floor_us"] = round(rope_floor_time(dev, T, Hq, Hkv, hd, 32) * 1e6, 3)
    row["rope_floor_one_token_us"] = round(rope_floor_time(dev, T, Hq, Hkv, hd, 1) * 1e6, 3)
    row["frac_of_rope_floor"] = round(row["rope_floor_us"] / row["us"], 4)


def all_kernels(mk, dev, iters, warmup):
    import numpy as np
    import torch
    gen = torch.Generator(device=dev).manual_seed(1)
    rng = np.random.default_rng(1)
    out = []
    f16 = torch.float16

    rope_inv = mk.rope_inv_freq

    # 1. RMSNorm [16, 3584]: launch-latency bound; back-to-back average.
    T, D = 16, 3584
    nb = 2 * T * D * 2 + D * 2
    w = randn16((D,), gen, dev, 1.0, 0.1)
    xs = [randn16((T, D), gen, dev) for _ in range(4)]
    ys = [torch.empty_like(xs[0]) for _ in range(4)]
    sec = time_launches(lambda i: mk.rmsnorm(xs[i], w, y=ys[i]), 4, iters * 4, warmup)
    out.append(report("rmsnorm", "[16,3584]", nb, sec, T))
    # launch-bound: set beside an empty launch replayed the same way
    out[-1]["empty_launch_us"] = round(empty_launch_time() * 1e6, 3)
    del xs, ys

    # 2. fused residual-add + RMSNorm [8192, 3584]
    T, D = 8192, 3584
    nb = 4 * T * D * 2 + D * 2
    ns = rotations(3 * T * D * 2)
    w, sets = fused_sets(mk, dev, gen, T, D, ns)
    sec = time_launches(lambda i: mk.fused_add_rmsnorm(sets[i][0], sets[i][1], w, y=sets[i][2]),
                        ns, iters, warmup)
    out.append(report("fused_add_rmsnorm", "[8192,3584]", nb, sec, T))
    del sets

    # 3. RoPE in place, Q [4096,28,128] + K [4096,4,128], theta 1e6
    T, Hq, Hkv, hd = 4096, 28, 4, 128
    nb = 2 * (T * Hq * hd + T * Hkv * hd) * 2 + T * 8
    ns = rotations((T * (Hq + Hkv) * hd) * 2)
    inv = rope_inv(hd)
    pos = torch.from_numpy(config3_positions(rng, T, 8, 28000)).to(dev)
    qs = [randn16((T, Hq, hd), gen, dev) for _ in range(ns)]
    ks = [randn16((T, Hkv, hd), gen, dev) for _ in range(ns)]
    sec = time_launches(lambda i: mk.rope_neox_qk(qs[i], ks[i], pos, inv), ns, iters, warmup)
    out.append(report("rope_neox_qk", "Q[4096,28,128]+K[4096,4,128]", nb, sec, T, "inplace"))
    del qs, ks
    attach_rope_floors(dev, out[-1], T, Hq, Hkv, hd)

    # 4a/4b. SwiGLU [4096,18944], GeGLU [4096,14336]
    for name, fn, I in (("swiglu", mk.swiglu, 18944), ("geglu", mk.geglu, 14336)):
        T = 4096
        nb = 3 * T * I * 2
        ns = rotations(3 * T * I * 2)
        sets = [(randn16((T, I), gen, dev), randn16((T, I), gen, dev),
                 torch.empty((T, I), dtype=f16, device=dev)) for _ in range(ns)]
        sec = time_launches(lambda i: fn(sets[i][0], sets[i][1], out=sets[i][2]), ns, iters, warmup)
        out.append(report(name, f"[4096,{I}]", nb, sec, T))
        del sets

    # 5. the decoder chain at T = 64 decode + 2 x 3000 prefill = 6064 tokens
    T, D, I, V = 6064, 3584, 18944, 152064
    # 5a. embedding gather from [152064, 3584]
    table = randn16((V, D), gen, dev, 0.0, 0.02)
    nb = T * 8 + 2 * T * D * 2
    ns = 8
    ids = [torch.from_numpy(rng.integers(0, V, T).astype(np.int64)).to(dev) for _ in range(ns)]
    outs = [torch.empty((T, D), dtype=f16, device=dev) for _ in range(ns)]
    sec = time_launches(lambda i: mk.embedding_gather(ids[i], table, out=outs[i]), ns, iters,
                        warmup)
    out.append(report("embedding_gather", "T=6064 from [152064,3584]", nb, sec, T))
    # 5a'. the gather fused with the input RMSNorm (writes hidden and normed)
    nb = T * 8 + 3 * T * D * 2 + D * 2
    w_in = randn16((D,), gen, dev, 1.0, 0.1)
    nrm = [torch.empty((T, D), dtype=f16, device=dev) for _ in range(ns)]
    sec = time_launches(lambda i: mk.embedding_rmsnorm(ids[i], table, w_in, hidden=outs[i],
                                                       y=nrm[i]), ns, iters, warmup)
    out.append(report("embedding_rmsnorm", "T=6064 from [152064,3584]", nb, sec, T))
    # its access pattern with no arithmetic: the gathered rows read, written twice
    fl = floors_lib()
    out[-1]["pattern_floor_us"] = round(time_launches(
        lambda i: _floor_ok(fl.mi_floor_gather2(ids[i].data_ptr(), table.data_ptr(),
                                                outs[i].data_ptr(), nrm[i].data_ptr(), T, D,
                                                torch.cuda.current_stream().cuda_stream)),
        ns, iters, warmup) * 1e6, 3)
    out[-1]["pattern_floor"] = "gather + two row writes, one wave per row (floors.hip)"
    del table, ids, outs, nrm
    # 5b. residual + RMSNorm
    nb = 4 * T * D * 2 + D * 2
    ns = rotations(3 * T * D * 2)
    w, sets = fused_sets(mk, dev, gen, T, D, ns)
    sec = time_launches(lambda i: mk.fused_add_rmsnorm(sets[i][0], sets[i][1], w, y=sets[i][2]),
                        ns, iters, warmup)
    out.append(report("fused_add_rmsnorm", "chain [6064,3584]", nb, sec, T))
    del sets
    # 5c. Q/K RMSNorm, head_dim 128, in place (Q rows and K rows in one launch)
    nb = 2 * (T * 32 * 128) * 2 + 2 * 128 * 2
    ns = rotations(T * 32 * 128 * 2)
    wq = randn16((128,), gen, dev, 1.0, 0.1)
    wk = randn16((128,), gen, dev, 1.0, 0.1)
    qs = [randn16((T * 28, 128), gen, dev) for _ in range(ns)]
    ks = [randn16((T * 4, 128), gen, dev) for _ in range(ns)]

    def qk(i):  # Q-norm and K-norm in one launch (mi_qk_rmsnorm_f16)
        mk.qk_rmsnorm(qs[i].view(T, 28, 128), ks[i].view(T, 4, 128), wq, wk)
    sec = time_launches(qk, ns, iters, warmup)
    out.append(report("qk_rmsnorm", "chain Q[6064*28,128]+K[6064*4,128]", nb, sec, T, "inplace"))
    # 5d. RoPE on the same Q/K (fused Q+K launch)
    nb = 2 * T * 32 * 128 * 2 + T * 8
    pos = torch.from_numpy(chain_positions(rng)).to(dev)
    inv = rope_inv(128)
    sec = time_launches(lambda i: mk.rope_neox_qk(qs[i].view(T, 28, 128), ks[i].view(T, 4, 128),
                                                  pos, inv), ns, iters, warmup)
    out.append(report("rope_neox_qk", "chain Q[6064,28,128]+K[6064,4,128]", nb, sec, T, "inplace"))
    rope_chain_row = out[-1]
    # 5c+5d fused: Q/K RMSNorm + RoPE in one pass (replaces the two rows above)
    nb = 2 * T * 32 * 128 * 2 + T * 8 + 2 * 128 * 2
    sec = time_launches(lambda i: mk.qk_norm_rope(qs[i].view(T, 28, 128), ks[i].view(T, 4, 128),
                                                  wq, wk, pos, inv), ns, iters, warmup)
    out.append(report("qk_norm_rope", "chain Q[6064,28,128]+K[6064,4,128]", nb, sec, T, "inplace"))
    # 5d'. Qwen2.5 proper: the q_proj / k_proj bias added and the rotation in
    # one pass (replaces launch_add_bias on Q and on K, then RoPE)
    bq, bk = randn16((28 * 128,), gen, dev, 0.0, 0.5), randn16((4 * 128,), gen, dev, 0.0, 0.5)
    nb = 2 * T * 32 * 128 * 2 + T * 8 + 32 * 128 * 2
    sec = time_launches(lambda i: mk.bias_rope_neox_qk(qs[i].view(T, 28, 128), ks[i].view(T, 4, 128),
                                                       bq, bk, pos, inv), ns, iters, warmup)
    out.append(report("bias_rope_neox_qk", "chain Q[6064,28,128]+K[6064,4,128]", nb, sec, T,
                      "inplace"))
    del qs, ks
    attach_rope_floors(dev, rope_chain_row, T, 28, 4, 128)
    # 5e. SwiGLU [6064, 18944]
    nb = 3 * T * I * 2
    ns = rotations(3 * T * I * 2)
    sets = [(randn16((T, I), gen, dev), randn16((T, I), gen, dev),
             torch.empty((T, I), dtype=f16, device=dev)) for _ in range(ns)]
    sec = time_launches(lambda i: mk.swiglu(sets[i][0], sets[i][1], out=sets[i][2]), ns, iters,
                        warmup)
    out.append(report("swiglu", "chain [6064,18944]", nb, sec, T))
    del sets
    # 5f. softmax over logits [64, 152064] ~N(0,4)
    N = 64
    nb = 2 * N * V * 2
    ns = rotations(2 * N * V * 2)
    sets = [(randn16((N, V), gen, dev, 0.0, 4.0), torch.empty((N, V), dtype=f16, device=dev))
            for _ in range(ns)]
    ws = torch.zeros(max(1, mk.softmax_workspace_bytes(N, V)), dtype=torch.uint8, device=dev)
    sec = time_launches(lambda i: mk.softmax(sets[i][0], y=sets[i][1], workspace=ws), ns, iters,
                        warmup)
    out.append(report("softmax", "[64,152064]", nb, sec, N))
    del sets
    # 5g. greedy argmax over logits of the same shape (the step after the LM head)
    nb = N * V * 2 + N * 4
    ns = rotations(N * V * 2)
    xs = [randn16((N, V), gen, dev, 0.0, 4.0) for _ in range(ns)]
    wsa = torch.zeros(max(1, mk.greedy_argmax_workspace_bytes(N, V)), dtype=torch.uint8, device=dev)
    outi = torch.empty(N, dtype=torch.int32, device=dev)
    sec = time_launches(lambda i: mk.greedy_argmax(xs[i], out=outi, workspace=wsa), ns, iters,
                        warmup)
    out.append(report("greedy_argmax", "[64,152064]", nb, sec, N))
    # its access pattern with no arithmetic: one workgroup per 8192-element
    # chunk, a row's chunks on one XCD (rows padded to whole chunks)
    fl = floors_lib()
    vp = -(-V // 8192) * 8192
    fbuf = [torch.ones(N * vp, dtype=f16, device=dev) for _ in range(rotations(N * vp * 2))]
    sink = torch.zeros(1 << 20, dtype=torch.int32, device=dev)
    out[-1]["pattern_floor_us"] = round(time_launches(
        lambda i: _floor_ok(fl.mi_floor_read_rows(fbuf[i].data_ptr(), N, vp, 1, sink.data_ptr(),
                                                  sink.numel(),
                                                  torch.cuda.current_stream().cuda_stream)),
        len(fbuf), iters, warmup) * 1e6, 3)
    out[-1]["pattern_floor"] = "8192-element chunk reads, a row's chunks on one XCD (floors.hip)"
    del fbuf
    # 5g''. top-p sampling of 64 rows of 30000 logits (the largest vocabulary
    # that takes the nucleus path; larger ones are greedy): latency-bound
    xt = [randn16((N, 30000), gen, dev, 0.0, 4.0) for _ in range(4)]
    sec = time_launches(lambda i: mk.top_p_sample(xt[i], 0.9, 0.8, 7, out=outi), 4, iters,
                        warmup)
    out.append(report("top_p_sample", "[64,30000] p=0.9 T=0.8", N * 30000 * 2 + N * 4, sec,
                      N))
    del xt
    # 5g'. softmax and argmax of the same logits in one pass
    nb = 2 * N * V * 2 + N * 4
    ysm = [torch.empty((N, V), dtype=f16, device=dev) for _ in range(ns)]
    wsf = torch.zeros(mk.softmax_argmax_workspace_bytes(N, V), dtype=torch.uint8, device=dev)
    sec = time_launches(lambda i: mk.softmax_argmax(xs[i], wsf, probs=ysm[i], out=outi), ns,
                        iters, warmup)
    out.append(report("softmax_argmax", "[64,152064]", nb, sec, N))
    del xs, ysm
    # 5h. paged KV scatter of the chain's K and V [6064, 4, 128], block size
    # 16, as one 6064-token sequence into shuffled physical blocks
    H, hd, bs = 4, 128, 16
    mb = -(-T // bs)
    bt = torch.from_numpy(rng.permutation(mb).astype(np.int32)).to(dev).view(1, mb)
    sl = torch.tensor([T], dtype=torch.int32, device=dev)
    sp = torch.tensor([0], dtype=torch.int32, device=dev)
    nb = 2 * 2 * T * H * hd * 2 + (mb + 2) * 4
    ns = rotations(nb, max_sets=32)
    kv = [(randn16((1, T, H, hd), gen, dev), randn16((1, T, H, hd), gen, dev),
           torch.empty((1, mb, H, bs, hd), dtype=f16, device=dev),
           torch.empty((1, mb, H, bs, hd), dtype=f16, device=dev)) for _ in range(ns)]
    sec = time_launches(lambda i: mk.paged_kv_scatter(kv[i][0], kv[i][2], bt, sl, sp, 0, bs,
                                                      v_src=kv[i][1], v_cache=kv[i][3]),
                        ns, iters, warmup)
    out.append(report("paged_kv_scatter_kv", "chain K+V [6064,4,128] bs=16", nb, sec, T))
    # 5h'. the same with Qwen2's V bias added on the way into the cache
    vb = randn16((H * hd,), gen, dev, 0.0, 0.5)
    sec = time_launches(lambda i: mk.paged_kv_scatter(kv[i][0], kv[i][2], bt, sl, sp, 0, bs,
                                                      v_src=kv[i][1], v_cache=kv[i][3],
                                                      v_bias=vb),
                        ns, iters, warmup)
    out.append(report("paged_kv_scatter_kv_bias", "chain K+V [6064,4,128] bs=16, V bias",
                      nb + H * hd * 2, sec, T))
    del kv
    # 5i. Qwen2.5 attention pre-processing in one launch: RoPE of Q/K in place
    # and the rotated K and the V rows into the paged cache (5d + 5h), with
    # and without the q/k/v bias, for the chain's continuous batch: 64 decode
    # tokens of 64 sequences, then two 3000-token prefills
    dec_start = rng.integers(0, 6000, 64)
    spans = [(0, 64, 1, dec_start), (64, 1, 3000, [0]), (3064, 1, 3000, [9000])]
    perm = rng.permutation(64 * 376 + 188 + 751)
    segs, nxt = [], 0
    for off, B, S, st in spans:
        sl = [int(x) + S for x in st]
        mbs = -(-max(sl) // bs)
        btab = perm[nxt:nxt + B * mbs].reshape(B, mbs).astype(np.int32)
        nxt += B * mbs
        segs.append(dict(token_offset=off, S=S, block_table=torch.from_numpy(btab).to(dev),
                         seq_len=torch.tensor(sl, dtype=torch.int32, device=dev),
                         start_pos=torch.tensor([int(x) for x in st], dtype=torch.int32,
                                                device=dev)))
    NBc = nxt
    nb = 2 * T * 32 * 128 * 2 + T * H * hd * 2 + 2 * T * H * hd * 2 + T * 8
    ns = rotations(nb, max_sets=32)
    sets = [(randn16((T, 28, 128), gen, dev), randn16((T, H, hd), gen, dev),
             randn16((T, H, hd), gen, dev)) for _ in range(ns)]
    kcache = torch.empty((1, NBc, H, bs, hd), dtype=f16, device=dev)
    vcache = torch.empty_like(kcache)
    bv = randn16((H * hd,), gen, dev, 0.0, 0.5)
    for tag, extra in (("", ()), ("_bias", (bq, bk, bv))):
        sec = time_launches(lambda i: mk.rope_kv_scatter(sets[i][0], sets[i][1], sets[i][2], pos,
                                                         inv, kcache, vcache, 0, bs, segs, *extra),
                            ns, iters, warmup)
        out.append(report("rope_kv_scatter" + tag,
                          "chain Q[6064,28,128]+K,V[6064,4,128] -> cache bs=16"
                          + (", q/k/v bias" if extra else ""),
                          nb + (len(extra) and 36 * 128 * 2), sec, T))
    # the same work as the reference composes it: RoPE (or bias + RoPE), then
    # one K+V scatter per segment (V bias on the way)

    def unfused(i, extra):
        qx, kx, vx = sets[i]
        if extra:
            mk.bias_rope_neox_qk(qx, kx, bq, bk, pos, inv)
        else:
            mk.rope_neox_qk(qx, kx, pos, inv)
        for g in segs:
            B, S, o = g["block_table"].shape[0], g["S"], g["token_offset"]
            mk.paged_kv_scatter(kx[o:o + B * S].view(B, S, H, hd), kcache, g["block_table"],
                                g["seq_len"], g["start_pos"], 0, bs,
                                v_src=vx[o:o + B * S].view(B, S, H, hd), v_cache=vcache,
                                v_bias=bv if extra else None)
    for tag, extra in (("", ()), ("_bias", (bq, bk, bv))):
        sec = time_launches(lambda i: unfused(i, extra), ns, iters, warmup)
        out.append(report("rope_kv_scatter" + tag + "_unfused",
                          "RoPE launch + 3 per-segment K+V scatters" + (", bias" if extra else ""),
                          nb + (len(extra) and 36 * 128 * 2), sec, T))
    # 5j. the Gemma-3 form: Q/K RMSNorm + RoPE + K/V scatter in one launch,
    # against qk_norm_rope then the three per-segment scatters
    nbn = nb + 2 * 128 * 2
    sec = time_launches(lambda i: mk.qk_norm_rope_kv_scatter(sets[i][0], sets[i][1], sets[i][2],
                                                             wq, wk, pos, inv, kcache, vcache, 0,
                                                             bs, segs), ns, iters, warmup)
    out.append(report("qk_norm_rope_kv_scatter",
                      "chain Q[6064,28,128]+K,V[6064,4,128] -> cache bs=16, Q/K norm", nbn, sec, T))

    def unfused_norm(i):
        qx, kx, vx = sets[i]
        mk.qk_norm_rope(qx, kx, wq, wk, pos, inv)
        for g in segs:
            B, S, o = g["block_table"].shape[0], g["S"], g["token_offset"]
            mk.paged_kv_scatter(kx[o:o + B * S].view(B, S, H, hd), kcache, g["block_table"],
                                g["seq_len"], g["start_pos"], 0, bs,
                                v_src=vx[o:o + B * S].view(B, S, H, hd), v_cache=vcache)
    sec = time_launches(unfused_norm, ns, iters, warmup)
    out.append(report("qk_norm_rope_kv_scatter_unfused",
                      "qk_norm_rope launch + 3 per-segment K+V scatters", nbn, sec, T))
    del sets, kcache, vcache
    torch.cuda.synchronize()
    for r in out:
        if r["bytes"] >= 8 << 20:
            attach_floors(dev, r, read_only=r["kernel"] == "greedy_argmax")
    return out


# ---------------------------------------------------------------------------
# CPU baseline: the oracle on the host, bounded sample of the headline config
# ---------------------------------------------------------------------------

def host_cpus():
    """The host's processor counts beside the threads a CPU leg used: `nproc`
    (the CPUs this process may run on, os.sched_getaffinity) and
    `hardware_concurrency` (the online CPUs, which C++'s
    std::thread::hardware_concurrency and os.cpu_count both report)."""
    return {"nproc": len(os.sched_getaffinity(0)), "hardware_concurrency": os.cpu_count()}


def cpu_baseline(budget_s=10.0):
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle  # the checker, timed here as the CPU reference implementation
    T, D = 8192, 3584
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    rng = np.random.default_rng(0)
    x = rng.standard_normal((T, D), dtype=np.float32).astype(np.float16)
    r = rng.standard_normal((T, D), dtype=np.float32).astype(np.float16)
    w = (rng.standard_normal(D, dtype=np.float32) * 0.1 + 1).astype(np.float16)
    oracle.fused_add_rmsnorm(x, r, w, 1e-6, nthreads=cores)  # warm
    n = 0
    t0 = time.perf_counter()
    while True:
        oracle.fused_add_rmsnorm(x, r, w, 1e-6, nthreads=cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    sec = el / n
    nbytes = 4 * T * D * 2 + D * 2
    return {
        "value": round(nbytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        **host_cpus(),
        "kind": "port",
        "sample": (f"oracle fused residual-add + RMSNorm (fp32 math) on the full [8192,3584] "
                   f"workload, {n} passes in {el:.1f} s with {cores} threads over rows; "
                   f"{sec * 1e3:.1f} ms/pass, {T / sec:.0f} tokens/s"),
    }


def cpu_torch_baseline(budget_s=5.0):
    """The reference's kernel tests check their GPU output against torch on
    the CPU (tests/verify/verify.py:30-42: fp32 x * rsqrt(mean(x^2) + eps) * w).
    This times that arithmetic, restated here in torch (verify.py is not run),
    on the headline workload: the residual add rounded to fp16 as the
    reference's add kernel does, then the fp32 RMSNorm of the result.  Threads:
    torch's intra-op pool, capped at 16."""
    import torch
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(cores)
    T, D = 8192, 3584
    g = torch.Generator().manual_seed(0)
    x = torch.randn((T, D), generator=g).half()
    r = torch.randn((T, D), generator=g).half()
    w = (torch.randn(D, generator=g) * 0.1 + 1).half()

    def step():
        res = (r.float() + x.float()).half()
        xf, wf = res.float(), w.float()
        return res, (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * wf).half()

    step()
    n, t0 = 0, time.perf_counter()
    while True:
        step()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    sec = el / n
    nbytes = 4 * T * D * 2 + D * 2
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "threads": cores,
            "sample": (f"torch {torch.__version__} CPU fp32 residual add + RMSNorm on the full "
                       f"[8192,3584] workload (the reference tests' torch arithmetic, restated), "
                       f"{n} passes in {el:.1f} s; {sec * 1e3:.1f} ms/pass")}


def cpu_kernel_table(budget_s=1.0):
    """The CPU oracle timed at every config of the kernel table (the
    cpu_baseline leg, per config): the same workload shapes, seeded host
    inputs, `budget_s` of repeated passes each (at least one), threads over
    rows.  Reported beside the GPU rows, not as a target."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle  # the checker, timed here as the CPU reference implementation
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    rng = np.random.default_rng(2)

    def h(shape, mean=0.0, std=1.0):
        return (rng.standard_normal(shape, dtype=np.float32) * std + mean).astype(np.float16)

    def timed(fn):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                return el / n

    rows = []

    def add(kernel, cfg, nbytes, tokens, fn, note=""):
        sec = timed(fn)
        rows.append({"kernel": kernel, "config": cfg, "cpu_us": round(sec * 1e6, 1),
                     "cpu_GBps": round(nbytes / sec / 1e9, 3),
                     "cpu_tokens_per_s": round(tokens / sec, 1), "cpu_note": note})

    D, I, V = 3584, 18944, 152064
    x, w = h((16, D)), h((D,), 1.0, 0.1)
    add("rmsnorm", "[16,3584]", 2 * 16 * D * 2 + D * 2, 16,
        lambda: oracle.rmsnorm(x, w, nthreads=cores))
    for T, cfg in ((8192, "[8192,3584]"), (6064, "chain [6064,3584]")):
        x, r = h((T, D)), h((T, D))
        add("fused_add_rmsnorm", cfg, 4 * T * D * 2 + D * 2, T,
            lambda: oracle.fused_add_rmsnorm(x, r, w, nthreads=cores))
    inv = oracle.rope_inv_freq(128, 1e6)
    for T, pos, cfg in ((4096, config3_positions(rng, 4096, 8, 28000), "Q[4096,28,128]+K[4096,4,128]"),
                        (6064, chain_positions(rng), "chain Q[6064,28,128]+K[6064,4,128]")):
        q, k = h((T, 28, 128)), h((T, 4, 128))

        def rope_qk():
            c, sn = oracle.rope_tables(inv, pos)
            oracle.rope_neox(q, c, sn, nthreads=cores)
            oracle.rope_neox(k, c, sn, nthreads=cores)
        add("rope_neox_qk", cfg, 2 * T * 32 * 128 * 2 + T * 8, T, rope_qk,
            "tables from positions, then Q and K rotated")
        if T == 6064:
            wq, wk = h((128,), 1.0, 0.1), h((128,), 1.0, 0.1)
            add("qk_rmsnorm", "chain Q[6064*28,128]+K[6064*4,128]", 2 * T * 32 * 128 * 2 + 512, T,
                lambda: (oracle.rmsnorm(q.reshape(-1, 128), wq, nthreads=cores),
                         oracle.rmsnorm(k.reshape(-1, 128), wk, nthreads=cores)))

            def qk_norm_rope():
                c, sn = oracle.rope_tables(inv, pos)
                for t, wt in ((q, wq), (k, wk)):
                    n16 = oracle.f32_to_f16(oracle.rmsnorm(t.reshape(-1, 128), wt, nthreads=cores))
                    oracle.rope_neox(n16.reshape(t.shape), c, sn, nthreads=cores)
            add("qk_norm_rope", cfg, 2 * T * 32 * 128 * 2 + T * 8 + 512, T, qk_norm_rope,
                "norm, fp16 rounding, then rotation (the reference's composition)")
            bq, bk = h((28 * 128,), 0.0, 0.5), h((4 * 128,), 0.0, 0.5)

            def bias_rope():
                c, sn = oracle.rope_tables(inv, pos)
                for t, bz in ((q, bq), (k, bk)):
                    n = t.shape[1] * 128
                    b16 = oracle.add_bias(t.reshape(-1), bz, T, n, T * n)
                    oracle.rope_neox(b16.reshape(t.shape), c, sn, nthreads=cores)
            add("bias_rope_neox_qk", cfg, 2 * T * 32 * 128 * 2 + T * 8 + 32 * 128 * 2, T,
                bias_rope, "bias add (fp16 rounding), then rotation (the reference's composition)")
    for name, fn, T, I_, cfg in (("swiglu", oracle.swiglu, 4096, I, "[4096,18944]"),
                                 ("geglu", oracle.geglu, 4096, 14336, "[4096,14336]"),
                                 ("swiglu", oracle.swiglu, 6064, I, "chain [6064,18944]")):
        g, u = h((T, I_)), h((T, I_))
        add(name, cfg, 3 * T * I_ * 2, T, lambda: fn(g, u, nthreads=cores))
        del g, u
    T, VR = 6064, 32768
    table = h((VR, D), 0.0, 0.02)
    ids = rng.integers(0, VR, T).astype(np.int64)
    add("embedding_gather", "T=6064 from [152064,3584]", T * 8 + 2 * T * D * 2, T,
        lambda: oracle.embedding_gather(ids, table, nthreads=cores),
        "from a 32768-row table (235 MB, past the host caches like the 1.09 GB one)")
    del table
    lg = h((64, V), 0.0, 4.0)
    add("softmax", "[64,152064]", 2 * 64 * V * 2, 64, lambda: oracle.softmax(lg, nthreads=cores))
    add("greedy_argmax", "[64,152064]", 64 * V * 2 + 64 * 4, 64, lambda: oracle.greedy_argmax(lg),
        "single thread: the oracle replays the reference's 256-thread scan and tree")
    H, hd, bs = 4, 128, 16
    mb = -(-T // bs)
    bt = rng.permutation(mb).astype(np.int32).reshape(1, mb)
    ksrc, kc = h((1, T, H, hd)), h((1, mb, H, bs, hd))
    sl, sp = np.array([T], np.int32), np.array([0], np.int32)
    add("paged_kv_scatter_kv", "chain K+V [6064,4,128] bs=16", 2 * 2 * T * H * hd * 2 + (mb + 2) * 4,
        T, lambda: (oracle.paged_kv_scatter(ksrc, kc, bt, sl, sp, 0, bs),
                    oracle.paged_kv_scatter(ksrc, kc, bt, sl, sp, 0, bs)),
        "single thread; K and V as two scatters")
    return cores, rows


def chain_bytes(s, segments_tokens):
    """Algorithmic HBM bytes of one chain step (each input read once, each
    output written once), from the workload's shapes."""
    T, D, I, V, N = s["T"], s["hidden_size"], s["intermediate_size"], s["vocab"], s["logit_rows"]
    Hq, Hkv, hd = s["num_heads"], s["num_kv_heads"], s["head_dim"]
    weights = (2 * hd * 2 if s["use_qk_norm"] else 0) + \
        ((Hq + 2 * Hkv) * hd * 2 if s.get("qkv_bias") else 0)       # q/k norm weights, qkv bias
    return ((T * 8 + 3 * T * D * 2 + D * 2)                           # gather + input norm
            + (2 * T * (Hq + Hkv) * hd * 2 + T * 8 + weights)         # (bias,) (qk-norm,) rope
            + (2 * 2 * segments_tokens * Hkv * hd * 2)                # K + V scatter
            + 2 * (4 * T * D * 2 + D * 2)                             # 2x residual add + norm
            + 3 * T * I * 2                                           # SwiGLU
            + (2 * N * V * 2 + N * 4))                                # softmax + argmax


def decoder_chain(mk, dev, iters, warmup, qwen2=False, prefills=(3000, 3000)):
    """The decoder-chain workload as one step: the C++ decoder chain (include/mi_chain.h)
    over one non-GEMM decoder layer at T = 6064 (64 decode tokens at random
    positions + two 3000-token prefills), then the sampling step:
      gather + input RMSNorm -> Q/K-norm + RoPE -> paged K+V scatter ->
      residual add + RMSNorm -> SwiGLU [6064,18944] -> residual add + final
      RMSNorm -> softmax + greedy argmax of the logits [64,152064],
    with seeded stand-ins for the GEMM outputs, captured as one graph.  Also
    timed: the same steps as the reference's caller composes them from its
    unfused launchers (src/model/transformer_model.cpp:561-660;
    src/layers/attention.cpp:743-846): gather, a device copy and RMSNorm, Q-norm and
    K-norm, cos/sin tables then RoPE of Q and of K, one scatter for K and one
    for V per segment, add in place + copy + RMSNorm twice.  Both run this
    library's kernels, so the difference is the fusion alone.  Bytes are the
    fused step's algorithmic bytes.  Two workloads alternate, so consecutive
    steps stream from HBM rather than the Infinity Cache.

    prefills=(): the decode-only step (T = 64), rows named decoder_chain_decode64.

    qwen2: Qwen2.5-7B's own attention pre-processing instead of the chain's
    Gemma-3-style Q/K norm -- the q/k/v_proj bias and no Q/K norm
    (attention.cpp:717-780): the chain adds the q/k/v bias, rotates and writes
    K and V into the cache in one launch; the unfused composition runs
    launch_add_bias on Q, K and V, the tables and two RoPE launches, then the
    two scatters (like the config-5 composition, without the reference's
    Q/K device copies)."""
    import torch
    import mi_chain
    extra = dict(use_qk_norm=0, qkv_bias=1) if qwen2 else {}
    ws = [mi_chain.Workload(dev, seed=5 + i, host=False, prefills=prefills, **extra)
          for i in range(2)]
    s = ws[0].shapes
    T, D, V, N = s["T"], s["hidden_size"], s["vocab"], s["logit_rows"]
    Hq, Hkv, hd = s["num_heads"], s["num_kv_heads"], s["head_dim"]
    inv = mk.rope_inv_freq(hd)
    cos_t = torch.empty((T, hd // 2), dtype=torch.float16, device=dev)
    sin_t = torch.empty_like(cos_t)
    tmp = torch.empty((T, D), dtype=torch.float16, device=dev)
    wss = torch.zeros(max(16, mk.softmax_workspace_bytes(N, V)), dtype=torch.uint8, device=dev)
    wsa = torch.zeros(max(16, mk.greedy_argmax_workspace_bytes(N, V)), dtype=torch.uint8,
                      device=dev)

    def fused(i):
        ws[i].run()

    def unfused(i):
        w = ws[i]
        t = w.t
        mk.embedding_gather(t["ids"], t["embed"], out=t["hidden"])
        tmp.copy_(t["hidden"])
        mk.rmsnorm(tmp, t["input_norm"], y=t["normed"])
        if qwen2:
            for name, n in (("q", Hq), ("k", Hkv), ("v", Hkv)):
                mk.add_bias(t[name], t[name + "_bias"], T, n * hd, T * n * hd)
        else:
            q2, k2 = t["q"].view(T * Hq, hd), t["k"].view(T * Hkv, hd)
            mk.rmsnorm(q2, t["q_norm"], y=q2)
            mk.rmsnorm(k2, t["k_norm"], y=k2)
        mk.rope_tables(inv, t["positions"], cos_t=cos_t, sin_t=sin_t)
        q4, k4 = t["q"].view(1, T, Hq, hd), t["k"].view(1, T, Hkv, hd)
        mk.rope_neox(q4, cos_t, sin_t, y=q4)
        mk.rope_neox(k4, cos_t, sin_t, y=k4)
        for g in w.segments:
            o, B, S = g["token_offset"], g["B"], g["S"]
            for src, cache in ((t["k"], t["k_cache"]), (t["v"], t["v_cache"])):
                mk.paged_kv_scatter(src[o:o + B * S].view(B, S, Hkv, hd), cache, g["block_table"],
                                    g["seq_len"], g["start_pos"], s["layer"], s["block_size"])
        for x, wt, y in ((t["attn_out"], t["post_attn_norm"], t["post_normed"]),
                         (t["mlp_out"], t["final_norm"], t["final_normed"])):
            mk.add_inplace(t["hidden"], x)
            tmp.copy_(t["hidden"])
            mk.rmsnorm(tmp, wt, y=y)
            if y is t["post_normed"]:
                mk.swiglu(t["gate"], t["up"], out=t["act_out"])
        mk.softmax(t["logits"], y=t["probs"], workspace=wss)
        mk.greedy_argmax(t["logits"], out=t["next_tokens"], workspace=wsa)

    nb = chain_bytes(s, sum(g["B"] * g["S"] for g in ws[0].segments))
    cfg = ("gather&norm+qk-norm&rope+kv+add&norm+swiglu+add&norm+softmax&argmax "
           f"T={T} (64 decode + 2x3000 prefill)")
    if qwen2:
        cfg = ("gather&norm+qkv-bias&rope+kv(v-bias)+add&norm+swiglu+add&norm+softmax&argmax "
               f"T={T} (64 decode + 2x3000 prefill)")
    if not prefills:
        cfg = cfg.replace(f"T={T} (64 decode + 2x3000 prefill)", f"T={T} (decode only)")
    rows = []
    suffix = ("_qwen2" if qwen2 else "") + ("" if prefills else f"_decode{T}")
    for name, fn in (("decoder_chain" + suffix, fused), ("decoder_chain" + suffix + "_unfused",
                                                          unfused)):
        sec = time_launches(fn, len(ws), iters, warmup)
        rows.append(report(name, cfg, nb, sec, T))
    rows[0]["speedup_over_unfused"] = round(rows[1]["us"] / rows[0]["us"], 3)
    rows[0]["impl"] = "C++ DecoderChain (mi_decoder_chain_run), one graph"
    del ws
    torch.cuda.synchronize()
    return rows


def shape_table(mk, dev, iters=40, warmup=5):
    """Beyond the benchmark workloads (`--shapes`): each kernel across common
    LLM shapes, ~100-260 MB per launch unless the shape is small by nature,
    timed like the kernel table (graph replay, buffers rotated past the
    Infinity Cache).  Rows: kernel, shape, us, % of HBM peak."""
    import numpy as np
    import torch
    gen = torch.Generator(device=dev).manual_seed(7)
    rng = np.random.default_rng(7)
    f16 = torch.float16
    R = randn16
    rows = []

    def run(kernel, shape, nbytes, fn, ns):
        sec = time_launches(fn, ns, iters, warmup)
        rows.append({"kernel": kernel, "shape": shape, "us": round(sec * 1e6, 2),
                     "frac": round(nbytes / sec / HBM_PEAK, 4)})
        log(f"[shapes]   {kernel:<20} {shape:<26} {sec * 1e6:9.2f} us {100 * nbytes / sec / HBM_PEAK:6.1f}%")

    for D in (1024, 2048, 4096, 5120, 8192, 16384):
        T = max(1, int(200e6 / (4 * D * 2)))
        ns = rotations(3 * T * D * 2)
        w = R((D,), gen, dev, 1, 0.1)
        sets = [(R((T, D), gen, dev), R((T, D), gen, dev), torch.empty((T, D), dtype=f16, device=dev))
                for _ in range(ns)]
        run("fused_add_rmsnorm", f"[{T},{D}]", 4 * T * D * 2,
            lambda i: mk.fused_add_rmsnorm(sets[i][0], sets[i][1], w, y=sets[i][2]), ns)
        del sets
    for (Hq, Hkv, hd) in ((28, 4, 128), (32, 8, 128), (32, 32, 128), (16, 8, 256), (64, 8, 128),
                          (32, 4, 64), (8, 1, 64)):
        T = int(100e6 / ((Hq + Hkv) * hd * 4))
        ns = rotations(T * (Hq + Hkv) * hd * 2)
        pos = torch.from_numpy(rng.integers(0, 32000, T).astype(np.int64)).to(dev)
        inv = mk.rope_inv_freq(hd)
        qs = [R((T, Hq, hd), gen, dev) for _ in range(ns)]
        ks = [R((T, Hkv, hd), gen, dev) for _ in range(ns)]
        wq, wk = R((hd,), gen, dev, 1, 0.1), R((hd,), gen, dev, 1, 0.1)
        nb = 2 * T * (Hq + Hkv) * hd * 2 + T * 8
        run("rope_neox_qk", f"T={T} {Hq}|{Hkv}x{hd}", nb,
            lambda i: mk.rope_neox_qk(qs[i], ks[i], pos, inv), ns)
        run("qk_norm_rope", f"T={T} {Hq}|{Hkv}x{hd}", nb,
            lambda i: mk.qk_norm_rope(qs[i], ks[i], wq, wk, pos, inv), ns)
        del qs, ks
    for N, D in ((57344, 512), (16384, 2048), (8192, 4096), (2048, 32000), (256, 65536),
                 (2048, 40000), (128, 152064), (512, 152064), (1024, 128256)):
        nb = 2 * N * D * 2
        ns = rotations(nb)
        sets = [(R((N, D), gen, dev, 0, 4), torch.empty((N, D), dtype=f16, device=dev))
                for _ in range(ns)]
        ws = torch.zeros(max(1, mk.softmax_workspace_bytes(N, D)), dtype=torch.uint8, device=dev)
        run("softmax", f"[{N},{D}]", nb,
            lambda i: mk.softmax(sets[i][0], y=sets[i][1], workspace=ws), ns)
        del sets
    for B, V in ((256, 152064), (512, 152064), (1024, 152064), (2048, 32000)):
        nb = B * V * 2
        ns = rotations(nb)
        xs = [R((B, V), gen, dev, 0, 4) for _ in range(ns)]
        ws = torch.zeros(max(1, mk.greedy_argmax_workspace_bytes(B, V)), dtype=torch.uint8,
                         device=dev)
        o = torch.empty(B, dtype=torch.int32, device=dev)
        run("greedy_argmax", f"[{B},{V}]", nb,
            lambda i: mk.greedy_argmax(xs[i], out=o, workspace=ws), ns)
        del xs
    for V, H, T in ((128256, 4096, 8192), (152064, 8192, 4096), (32000, 2048, 16384),
                    (128256, 1024, 32768)):
        table = R((V, H), gen, dev, 0, 0.02)
        ids = [torch.from_numpy(rng.integers(0, V, T).astype(np.int64)).to(dev) for _ in range(8)]
        outs = [torch.empty((T, H), dtype=f16, device=dev) for _ in range(8)]
        run("embedding_gather", f"T={T} from [{V},{H}]", T * 8 + 2 * T * H * 2,
            lambda i: mk.embedding_gather(ids[i], table, out=outs[i]), 8)
        del table, outs
    for T, H, hd, bs in ((8192, 8, 128, 16), (16384, 1, 128, 16), (4096, 8, 128, 32)):
        mb = -(-T // bs)
        bt = torch.from_numpy(rng.permutation(mb).astype(np.int32)).to(dev).view(1, mb)
        sl = torch.tensor([T], dtype=torch.int32, device=dev)
        sp = torch.tensor([0], dtype=torch.int32, device=dev)
        nb = 2 * 2 * T * H * hd * 2
        ns = rotations(nb)
        kv = [(R((1, T, H, hd), gen, dev), R((1, T, H, hd), gen, dev),
               torch.empty((1, mb, H, bs, hd), dtype=f16, device=dev),
               torch.empty((1, mb, H, bs, hd), dtype=f16, device=dev)) for _ in range(ns)]
        run("paged_kv_scatter_kv", f"T={T} {H}x{hd} bs={bs}", nb,
            lambda i: mk.paged_kv_scatter(kv[i][0], kv[i][2], bt, sl, sp, 0, bs, v_src=kv[i][1],
                                          v_cache=kv[i][3]), ns)
        del kv
    torch.cuda.synchronize()
    return rows


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-config table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--shapes", action="store_true",
                    help="also time each kernel across common LLM shapes beyond the configs")
    ap.add_argument("--floors", action="store_true",
                    help="also print every calibration-stream form at a range of sizes")
    ap.add_argument("--no-chain", action="store_true",
                    help="skip the whole-chain rows (profiling runs: one row per kernel and grid)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-seconds-per-config", type=float, default=1.0,
                    help="CPU oracle time per kernel-table config")
    ap.add_argument("--eager", action="store_true",
                    help="launch eagerly instead of replaying a HIP graph (profiler counter runs)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: these layer kernels are row-independent and run "
              "without communication, so a multi-GPU run would only repeat the one-GPU figure "
              "per rank; --gpus N > 1 is not benchmarked.", file=sys.stderr)
        sys.exit(2)

    import torch
    import mi_kernels as mk
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    mk.load_library()
    dev = torch.device("cuda:0")

    log("[bench] headline: fused residual-add + RMSNorm [8192,3584]")
    T, D, nbytes, sec = headline(mk, dev, args.steps, args.warmup)
    gbps = nbytes / sec / 1e9

    copy_gbps = copy_calibration(dev)
    log(f"[bench] copy calibration: {copy_gbps:.0f} GB/s")

    kernels = None
    if not args.no_kernels:
        log("[bench] per-config kernel table")
        # The table's rows average at least KERNEL_ITERS back-to-back launches
        # per graph replay whatever --steps is, so the replay's fixed start
        # cost (a few us per graph) stays out of the per-launch figures.
        kit, kwu = max(KERNEL_ITERS, args.steps // 2), max(10, args.warmup // 2)
        cit, cwu = max(CHAIN_ITERS, args.steps // 8), max(5, args.warmup // 4)
        kernels = all_kernels(mk, dev, kit, kwu)
        if not args.no_chain:
            kernels += decoder_chain(mk, dev, cit, cwu)
            kernels += decoder_chain(mk, dev, cit, cwu, qwen2=True)
            # the decode-only step of the same model (64 sequences, one token each):
            # launch-latency territory, where the fusion's saved launches show most
            kernels += decoder_chain(mk, dev, cit, cwu, prefills=())
        for k in kernels:
            floor = ""
            if "frac_of_floor" in k:
                floor = (f"  floors oop {k['oop_floor_us']:7.2f} inplace {k['inplace_floor_us']:7.2f}"
                         + (f" read {k['read_floor_us']:7.2f}" if "read_floor_us" in k else "")
                         + f" us -> {100 * k['frac_of_floor']:5.1f}% of {k['floor_kind']}")
            elif "empty_launch_us" in k:
                floor = f"  empty launch {k['empty_launch_us']:.2f} us"
            if "pattern_floor_us" in k:
                floor += f"  pattern {k['pattern_floor_us']:.2f} us"
            if "rope_floor_us" in k:
                floor += (f"  rope pattern {k['rope_floor_us']:.2f} us (one-token pattern "
                          f"{k['rope_floor_one_token_us']:.2f})")
            log(f"[bench]   {k['kernel']:<18} {k['config']:<38} {k['us']:>9.2f} us "
                f"{k['GBps']:>8.1f} GB/s  {100 * k['frac']:5.1f}%{floor}")

    floors = None
    if args.floors:
        log("[bench] floor sweep")
        floors = floor_sweep(dev)

    shapes = None
    if args.shapes:
        log("[bench] shape table")
        shapes = shape_table(mk, dev)

    cpu = cpu_torch = None
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle on host cores)")
        cpu = cpu_baseline(args.cpu_seconds)
        cpu_torch = cpu_torch_baseline(min(5.0, args.cpu_seconds))
        log(f"[bench] CPU oracle {cpu['value']} GB/s, torch CPU {cpu_torch['value']} GB/s "
            f"({cpu['cores']} threads; nproc {cpu['nproc']}, "
            f"hardware_concurrency {cpu['hardware_concurrency']})")
        if kernels is not None:
            cores, cpu_rows = cpu_kernel_table(args.cpu_seconds_per_config)
            by_key = {(r["kernel"], r["config"]): r for r in cpu_rows}
            for k in kernels:
                c = by_key.get((k["kernel"], k["config"]))
                if c is None:
                    continue
                k.update({kk: v for kk, v in c.items() if kk not in ("kernel", "config")})
                k["cpu_cores"] = cores
                k.update({"cpu_" + kk: v for kk, v in host_cpus().items()})
                k["gpu_over_cpu"] = round(c["cpu_us"] / k["us"], 1)
                log(f"[bench]   cpu {k['kernel']:<18} {k['config']:<38} {c['cpu_us']:>11.1f} us "
                    f"{c['cpu_GBps']:>8.2f} GB/s  ({cores} threads)")

    traffic = None
    tf = ROOT / "profiles" / "fused_add_rmsnorm_8192x3584_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": round(gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) fp16 inputs, N(1,0.1) weight)",
        "config": {
            "workload": "fused residual-add + RMSNorm, Qwen2.5-7B prefill (BASELINE config 2)",
            "tokens": T, "hidden": D, "eps": 1e-6,
            "global_batch": T, "parallelism": "none (1 GPU)",
        },
        "tokens_per_s": round(T / sec, 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbps, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(nbytes / sec / HBM_PEAK, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "cpu_torch": cpu_torch,
        "timing": ("eager launches; HIP events on the launch stream" if EAGER else
                   "HIP graph replay of back-to-back launches; HIP events on the replay stream"),
        "copy_calibration_GBps": round(copy_gbps, 1),
        "kernels": kernels,
    }
    if shapes is not None:
        line["shapes"] = shapes
    if floors is not None:
        line["floors"] = floors
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
