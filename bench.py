#!/usr/bin/env python3
"""Benchmark of the MI355X layer kernels (one GPU).

Headline (the JSON line's `value`): achieved HBM bandwidth of the fused
residual-add + RMSNorm kernel at Qwen2.5-7B prefill, x / residual fp16
[8192, 3584].  One step = one launch over that batch;
inputs are resident in HBM before the timed region.  Buffer sets are rotated
so the working set of consecutive launches exceeds the 256 MB Infinity Cache
and every launch streams from HBM.

Also reported, under "kernels": every BASELINE config, each kernel timed the
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


_FLOOR = {}


def copy_floor(mk, dev, nbytes, iters=50):
    """Seconds for a plain device copy moving the same bytes (half read, half
    written), through the library's gather kernel with identity ids, buffers
    rotated past the Infinity Cache like the kernel under test.  Small
    transfers pay a fixed launch / ramp cost, so this is the practical floor
    for a kernel of that size."""
    import torch
    H = 3584
    rows = max(1, int(round(nbytes / (4 * H))))
    if rows in _FLOOR:
        return _FLOOR[rows]
    ns = rotations(2 * rows * H * 2)
    ids = torch.arange(rows, dtype=torch.int64, device=dev)
    src = [torch.zeros((rows, H), dtype=torch.float16, device=dev) for _ in range(ns)]
    dst = [torch.empty((rows, H), dtype=torch.float16, device=dev) for _ in range(ns)]
    sec = time_launches(lambda i: mk.embedding_gather(ids, src[i], out=dst[i]), ns, iters, 5)
    del src, dst
    _FLOOR[rows] = sec
    return sec


def report(name, cfg, nbytes, seconds, tokens, floor=None):
    r = {
        "kernel": name,
        "config": cfg,
        "bytes": int(nbytes),
        "us": round(seconds * 1e6, 3),
        "GBps": round(nbytes / seconds / 1e9, 1),
        "frac": round(nbytes / seconds / HBM_PEAK, 4),
        "tokens_per_s": round(tokens / seconds, 1),
    }
    if floor is not None:
        r["copy_floor_us"] = round(floor * 1e6, 3)
        r["frac_of_copy_floor"] = round(floor / seconds, 4)
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
# Every BASELINE config
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
    out.append(report("rope_neox_qk", "Q[4096,28,128]+K[4096,4,128]", nb, sec, T))
    del qs, ks

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
    del table, ids, outs
    # 5b. residual + RMSNorm
    nb = 4 * T * D * 2 + D * 2
    ns = rotations(3 * T * D * 2)
    w, sets = fused_sets(mk, dev, gen, T, D, ns)
    sec = time_launches(lambda i: mk.fused_add_rmsnorm(sets[i][0], sets[i][1], w, y=sets[i][2]),
                        ns, iters, warmup)
    out.append(report("fused_add_rmsnorm", "chain [6064,3584]", nb, sec, T))
    del sets
    # 5c. Q/K RMSNorm, head_dim 128, in place (two launches: Q rows, K rows)
    nb = 2 * (T * 32 * 128) * 2 + 2 * 128 * 2
    ns = rotations(T * 32 * 128 * 2)
    wq = randn16((128,), gen, dev, 1.0, 0.1)
    wk = randn16((128,), gen, dev, 1.0, 0.1)
    qs = [randn16((T * 28, 128), gen, dev) for _ in range(ns)]
    ks = [randn16((T * 4, 128), gen, dev) for _ in range(ns)]

    def qk(i):
        mk.rmsnorm(qs[i], wq, y=qs[i])
        mk.rmsnorm(ks[i], wk, y=ks[i])
    sec = time_launches(qk, ns, iters, warmup)
    out.append(report("qk_rmsnorm", "chain Q[6064*28,128]+K[6064*4,128]", nb, sec, T))
    # 5d. RoPE on the same Q/K (fused Q+K launch)
    nb = 2 * T * 32 * 128 * 2 + T * 8
    pos = torch.from_numpy(chain_positions(rng)).to(dev)
    inv = rope_inv(128)
    sec = time_launches(lambda i: mk.rope_neox_qk(qs[i].view(T, 28, 128), ks[i].view(T, 4, 128),
                                                  pos, inv), ns, iters, warmup)
    out.append(report("rope_neox_qk", "chain Q[6064,28,128]+K[6064,4,128]", nb, sec, T))
    # 5c+5d fused: Q/K RMSNorm + RoPE in one pass (replaces the two rows above)
    nb = 2 * T * 32 * 128 * 2 + T * 8 + 2 * 128 * 2
    sec = time_launches(lambda i: mk.qk_norm_rope(qs[i].view(T, 28, 128), ks[i].view(T, 4, 128),
                                                  wq, wk, pos, inv), ns, iters, warmup)
    out.append(report("qk_norm_rope", "chain Q[6064,28,128]+K[6064,4,128]", nb, sec, T))
    del qs, ks
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
    del xs
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
    del kv
    torch.cuda.synchronize()
    for r in out:
        if r["bytes"] >= 8 << 20:
            f = copy_floor(mk, dev, r["bytes"])
            r["copy_floor_us"] = round(f * 1e6, 3)
            r["frac_of_copy_floor"] = round(f / (r["us"] * 1e-6), 4)
    return out


# ---------------------------------------------------------------------------
# CPU baseline: the oracle on the host, bounded sample of the headline config
# ---------------------------------------------------------------------------

def cpu_baseline(budget_s=10.0):
    import numpy as np
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle  # the checker, timed here as the CPU reference implementation
    T, D = 8192, 3584
    cores = max(1, min(16, os.cpu_count() or 1))
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
    cores = max(1, min(16, os.cpu_count() or 1))
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
    cores = max(1, min(16, os.cpu_count() or 1))
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


def decoder_chain(mk, dev, iters, warmup):
    """BASELINE config 5 as one step: the non-GEMM launches of a decoder layer
    at T = 6064 (64 decode tokens + two 3000-token prefills), then the LM-head
    side, all captured back to back:
      gather -> residual-add + RMSNorm -> Q/K-norm + RoPE -> paged K+V scatter
      -> SwiGLU [6064,18944] -> softmax [64,152064] -> greedy argmax.
    Timed twice: with this library's fused entry points, and as the
    reference's caller composes the same steps from its unfused launchers
    (src/model/transformer_model.cpp:414-424, :448; src/layers/attention.cpp:
    754-780): add in place, a device copy, RMSNorm; Q-norm and K-norm; cos/sin
    tables, then RoPE of Q and of K from the tables; one scatter for K and one
    for V.  Both run this library's kernels, so the difference is the fusion
    alone.  Bytes are the fused step's algorithmic bytes."""
    import numpy as np
    import torch
    gen = torch.Generator(device=dev).manual_seed(5)
    rng = np.random.default_rng(5)
    f16 = torch.float16
    T, D, I, V, N = 6064, 3584, 18944, 152064, 64
    Hq, Hkv, hd, bs = 28, 4, 128, 16
    table = randn16((V, D), gen, dev, 0.0, 0.02)
    w1 = randn16((D,), gen, dev, 1.0, 0.1)
    wq, wk = randn16((hd,), gen, dev, 1.0, 0.1), randn16((hd,), gen, dev, 1.0, 0.1)
    inv = mk.rope_inv_freq(hd)
    pos = torch.from_numpy(chain_positions(rng)).to(dev)
    mb = -(-T // bs)
    bt = torch.from_numpy(rng.permutation(mb).astype(np.int32)).to(dev).view(1, mb)
    sl = torch.tensor([T], dtype=torch.int32, device=dev)
    sp = torch.tensor([0], dtype=torch.int32, device=dev)
    cos_t = torch.empty((T, hd // 2), dtype=f16, device=dev)
    sin_t = torch.empty_like(cos_t)
    wss = torch.zeros(max(1, mk.softmax_workspace_bytes(N, V)), dtype=torch.uint8, device=dev)
    wsa = torch.zeros(max(1, mk.greedy_argmax_workspace_bytes(N, V)), dtype=torch.uint8,
                      device=dev)
    am = torch.empty(N, dtype=torch.int32, device=dev)

    def make_set():
        return {
            "ids": torch.from_numpy(rng.integers(0, V, T).astype(np.int64)).to(dev),
            "hidden": torch.empty((T, D), dtype=f16, device=dev),
            "attn": randn16((T, D), gen, dev),
            "hid2d": torch.empty((T, D), dtype=f16, device=dev),
            "normed": torch.empty((T, D), dtype=f16, device=dev),
            "q": randn16((T, Hq, hd), gen, dev), "k": randn16((T, Hkv, hd), gen, dev),
            "v": randn16((T, Hkv, hd), gen, dev),
            "kc": torch.empty((1, mb, Hkv, bs, hd), dtype=f16, device=dev),
            "vc": torch.empty((1, mb, Hkv, bs, hd), dtype=f16, device=dev),
            "g": randn16((T, I), gen, dev), "u": randn16((T, I), gen, dev),
            "act": torch.empty((T, I), dtype=f16, device=dev),
            "logits": randn16((N, V), gen, dev, 0.0, 4.0),
            "probs": torch.empty((N, V), dtype=f16, device=dev),
        }
    sets = [make_set() for _ in range(2)]  # ~1.1 GB of streamed data per step

    def tail(b):
        mk.swiglu(b["g"], b["u"], out=b["act"])
        mk.softmax(b["logits"], y=b["probs"], workspace=wss)
        mk.greedy_argmax(b["logits"], out=am, workspace=wsa)

    def fused(i):
        b = sets[i]
        mk.embedding_gather(b["ids"], table, out=b["hidden"])
        mk.fused_add_rmsnorm(b["attn"], b["hidden"], w1, y=b["normed"])
        mk.qk_norm_rope(b["q"], b["k"], wq, wk, pos, inv)
        mk.paged_kv_scatter(b["k"].view(1, T, Hkv, hd), b["kc"], bt, sl, sp, 0, bs,
                            v_src=b["v"].view(1, T, Hkv, hd), v_cache=b["vc"])
        tail(b)

    def unfused(i):
        b = sets[i]
        mk.embedding_gather(b["ids"], table, out=b["hidden"])
        mk.add_inplace(b["hidden"], b["attn"])
        b["hid2d"].copy_(b["hidden"])
        mk.rmsnorm(b["hid2d"], w1, y=b["normed"])
        q2, k2 = b["q"].view(T * Hq, hd), b["k"].view(T * Hkv, hd)
        mk.rmsnorm(q2, wq, y=q2)
        mk.rmsnorm(k2, wk, y=k2)
        mk.rope_tables(inv, pos, cos_t=cos_t, sin_t=sin_t)
        q4, k4 = b["q"].view(1, T, Hq, hd), b["k"].view(1, T, Hkv, hd)
        mk.rope_neox(q4, cos_t, sin_t, y=q4)
        mk.rope_neox(k4, cos_t, sin_t, y=k4)
        mk.paged_kv_scatter(k4, b["kc"], bt, sl, sp, 0, bs)
        mk.paged_kv_scatter(b["v"].view(1, T, Hkv, hd), b["vc"], bt, sl, sp, 0, bs)
        tail(b)

    nb = ((T * 8 + 2 * T * D * 2) + (4 * T * D * 2 + D * 2)
          + (2 * T * (Hq + Hkv) * hd * 2 + T * 8 + 2 * hd * 2)
          + (2 * 2 * T * Hkv * hd * 2 + (mb + 2) * 4) + 3 * T * I * 2
          + 2 * N * V * 2 + (N * V * 2 + N * 4))
    cfg = "gather+add&norm+qk-norm&rope+kv+swiglu+softmax+argmax T=6064"
    rows = []
    for name, fn in (("decoder_chain_fused", fused), ("decoder_chain_unfused", unfused)):
        sec = time_launches(fn, len(sets), iters, warmup)
        rows.append(report(name, cfg, nb, sec, T))
    rows[0]["speedup_over_unfused"] = round(rows[1]["us"] / rows[0]["us"], 3)
    del sets, table
    torch.cuda.synchronize()
    return rows


def shape_table(mk, dev, iters=40, warmup=5):
    """Beyond the BASELINE configs (`--shapes`): each kernel across common
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
        kernels = all_kernels(mk, dev, max(20, args.steps // 2), max(5, args.warmup // 2))
        if not args.no_chain:
            kernels += decoder_chain(mk, dev, max(10, args.steps // 8), max(3, args.warmup // 4))
        for k in kernels:
            floor = (f"  copy floor {k['copy_floor_us']:7.2f} us ({100 * k['frac_of_copy_floor']:5.1f}%)"
                     if "copy_floor_us" in k else "")
            log(f"[bench]   {k['kernel']:<18} {k['config']:<38} {k['us']:>9.2f} us "
                f"{k['GBps']:>8.1f} GB/s  {100 * k['frac']:5.1f}%{floor}")

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
            f"({cpu['cores']} threads)")
        if kernels is not None:
            cores, cpu_rows = cpu_kernel_table(args.cpu_seconds_per_config)
            by_key = {(r["kernel"], r["config"]): r for r in cpu_rows}
            for k in kernels:
                c = by_key.get((k["kernel"], k["config"]))
                if c is None:
                    continue
                k.update({kk: v for kk, v in c.items() if kk not in ("kernel", "config")})
                k["cpu_cores"] = cores
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
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
