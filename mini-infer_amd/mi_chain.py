"""ctypes binding of the decoder-step chain (include/mi_chain.h, in
libmini_infer.so): the non-GEMM launches of one decoder layer and the
sampling step, in the order of the reference's batched paged forward
(src/model/transformer_model.cpp:545-660).

``ChainDesc`` mirrors ``mi_chain_desc`` field for field; ``run`` checks the
status and raises with the library's message.  ``Stage`` names the stages.
PyTorch supplies device memory and the stream only.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import mi_kernels

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libmini_infer.so"

_i64, _f32, _int, _vp = ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_void_p


class Stage:
    EMBED = 1
    INPUT_NORM = 2
    QK_ROPE = 3
    KV_SCATTER = 4
    POST_ATTN_NORM = 5
    ACTIVATION = 6
    FINAL_NORM = 7
    SAMPLE = 8


class KvSegment(ctypes.Structure):
    _fields_ = [("token_offset", _i64), ("B", _i64), ("S", _i64), ("block_table", _vp),
                ("seq_len", _vp), ("start_pos", _vp), ("max_blocks_per_seq", _i64)]


_PTRS = ["embed", "input_norm", "post_attn_norm", "pre_ff_norm", "post_ff_norm", "final_norm",
         "q_norm", "k_norm", "ids", "positions"]
_BIAS = ["q_bias", "k_bias", "v_bias"]
_BUFS = ["hidden", "normed", "q", "k", "v", "k_cache", "v_cache", "attn_out", "post_normed",
         "gate", "up", "act_out", "mlp_out", "final_normed", "logits", "probs", "next_tokens"]


class ChainDesc(ctypes.Structure):
    _fields_ = ([(n, _i64) for n in ("T", "hidden_size", "intermediate_size", "num_heads",
                                     "num_kv_heads", "head_dim", "vocab", "logit_rows",
                                     "layer", "num_layers", "num_blocks", "block_size")]
                + [(n, _f32) for n in ("rms_eps", "qk_norm_eps", "rope_theta")]
                + [(n, _int) for n in ("norm_add_one", "use_qk_norm", "embed_scale",
                                       "double_norm", "act")]
                + [(n, _vp) for n in _PTRS]
                + [("num_kv_segments", _int), ("kv_segments", ctypes.POINTER(KvSegment))]
                + [(n, _vp) for n in _BUFS]
                + [("sample_ws", _vp), ("sample_ws_bytes", _i64)]
                + [(n, _vp) for n in _BIAS])


_lib = None


def load_library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        mi_kernels.load_library()  # libmini_infer.so depends on it
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C mini-infer_amd`")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.mi_decoder_chain_run.argtypes = [ctypes.POINTER(ChainDesc), _int, _vp]
        lib.mi_decoder_chain_run.restype = _int
        lib.mi_decoder_chain_last_error.argtypes = []
        lib.mi_decoder_chain_last_error.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def make_desc(shapes: dict, tensors: dict, segments) -> tuple:
    """A ChainDesc from `shapes` (ints / floats / flags by field name),
    `tensors` (torch tensors or None by field name) and KV segments (dicts
    with token_offset, B, S and int32 tensors block_table, seq_len,
    start_pos).  Returns (desc, keepalive): keep the second alive as long as
    the first is used."""
    d = ChainDesc()
    for name, _ in ChainDesc._fields_:
        if name in shapes:
            setattr(d, name, shapes[name])
    for name in _PTRS + _BUFS + ["sample_ws"] + _BIAS:
        t = tensors.get(name)
        setattr(d, name, t.data_ptr() if t is not None else None)
    t = tensors.get("sample_ws")
    d.sample_ws_bytes = t.numel() * t.element_size() if t is not None else 0
    segs = (KvSegment * max(1, len(segments)))()
    for i, g in enumerate(segments):
        bt = g["block_table"]
        segs[i] = KvSegment(g["token_offset"], g["B"], g["S"], bt.data_ptr(),
                            g["seq_len"].data_ptr(), g["start_pos"].data_ptr(), bt.shape[-1])
    d.num_kv_segments = len(segments)
    d.kv_segments = segs
    return d, (segs, tensors, segments)


def run(desc: ChainDesc, last_stage: int = Stage.SAMPLE, stream=None) -> None:
    """Enqueue the chain up to `last_stage` on `stream` (default: torch's
    current stream)."""
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    lib = load_library()
    st = lib.mi_decoder_chain_run(ctypes.byref(desc), int(last_stage), ctypes.c_void_p(s.cuda_stream))
    if st != 0:
        raise RuntimeError(f"mi_decoder_chain_run failed: status {st} "
                           f"({lib.mi_decoder_chain_last_error().decode()})")


# ---------------------------------------------------------------------------
# Synthetic workload: a mixed continuous batch (decode tokens + prefills) with
# seeded inputs standing in for the GEMM outputs.  Shared by the tests and
# the benchmark; the shapes default to Qwen2.5-7B.
# ---------------------------------------------------------------------------

QWEN25_7B = dict(hidden_size=3584, intermediate_size=18944, num_heads=28, num_kv_heads=4,
                 head_dim=128, vocab=152064, rms_eps=1e-6, qk_norm_eps=1e-6, rope_theta=1e6,
                 norm_add_one=0, use_qk_norm=1, embed_scale=0, double_norm=0, act=0,
                 qkv_bias=0)


def batch_layout(rng, n_decode, prefills, max_start=28000, block_size=16):
    """Positions and per-sequence KV metadata of a packed batch: `n_decode`
    decode tokens (one each, at a uniform position in [0, max_start)) then
    one prefill per entry of `prefills` (that many tokens from a uniform
    start in [0, max_start), a cached prefix before it).  Returns positions
    [T] and two groups (decode: B = n_decode, S = 1; prefill: B = len,
    S = prompt length, equal lengths) as numpy dicts with start_pos, seq_len,
    block_table [B, max_blocks] (every written logical block mapped to a
    distinct physical block, the rest to block 0), and the pool size."""
    import numpy as np
    dec = rng.integers(0, max_start, n_decode)
    pre_start = rng.integers(0, max_start, len(prefills))
    pos = np.concatenate([dec] + [s + np.arange(n) for s, n in zip(pre_start, prefills)])
    groups = []
    if n_decode:
        groups.append(dict(token_offset=0, S=1, start_pos=dec, seq_len=dec + 1))
    if prefills:
        assert len(set(prefills)) == 1, "prefills of one group share S"
        groups.append(dict(token_offset=n_decode, S=prefills[0], start_pos=pre_start,
                           seq_len=pre_start + prefills[0]))
    need = 0
    for g in groups:
        g["B"] = len(g["start_pos"])
        need += sum((s + g["S"] - 1) // block_size - s // block_size + 1 for s in g["start_pos"])
    num_blocks = need + 64
    phys = rng.permutation(num_blocks)
    nxt = 0
    max_blocks = int(max((g["seq_len"].max() for g in groups), default=1) - 1) // block_size + 1
    for g in groups:
        bt = np.zeros((g["B"], max_blocks), np.int32)
        for b, s in enumerate(g["start_pos"]):
            for lb in range(s // block_size, (s + g["S"] - 1) // block_size + 1):
                bt[b, lb] = phys[nxt]
                nxt += 1
        g["block_table"] = bt
        g["start_pos"] = g["start_pos"].astype(np.int32)
        g["seq_len"] = g["seq_len"].astype(np.int32)
    return pos.astype(np.int64), groups, num_blocks


class Workload:
    """Host inputs (numpy fp16 / int) when built with host=True, and the
    device tensors of one chain step.  Inputs: ids, positions, weights, and
    the GEMM stand-ins q, k, v, attn_out, gate, up, mlp_out, logits."""

    INPUTS = ("ids", "positions", "embed", "input_norm", "post_attn_norm", "pre_ff_norm",
              "post_ff_norm", "final_norm", "q_norm", "k_norm", "q", "k", "v", "attn_out",
              "gate", "up", "mlp_out", "logits", "q_bias", "k_bias", "v_bias")

    def __init__(self, dev, seed=0, n_decode=64, prefills=(3000, 3000), logit_rows=64,
                 num_layers=2, layer=1, block_size=16, host=True, **overrides):
        import numpy as np
        import torch
        cfg = dict(QWEN25_7B)
        cfg.update(overrides)
        rng = np.random.default_rng(seed)
        pos, groups, num_blocks = batch_layout(rng, n_decode, list(prefills), block_size=block_size)
        T = len(pos)
        D, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab"]
        Hq, Hkv, hd = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
        self.cfg = cfg
        self.shapes = dict(cfg, T=T, logit_rows=logit_rows, layer=layer, num_layers=num_layers,
                           num_blocks=num_blocks, block_size=block_size)
        f16 = torch.float16
        spec = {  # name: (shape, mean, std)
            "embed": ((V, D), 0.0, 0.02), "input_norm": ((D,), 1.0, 0.1),
            "post_attn_norm": ((D,), 1.0, 0.1), "pre_ff_norm": ((D,), 1.0, 0.1),
            "post_ff_norm": ((D,), 1.0, 0.1), "final_norm": ((D,), 1.0, 0.1),
            "q_norm": ((hd,), 1.0, 0.1), "k_norm": ((hd,), 1.0, 0.1),
            "q": ((T, Hq, hd), 0.0, 1.0), "k": ((T, Hkv, hd), 0.0, 1.0),
            "v": ((T, Hkv, hd), 0.0, 1.0), "attn_out": ((T, D), 0.0, 1.0),
            "gate": ((T, I), 0.0, 1.0), "up": ((T, I), 0.0, 1.0), "mlp_out": ((T, D), 0.0, 1.0),
            "logits": ((logit_rows, V), 0.0, 4.0),
        }
        if cfg["qkv_bias"]:  # Qwen2 q/k/v_proj bias
            spec.update({"q_bias": ((Hq * hd,), 0.0, 0.5), "k_bias": ((Hkv * hd,), 0.0, 0.5),
                         "v_bias": ((Hkv * hd,), 0.0, 0.5)})
        self.host = {}
        t = {}
        ids = rng.integers(0, V, T).astype(np.int64)
        if host:
            self.host["ids"], self.host["positions"] = ids, pos
            for name, (shape, mean, std) in spec.items():
                a = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
                     + np.float32(mean)).astype(np.float16)
                self.host[name] = a
                t[name] = torch.from_numpy(a).to(dev)
        else:
            gen = torch.Generator(device=dev).manual_seed(seed)
            for name, (shape, mean, std) in spec.items():
                t[name] = (torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)
                           * std + mean).to(f16)
        t["ids"] = torch.from_numpy(ids).to(dev)
        t["positions"] = torch.from_numpy(pos).to(dev)
        for name, shape in (("hidden", (T, D)), ("normed", (T, D)), ("post_normed", (T, D)),
                            ("act_out", (T, I)), ("final_normed", (T, D)),
                            ("probs", (logit_rows, V))):
            t[name] = torch.empty(shape, dtype=f16, device=dev)
        cache = (num_layers, num_blocks, Hkv, block_size, hd)
        t["k_cache"] = torch.zeros(cache, dtype=f16, device=dev)
        t["v_cache"] = torch.zeros(cache, dtype=f16, device=dev)
        t["next_tokens"] = torch.empty(logit_rows, dtype=torch.int32, device=dev)
        t["sample_ws"] = torch.zeros(mi_kernels.softmax_argmax_workspace_bytes(logit_rows, V),
                                     dtype=torch.uint8, device=dev)
        self.groups = groups
        self.segments = [dict(token_offset=g["token_offset"], B=g["B"], S=g["S"],
                              block_table=torch.from_numpy(g["block_table"]).to(dev),
                              seq_len=torch.from_numpy(g["seq_len"]).to(dev),
                              start_pos=torch.from_numpy(g["start_pos"]).to(dev))
                         for g in groups]
        self.t = t
        self.desc, self._keep = make_desc(self.shapes, t, self.segments)

    def reload(self, *names):
        """Copy host inputs back over device buffers a run rewrote in place
        (q and k are rotated in place)."""
        for n in names:
            self.t[n].copy_(__import__("torch").from_numpy(self.host[n]))

    def run(self, last_stage=Stage.SAMPLE, stream=None):
        run(self.desc, last_stage, stream)
