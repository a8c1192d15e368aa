"""Synthetic Gemma-family GGUF files: the tensor names, shapes, types and metadata a
ziglm GGUF model has (model.zig:156-300 names; gguf.zig:399-451 keys), with seeded
weights from ziglm_amd.synth. Used where no real model file can be fetched: the tests
load small ones, the benchmark a full-size gemma-4-E2B-shaped one.

E2B below is the architecture the reference's benchmark runs (gemma-4-E2B q4_0,
benchmarks/benchmark_final.md:4) as far as the reference's own code fixes it: 35 layers
(per-layer embedding projection of 35 x 256 = 8960 rows over 1536 columns,
cuda_model.zig:513), head_dim 512 layers global (model.zig:270-278), 15 unshared KV
layers for a 35-layer gemma4 (model.zig:600-604). Head counts, the global-layer pattern
and the FFN width are not in the reference and are assumptions (8 query heads, 1 KV head,
every 5th layer global, 6144).
"""
from dataclasses import dataclass, field

import numpy as np

from . import bridge as B
from . import gguf as G
from . import synth


@dataclass
class GgufModelConfig:
    arch: str = "gemma4"
    dim: int = 1536
    n_layers: int = 35
    n_heads: int = 8
    n_kv_heads: int = 1
    head_dim: int = 256          # local (sliding-window) layers
    global_head_dim: int = 512   # every `global_every`-th layer
    global_every: int = 5
    inter: int = 6144
    vocab: int = 262144
    ple: bool = True
    final_softcap: float = 30.0
    eps: float = 1e-6
    weight_type: int = B.Q4_0
    norm_type: int = B.F32
    types: dict = field(default_factory=dict)   # per-kind overrides: "q", "k", "v", "o", "gate", "up",
                                                # "down", "emb", "ple", "ple_proj", "ple_gate", "ple_out"
    no_kv_from: int = -1         # layers from this index on carry no attn_k / attn_v (-1: all do)
    scalars: dict = field(default_factory=dict)  # layer -> (ggml type, value) of layer_output_scale
    tile_rows: int = 64          # seeded rows per matrix, tiled over the rest (0: all rows seeded)


E2B = GgufModelConfig()


def _is_global(cfg, i):
    return cfg.global_every > 0 and (i + 1) % cfg.global_every == 0


def _matrix(cfg, seed, name, qtype, rows, cols):
    """Raw GGUF bytes [rows, row_bytes] of a seeded matrix of type qtype."""
    n = rows if cfg.tile_rows <= 0 else min(rows, cfg.tile_rows)
    if qtype == B.Q4_0:
        src = synth.q4_0_table(seed, n, cols, name)
    elif qtype == B.Q8_0:
        src = synth.q8_0_table(seed, n, cols, name)
    elif qtype == B.Q4_K:
        src = synth.q4_k_table(seed, n, cols, name)
    elif qtype == B.Q6_K:
        src = synth.q6_k_table(seed, n, cols, name)
    else:
        w = synth.normal_f32(seed, name, (n, cols), 0.0, 0.02)
        if qtype == B.F32:
            src = w.view(np.uint8)
        elif qtype == B.F16:
            src = w.astype(np.float16).view(np.uint8)
        elif qtype == B.BF16:
            src = synth.f32_to_bf16(w).view(np.uint8)
        else:
            raise ValueError(f"no synthetic generator for GGML type {qtype}")
    src = src.reshape(n, -1)
    if n == rows:
        return src
    reps = -(-rows // n)
    return np.tile(src, (reps, 1))[:rows]


def _norm(cfg, seed, name, n, qtype=None):
    w = synth.normal_f32(seed, name, (n,), 0.0, 0.1)
    t = cfg.norm_type if qtype is None else qtype
    if t == B.F32:
        return t, w
    if t == B.F16:
        return t, w.astype(np.float16)
    if t == B.BF16:
        return t, synth.f32_to_bf16(w)
    raise ValueError(f"norm type {t}")


def build(cfg=E2B, seed=11):
    """A GGUFWriter holding the model (call .write(path) or .tobytes())."""
    w = G.GGUFWriter()
    a = cfg.arch
    w.kv("general.architecture", G.STRING, a)
    w.kv("general.name", G.STRING, f"synthetic-{a}")
    for k, v in [("block_count", cfg.n_layers), ("context_length", 32768), ("embedding_length", cfg.dim),
                 ("feed_forward_length", cfg.inter), ("attention.head_count", cfg.n_heads),
                 ("attention.head_count_kv", cfg.n_kv_heads), ("attention.key_length", cfg.head_dim),
                 ("attention.sliding_window", 512)]:
        w.kv(f"{a}.{k}", G.UINT32, v)
    w.kv(f"{a}.attention.layer_norm_rms_epsilon", G.FLOAT32, cfg.eps)
    w.kv(f"{a}.rope.freq_base", G.FLOAT32, 1e6)
    if cfg.final_softcap > 0:
        w.kv(f"{a}.final_logit_softcapping", G.FLOAT32, cfg.final_softcap)
    ty = lambda kind: cfg.types.get(kind, cfg.weight_type)  # noqa: E731
    D, L = cfg.dim, cfg.n_layers

    def mat(name, kind, rows, cols, sd):
        t = ty(kind)
        w.tensor(name, t, (cols, rows), _matrix(cfg, sd, name, t, rows, cols))

    def nrm(name, n, sd, qtype=None):
        t, v = _norm(cfg, sd, name, n, qtype)
        w.tensor(name, t, (n,), v)

    mat("token_embd.weight", "emb", cfg.vocab, D, seed)
    if cfg.ple:
        mat("per_layer_token_embd.weight", "ple", cfg.vocab, L * 256, seed + 1)
        mat("per_layer_model_proj.weight", "ple_proj", L * 256, D, seed + 2)
        nrm("per_layer_proj_norm.weight", 256, seed + 3)
    for i in range(L):
        sd = seed * 1000 + 20 * i
        hd = cfg.global_head_dim if _is_global(cfg, i) else cfg.head_dim
        qn, kn = cfg.n_heads * hd, cfg.n_kv_heads * hd
        p = f"blk.{i}."
        nrm(p + "attn_norm.weight", D, sd)
        mat(p + "attn_q.weight", "q", qn, D, sd + 1)
        if cfg.no_kv_from < 0 or i < cfg.no_kv_from:
            mat(p + "attn_k.weight", "k", kn, D, sd + 2)
            mat(p + "attn_v.weight", "v", kn, D, sd + 3)
            nrm(p + "attn_k_norm.weight", hd, sd + 5)
        mat(p + "attn_output.weight", "o", D, qn, sd + 4)
        nrm(p + "attn_q_norm.weight", hd, sd + 6)
        nrm(p + "post_attention_norm.weight", D, sd + 7)
        nrm(p + "ffn_norm.weight", D, sd + 8)
        mat(p + "ffn_gate.weight", "gate", cfg.inter, D, sd + 9)
        mat(p + "ffn_up.weight", "up", cfg.inter, D, sd + 10)
        mat(p + "ffn_down.weight", "down", D, cfg.inter, sd + 11)
        nrm(p + "post_ffw_norm.weight", D, sd + 12)
        if cfg.ple:
            mat(p + "inp_gate.weight", "ple_gate", 256, D, sd + 13)
            mat(p + "proj.weight", "ple_out", D, 256, sd + 14)
            nrm(p + "post_norm.weight", D, sd + 15)
        if i in cfg.scalars:
            t, v = cfg.scalars[i]
            arr = {B.F32: np.array([v], np.float32), B.F16: np.array([v], np.float16),
                   B.BF16: synth.f32_to_bf16(np.array([v], np.float32))}[t]
            w.tensor(p + "layer_output_scale.weight", t, (1,), arr)
    nrm("output_norm.weight", D, seed + 4)
    return w


def weight_bytes(cfg=E2B):
    """Bytes of weights one decode step streams (every matrix once, K/V projections of
    KV-shared layers skipped; the embedding and PLE tables contribute one row each, the
    tied LM head the whole table)."""
    def rb(kind, cols):
        t = cfg.types.get(kind, cfg.weight_type)
        return cols // G.block_size(t) * G.type_size(t)
    D, L = cfg.dim, cfg.n_layers
    unshared = (24 if L == 42 else 15) if cfg.arch == "gemma4" else L  # model.zig:600-604
    total = cfg.vocab * rb("emb", D) + rb("emb", D)
    if cfg.ple:
        total += rb("ple", L * 256) + L * 256 * rb("ple_proj", D)
    for i in range(L):
        hd = cfg.global_head_dim if _is_global(cfg, i) else cfg.head_dim
        qn, kn = cfg.n_heads * hd, cfg.n_kv_heads * hd
        kv = (cfg.no_kv_from < 0 or i < cfg.no_kv_from) and i < unshared
        total += qn * rb("q", D) + (2 * kn * rb("k", D) if kv else 0) + D * rb("o", qn)
        total += 2 * cfg.inter * rb("gate", D) + D * rb("down", cfg.inter)
        if cfg.ple:
            total += 256 * rb("ple_gate", D) + D * rb("ple_out", 256)
    return total
