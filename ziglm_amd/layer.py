"""The per-layer fused-op chain of a Gemma layer, as ziglm's GPU layer loop sequences it
(cuda_model.zig:579-730 token path, 1251-1419 batched prefill), with the GEMMs and
attention between the ops left out:

  1. input RMSNorm                      x -> xb                     (cuda_model.zig:580-585)
  2. QK-norm + RoPE + KV append         q in place, K/V -> cache    (643-662)
  3. post-attn norm + add + pre-FFN norm  x += norm(ao); xb = norm(x) (930-942)
  4. GeGLU                              act = gelu(gate) * up       (946-956)
  5. post-FFN norm + add                x += norm(fo)               (962-967)

Steps 3 and 5 read the attention output `ao` and the FFN output `fo` from their own
buffers (in the model they come from the O and down projections). With fuse_next=True,
step 5 also produces the next layer's input norm (xb = norm(x)), so step 1 of the next
layer disappears.

Algorithmic bytes per op are each tensor read once and written once (weights and
positions included), the figures the roofline fractions are computed from.
"""
from dataclasses import dataclass

import numpy as np

from . import bridge as B
from . import synth


@dataclass(frozen=True)
class Shape:
    name: str
    H: int          # hidden
    nh: int         # query heads
    nkv: int        # KV heads
    D: int          # head_dim
    I: int          # FFN intermediate
    max_seq: int
    theta: float = 10000.0
    eps: float = 1e-6
    uo: bool = True  # Gemma (1 + w)


GEMMA_4B = Shape("gemma-4b", 2560, 8, 4, 256, 10240, 4096)
GEMMA_27B = Shape("gemma-27b", 5376, 32, 16, 128, 21504, 8192)


def op_bytes(shape, T, esize, pos_array=True):
    """Algorithmic HBM bytes per op for T tokens, activations of `esize` bytes."""
    H, I = shape.H, shape.I
    qn, kn = shape.nh * shape.D, shape.nkv * shape.D
    w = 4 * H
    return {
        "input_norm": 2 * T * H * esize + w,
        "add_rmsnorm": 4 * T * H * esize + w,
        "qk_norm_rope_kv": (2 * T * qn + 4 * T * kn) * esize + 2 * 4 * shape.D + (4 * T if pos_array else 0),
        "norm_add_norm": 4 * T * H * esize + 2 * w,
        "geglu": 3 * T * I * esize,
        "norm_add": 3 * T * H * esize + w,
        "norm_add_norm_next": 4 * T * H * esize + 2 * w,
    }


CHAIN = ["input_norm", "qk_norm_rope_kv", "norm_add_norm", "geglu", "norm_add"]
CHAIN_FUSED = ["qk_norm_rope_kv", "norm_add_norm", "geglu", "norm_add_norm_next"]


def chain_bytes(shape, T, esize, fused=False):
    b = op_bytes(shape, T, esize)
    return sum(b[k] for k in (CHAIN_FUSED if fused else CHAIN))


class LayerBuffers:
    """Device buffers of one layer instance for T tokens (dtype: B.F32 or B.BF16)."""

    def __init__(self, dev, shape, T, dtype, cache_rows=None):
        self.dev, self.shape, self.T, self.dtype = dev, shape, T, dtype
        es = 4 if dtype == B.F32 else 2
        self.esize = es
        H, I = shape.H, shape.I
        qn, kn = shape.nh * shape.D, shape.nkv * shape.D
        self.cache_rows = cache_rows or shape.max_seq
        a = dev.alloc
        self.x, self.xb, self.ao, self.fo = (a(T * H * es) for _ in range(4))
        self.q, self.k, self.v = a(T * qn * es), a(T * kn * es), a(T * kn * es)
        self.gate, self.up, self.act = (a(T * I * es) for _ in range(3))
        self.kc, self.vc = a(self.cache_rows * kn * es), a(self.cache_rows * kn * es)
        self.pos = a(T * 4)
        self.w = {k: a(H * 4) for k in ("in", "post_attn", "pre_ffn", "post_ffn")}
        self.wq, self.wk = a(shape.D * 4), a(shape.D * 4)

    def fill_random(self, seed=1, pos0=0):
        """Seeded N(0,1) activations, N(0,0.1) weights, positions pos0..pos0+T-1."""
        s, T, H, I = self.shape, self.T, self.shape.H, self.shape.I
        gen = synth.normal_bf16 if self.dtype == B.BF16 else synth.normal_f32
        qn, kn = s.nh * s.D, s.nkv * s.D
        host = {
            "x": gen(seed, "x", (T, H)), "ao": gen(seed, "ao", (T, H)), "fo": gen(seed, "fo", (T, H)),
            "xb": gen(seed, "xb", (T, H)),
            "q": gen(seed, "q", (T, qn)), "k": gen(seed, "k", (T, kn)), "v": gen(seed, "v", (T, kn)),
            "gate": gen(seed, "gate", (T, I)), "up": gen(seed, "up", (T, I)),
        }
        for k, arr in host.items():
            getattr(self, k).upload(arr)
        for k in self.w:
            self.w[k].upload(synth.normal_f32(seed, "w_" + k, (H,), 0, 0.1))
        self.wq.upload(synth.normal_f32(seed, "wq", (s.D,), 0, 0.1))
        self.wk.upload(synth.normal_f32(seed, "wk", (s.D,), 0, 0.1))
        self.pos.upload(np.arange(pos0, pos0 + T, dtype=np.int32))
        self.kc.fill(0)
        self.vc.fill(0)
        return host

    def copy_from(self, other):
        for name in ("x", "xb", "ao", "fo", "q", "k", "v", "gate", "up", "act", "pos", "wq", "wk"):
            getattr(self, name).copy_from(getattr(other, name), getattr(other, name).size_bytes)
        for k in self.w:
            self.w[k].copy_from(other.w[k], other.w[k].size_bytes)


# ---- the five ops -------------------------------------------------------------------

def op_input_norm(dev, L):
    s = L.shape
    dev.rmsNormRows(L.dtype, L.x, L.w["in"], L.xb, L.T, s.H, s.eps, s.uo)


def op_add_rmsnorm(dev, L):
    """Residual add + RMSNorm as the BASELINE.json configs state it: x += r, out = norm(x)
    (r = attention output buffer)."""
    s = L.shape
    dev.addRmsNormRows(L.dtype, L.x, L.ao, L.w["pre_ffn"], L.xb, L.T, s.H, s.eps, s.uo)


def op_qk(dev, L, layer_idx=0):
    s = L.shape
    dev.qkNormRopeKv(L.dtype, L.q, L.k, L.v, L.wq, L.wk, 0, L.kc, L.vc, L.cache_rows, layer_idx,
                     s.max_seq, s.nkv * s.D, L.pos, 0, None, L.T, s.nh, s.nkv, s.D, 0, s.theta,
                     1.0, s.eps, s.uo)


def op_norm_add_norm(dev, L):
    s = L.shape
    dev.rmsNormAddRmsNorm(L.dtype, L.x, L.ao, L.w["post_attn"], L.w["pre_ffn"], L.xb, L.T, s.H,
                          s.eps, s.uo)


def op_geglu(dev, L):
    dev.gegluEx(L.dtype, L.gate, L.up, L.act, L.T * L.shape.I)


def op_norm_add(dev, L):
    s = L.shape
    dev.rmsnormAddRows(L.dtype, L.x, L.fo, L.w["post_ffn"], L.T, s.H, s.eps, s.uo)


def op_norm_add_norm_next(dev, L):
    s = L.shape
    dev.rmsNormAddRmsNorm(L.dtype, L.x, L.fo, L.w["post_ffn"], L.w["in"], L.xb, L.T, s.H, s.eps, s.uo)


OPS = {
    "input_norm": op_input_norm,
    "add_rmsnorm": op_add_rmsnorm,
    "qk_norm_rope_kv": op_qk,
    "norm_add_norm": op_norm_add_norm,
    "geglu": op_geglu,
    "norm_add": op_norm_add,
    "norm_add_norm_next": op_norm_add_norm_next,
}


def run_chain(dev, L, fused=False):
    for name in (CHAIN_FUSED if fused else CHAIN):
        OPS[name](dev, L)
