"""One greedy decode step of a model (ziglm_amd.model.Model: synthetic, or loaded from a
GGUF file), enqueued entirely on the device and captured once as a hipGraph (the
reference's graph decode, cuda_model.zig:1008-1080).

Per step, with the token id and position in device buffers, in the CPU forward's order
(model.zig:486-812):
  x = embedding row of the token * embed_scale                       (494-503)
  PLE: ple = dequant(PLE row) * 16; ctx = proj(x / sqrt(dim)) RMSNorm'd per layer;
       ple = (ple + ctx) / sqrt(2)                                   (506-540)
  per layer l:
    xb = input RMSNorm(x) (or x)                                     (543-548)
    q[, k, v] = QKV projections (one fused launch when all are Q4_0)  (555-558, 617-623)
    Q-norm, K-norm, Gemma-4 V no-scale norm, RoPE(pos), K/V append to layer l's rows
      (one fused launch; a KV-shared layer only normalises and rotates Q) (560-656)
    attn = decode attention over the rows of layer kv_layer          (658-700)
    x += post-attn-norm(O attn); xb = pre-FFN-norm(x)                 (702-727)
    act = GeGLU(gate xb, up xb) (fused with the GEMVs when both Q4_0)   (729-744)
    x += post-FFN-norm(down act)                                      (746-755)
    PLE: x += norm(proj(ple_l * gelu(gate x)))                        (757-781)
    x *= layer_scalar                                                 (783-788)
  logits = LM head(final RMSNorm(x)); soft-cap; token = greedy argmax (792-810, sampler)
Adjacent norms fuse where nothing sits between them: the post-attention norm, residual
add and pre-FFN norm are one launch, and so are the post-FFN norm, add and the next
layer's input norm when the layer has no PLE and no scalar.

The argmax writes the token buffer the next step's embedding gather reads, so consecutive
replays decode autoregressively without the host; only the position is uploaded (an
ordered asynchronous copy on the same stream) before each replay.
"""
import ctypes

import numpy as np

from . import bridge as B
from .device import Graph
from .layer import GEMMA_4B
from .model import PLE_DIM, Model


class DecodeModel:
    def __init__(self, dev, model, max_seq=4096, own_model=False):
        """Decode state (activations, f32 KV cache [layers][max_seq][max_kv_dim],
        attention workspace) for `model`; own_model: free the model with this object."""
        if model.activation != "geglu":
            raise NotImplementedError(f"{model.arch}: only the GeGLU (Gemma) feed-forward is built")
        m = self.model = model
        self.dev, self.max_seq, self.own_model = dev, max_seq, own_model
        self.L, self.V, self.H = len(m.layers), m.vocab, m.dim
        self.host = m.host
        H = m.dim
        qmax = max(l.n_heads * l.head_dim for l in m.layers)
        kmax = m.max_kv_dim
        imax = max(l.intermediate_size for l in m.layers)
        f4 = lambda n: dev.alloc(max(n, 1) * 4)  # noqa: E731
        self.x, self.xb, self.q, self.k, self.v = f4(H), f4(H), f4(qmax), f4(kmax), f4(kmax)
        self.attn, self.ao, self.act, self.fo, self.logits = f4(qmax), f4(H), f4(imax), f4(H), f4(m.vocab)
        self.up = f4(imax)
        self.cache_rows = self.L * max_seq
        self.kv_dim = kmax
        self.kc, self.vc = f4(self.cache_rows * kmax), f4(self.cache_rows * kmax)
        self.kc.fill(0)
        self.vc.fill(0)
        self.ple = None
        if m.ple_table is not None:
            n = self.L * PLE_DIM
            self.ple, self.ple_ctx, self.ple_gate, self.ple_buf = f4(n), f4(n), f4(PLE_DIM), f4(PLE_DIM)
        self.token, self.pos = dev.alloc(16), dev.alloc(16)
        self.ws_bytes = max(dev.attentionWorkspaceBytes(1, l.n_heads, l.n_kv_heads, l.head_dim, max_seq,
                                                        l.sliding_window) for l in m.layers)
        self.ws = dev.alloc(max(self.ws_bytes, 16))
        self.graph = None

    @classmethod
    def synthetic(cls, dev, shape=GEMMA_4B, n_layers=34, vocab=262144, max_seq=4096, seed=7, final_softcap=30.0,
                  attn_scale=1.0, host_weights=False):
        """The synthetic Gemma-shaped model of Model.synthetic (host_weights: keep every
        weight on the host too, for checking)."""
        m = Model.synthetic(dev, shape, n_layers, vocab, seed, final_softcap, attn_scale, host_weights)
        return cls(dev, m, max_seq, own_model=True)

    # ---- the step -------------------------------------------------------------------------
    def _norm(self, x, w, out, n, uo=None):
        m = self.model
        self.dev.rmsNorm(x, w, out, n, m.eps, m.unit_offset if uo is None else uo)

    def _gemv(self, t, x, y):
        self.dev.gemv(t.qtype, t.buf, x, y, t.rows, t.cols)

    def _input_norm(self, layer):
        m, d = self.model, self.dev
        if layer is None:
            self._norm(self.x, m.output_norm, self.xb, m.dim)
        elif layer.input_layernorm is not None:
            self._norm(self.x, layer.input_layernorm, self.xb, m.dim)
        else:
            d.copyF32(self.x, self.xb, m.dim)

    def _ple_prologue(self):
        """model.zig:506-540 (token path)."""
        m, d = self.model, self.dev
        n = self.L * PLE_DIM
        d.embedGather(m.ple_table.buf, m.ple_table.qtype, m.ple_table.rows, self.token, B.F32, self.ple, 1, n,
                      float(np.sqrt(np.float32(PLE_DIM))))
        if m.ple_proj is None:
            return
        d.scaleEx(B.F32, self.x, float(np.float32(1.0) / np.sqrt(np.float32(m.dim))), self.xb, m.dim)
        self._gemv(m.ple_proj, self.xb, self.ple_ctx)
        if m.ple_proj_norm is not None:
            d.rmsNormRows(B.F32, self.ple_ctx, m.ple_proj_norm, self.ple_ctx, self.L, PLE_DIM, m.eps, False)
            d.add(self.ple, self.ple_ctx, n)
            d.scale(self.ple, float(np.float32(1.0) / np.sqrt(np.float32(2.0))), n)

    def _ple_layer(self, ly):
        """model.zig:757-781."""
        m, d = self.model, self.dev
        self._gemv(ly.per_layer_input_gate, self.x, self.ple_gate)
        d.geglu(self.ple_gate, self.ple.at(4 * ly.index * PLE_DIM), self.ple_buf, PLE_DIM)
        self._gemv(ly.per_layer_projection, self.ple_buf, self.fo)
        if ly.post_per_layer_input_norm is not None:
            self._norm(self.fo, ly.post_per_layer_input_norm, self.fo, m.dim, uo=False)
        d.add(self.x, self.fo, m.dim)

    def step_ops(self):
        """Enqueue one decode step on dev.stream (token and position read from the device)."""
        m, d = self.model, self.dev
        H = m.dim
        d.embedGather(m.token_embd.buf, m.token_embd.qtype, m.token_embd.rows, self.token, B.F32, self.x, 1, H,
                      m.embed_scale)
        if self.ple is not None:
            self._ple_prologue()
        self._input_norm(m.layers[0])
        for i, ly in enumerate(m.layers):
            nxt = m.layers[i + 1] if i + 1 < self.L else None
            self._attention_block(ly)
            self._ffn_block(ly)
            # post-FFN norm + residual, then PLE / scalar, then the next input norm
            has_ple = self.ple is not None and ly.per_layer_input_gate is not None and \
                ly.per_layer_projection is not None
            tail_plain = not has_ple and ly.layer_scalar == 1.0
            nxt_w = m.output_norm if nxt is None else nxt.input_layernorm
            if tail_plain and ly.post_feedforward_layernorm is not None and nxt_w is not None:
                d.rmsNormAddRmsNorm(B.F32, self.x, self.fo, ly.post_feedforward_layernorm, nxt_w, self.xb, 1, H,
                                    m.eps, m.unit_offset)
                continue
            if ly.post_feedforward_layernorm is not None:
                d.rmsnormAdd(self.x, self.fo, ly.post_feedforward_layernorm, H, m.eps, m.unit_offset)
            else:
                d.add(self.x, self.fo, H)
            if has_ple:
                self._ple_layer(ly)
            if ly.layer_scalar != 1.0:
                d.scale(self.x, ly.layer_scalar, H)
            self._input_norm(nxt)
        self._gemv(m.lm_head, self.xb, self.logits)
        if m.final_softcap > 0.0:
            d.tanhSoftcap(self.logits, m.final_softcap, self.V)
        d.argmax(self.logits, self.V, self.token)

    def _attention_block(self, ly):
        m, d = self.model, self.dev
        H = m.dim
        qn, kn = ly.n_heads * ly.head_dim, ly.n_kv_heads * ly.head_dim
        q, k, v = ly.attn_q, ly.attn_k, ly.attn_v
        if not ly.kv_shared and all(t is not None and t.qtype == B.Q4_0 for t in (q, k, v)):
            d.gemvQkvQ4_0(q.buf, k.buf, v.buf, self.xb, self.q, self.k, self.v, qn, kn, kn, H)
        else:
            if q is not None:
                self._gemv(q, self.xb, self.q)
            if not ly.kv_shared:
                if k is not None:
                    self._gemv(k, self.xb, self.k)
                if v is not None:
                    self._gemv(v, self.xb, self.v)
        shared = ly.kv_shared
        d.qkNormRopeKv(B.F32, self.q, None if shared else self.k, None if shared else self.v, ly.attn_q_norm,
                       None if shared else ly.attn_k_norm, ly.v_norm and not shared, self.kc, self.vc,
                       self.cache_rows, ly.index, self.max_seq, self.kv_dim, self.pos, 0, None, 1, ly.n_heads,
                       0 if shared else ly.n_kv_heads, ly.head_dim, ly.rotary_dim, ly.rope_theta, m.rope_freq_scale,
                       m.eps, m.unit_offset)
        d.attentionDecode(B.F32, self.q, self.kc, self.vc, self.attn, self.cache_rows, self.kv_dim, None,
                          ly.kv_layer * self.max_seq, self.pos, 0, self.max_seq, 1, ly.n_heads, ly.n_kv_heads,
                          ly.head_dim, ly.attn_scale, m.attn_softcap, ly.sliding_window, self.ws, self.ws_bytes)
        if ly.attn_output is not None:
            self._gemv(ly.attn_output, self.attn, self.ao)
        # x += post-attn-norm(ao); xb = pre-FFN-norm(x)
        pa, pf = ly.post_attention_layernorm, ly.pre_feedforward_layernorm
        if pa is not None and pf is not None:
            d.rmsNormAddRmsNorm(B.F32, self.x, self.ao, pa, pf, self.xb, 1, H, m.eps, m.unit_offset)
            return
        if pa is not None:
            d.rmsnormAdd(self.x, self.ao, pa, H, m.eps, m.unit_offset)
        else:
            d.add(self.x, self.ao, H)
        if pf is not None:
            self._norm(self.x, pf, self.xb, H)
        else:
            d.copyF32(self.x, self.xb, H)

    def _ffn_block(self, ly):
        m, d = self.model, self.dev
        H, I = m.dim, ly.intermediate_size
        g, u = ly.ffn_gate, ly.ffn_up
        if g is not None and u is not None and g.qtype == B.Q4_0 and u.qtype == B.Q4_0:
            d.gemvGegluQ4_0(g.buf, u.buf, self.xb, self.act, I, H)
        else:
            if g is not None:
                self._gemv(g, self.xb, self.act)
            if u is not None:
                self._gemv(u, self.xb, self.up)
            d.geglu(self.act, self.up, self.act, I)
        if ly.ffn_down is not None:
            self._gemv(ly.ffn_down, self.act, self.fo)

    # ---- driving -------------------------------------------------------------------------
    def capture(self):
        self.graph = Graph(self.dev, self.step_ops)
        return self.graph

    def reset(self, token):
        """Empty KV cache and the given current token."""
        self.kc.fill(0, self.dev.stream)
        self.vc.fill(0, self.dev.stream)
        self.dev.sync()
        self.set_token(token)

    def set_token(self, token):
        self.token.upload(np.array([token], np.uint32))

    def step(self, pos, graph=True):
        """Upload pos (synchronously) and enqueue one step; the next token stays on the
        device."""
        self.pos.upload(np.array([pos], np.int32))
        if graph:
            self.graph.launch()
        else:
            self.step_ops()

    def run(self, pos0, n_steps):
        """Enqueue n_steps graph replays at positions pos0, pos0+1, ... without host syncs:
        the positions are staged in pinned host memory that stays untouched until the run
        has finished, and each replay is preceded by an ordered copy of its slot."""
        b = self.dev.b
        host = ctypes.c_void_p()
        b.check(b.hip_malloc_host(ctypes.byref(host), 4 * n_steps), "malloc_host")
        try:
            arr = (ctypes.c_int32 * n_steps).from_address(host.value)
            for k in range(n_steps):
                arr[k] = pos0 + k
            for k in range(n_steps):
                b.check(b.hip_memcpy_h2d(self.pos.ptr, host.value + 4 * k, 4, self.dev.stream), "pos upload")
                self.graph.launch()
            self.dev.sync()
        finally:
            b.hip_free_host(host)

    def read_token(self):
        return int(self.token.to_numpy((4,), np.uint32)[0])

    def free(self):
        if self.graph is not None:
            self.graph.destroy()
            self.graph = None
        bufs = [self.x, self.xb, self.q, self.k, self.v, self.attn, self.ao, self.act, self.up, self.fo, self.logits,
                self.kc, self.vc, self.token, self.pos, self.ws]
        if self.ple is not None:
            bufs += [self.ple, self.ple_ctx, self.ple_gate, self.ple_buf]
        for b in bufs:
            b.deinit()
        if self.own_model:
            self.model.free()


def cache_bytes(model, max_seq):
    """Device bytes of the f32 K and V caches for `model` at max_seq positions."""
    return 2 * 4 * len(model.layers) * max_seq * model.max_kv_dim

