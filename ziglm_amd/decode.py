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
    q[, k, v] = QKV projections (one launch when all three share a type) (555-558, 617-623)
    Q-norm, K-norm, Gemma-4 V no-scale norm, RoPE(pos), K/V append to layer l's rows
      (a KV-shared layer only normalises and rotates Q) (560-656), then
    attn = decode attention over the rows of layer kv_layer          (658-700):
      one launch for both by default ("attn": hip_attention_decode_qk), else two
    x += post-attn-norm(O attn); xb = pre-FFN-norm(x)                 (702-727)
    act = GeGLU(gate xb, up xb) (in the GEMV when both share a type)   (729-744)
    x += post-FFN-norm(down act)                                      (746-755)
    PLE: x += norm(proj(ple_l * gelu(gate x)))                        (757-781)
    x *= layer_scalar                                                 (783-788)
  logits = LM head(final RMSNorm(x)); soft-cap; token = greedy argmax (792-810, sampler)
A norm / residual add runs either as its own launch (adjacent ones fused: post-attention
norm + add + pre-FFN norm; post-FFN [or PLE] norm + add + next input norm) or in the input
prologue of the product that consumes it (hip_gemv_pro / hip_gemv_qkv_pro), chosen per
product ("qkv", "ffn", "ple", "head"; default_fuse): the QKV product can add the previous
layer's pending residual term and apply the input norm, the gate.up GeGLU product the
attention branch and the pre-FFN norm, the PLE gate product the FFN branch, the PLE
projection its gelu(gate) * ple input, the LM head the final norm.

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
    def __init__(self, dev, model, max_seq=4096, own_model=False, fused=True):
        """Decode state (activations, f32 KV cache [layers][max_seq][max_kv_dim],
        attention workspace) for `model`; own_model: free the model with this object;
        fused: True for the default set of products that take their norms / residual adds
        in a prologue, and whether attention takes the QK-norm / RoPE / KV append
        (default_fuse), False for none, or a set of "qkv", "ffn", "ple", "head", "attn"."""
        if model.activation != "geglu":
            raise NotImplementedError(f"{model.arch}: only the GeGLU (Gemma) feed-forward is built")
        missing = [f"blk.{l.index}" for l in model.layers
                   if l.attn_q is None or l.attn_output is None or l.ffn_gate is None or l.ffn_up is None or
                   l.ffn_down is None or (not l.kv_shared and (l.attn_k is None or l.attn_v is None))]
        if missing:
            raise NotImplementedError(f"layers without all projections are not built: {missing[:4]}")
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
        self.x2 = f4(H)
        self.fuse = set(default_fuse(m) if fused is True else (fused or ()))
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
                  attn_scale=1.0, host_weights=False, fused=True):
        """The synthetic Gemma-shaped model of Model.synthetic (host_weights: keep every
        weight on the host too, for checking)."""
        m = Model.synthetic(dev, shape, n_layers, vocab, seed, final_softcap, attn_scale, host_weights)
        return cls(dev, m, max_seq, own_model=True, fused=fused)

    # ---- the step -------------------------------------------------------------------------
    def _norm(self, x, w, out, n, uo=None):
        m = self.model
        self.dev.rmsNorm(x, w, out, n, m.eps, m.unit_offset if uo is None else uo)

    def _gemv(self, t, x, y):
        self.dev.gemv(t.qtype, t.buf, x, y, t.rows, t.cols)

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
            d.pleCtxFuse(self.ple, self.ple_ctx, n, True)

    def step_ops(self):
        """Enqueue one decode step on dev.stream (token and position read from the device)."""
        self._step()

    # ---- fused step: norms and residual adds in the products' input prologues -------------
    def _input(self, pend, weight, fuse, xb_out=None):
        """Source vector and prologue of a product whose input is [RMSNorm](x + pending term),
        the pending term (r, r_weight, r_unit_offset, scale) being x's update from the block
        before. fuse: the product's prologue computes it (x is read from one buffer and
        workgroup 0 writes the updated x to the other; xb_out receives the input). Otherwise
        the norm kernels update x in place and write xb first, and the product reads xb."""
        m, d = self.model, self.dev
        H = m.dim
        if fuse:
            r, rw, ruo, sc = pend if pend is not None else (None, None, False, 1.0)
            pro = d.prologue(B.PRO_NORM, r=r, r_weight=rw, r_unit_offset=ruo, scale=sc,
                             x_out=self.x_alt if pend is not None else None, weight=weight, unit_offset=m.unit_offset,
                             eps=m.eps, xb_out=xb_out)
            src = self.x_cur
            if pend is not None:
                self.x_cur, self.x_alt = self.x_alt, self.x_cur
            return src, pro
        if pend is not None:
            r, rw, ruo, sc = pend
            if rw is not None and weight is not None and sc == 1.0 and ruo == m.unit_offset:
                d.rmsNormAddRmsNorm(B.F32, self.x_cur, r, rw, weight, self.xb, 1, H, m.eps, m.unit_offset)
                return self.xb, None
            if rw is not None:
                d.rmsnormAdd(self.x_cur, r, rw, H, m.eps, ruo)
            else:
                d.add(self.x_cur, r, H)
            if sc != 1.0:
                d.scale(self.x_cur, sc, H)
        if weight is not None:
            self._norm(self.x_cur, weight, self.xb, H)
            return self.xb, None
        if xb_out is not None:
            d.copyF32(self.x_cur, self.xb, H)
            return self.xb, None
        return self.x_cur, None

    def _step(self):
        """Per layer: QKV, QK-norm / RoPE / KV append, attention, O, gate.up GeGLU, down
        [, PLE gate, PLE projection]; then the LM head, soft-cap and argmax. Each norm /
        residual add runs in the prologue of the product that consumes it when that product
        is in self.fuse ("qkv", "ffn", "ple", "head"; "attn": QK work inside attention),
        else as its own launch (adjacent norms
        fused: post-attention norm + add + pre-FFN norm; post-FFN norm + add + next input
        norm)."""
        m, d, F = self.model, self.dev, self.fuse
        H = m.dim
        self.x_cur, self.x_alt = self.x, self.x2
        d.embedGather(m.token_embd.buf, m.token_embd.qtype, m.token_embd.rows, self.token, B.F32, self.x, 1, H,
                      m.embed_scale)
        if self.ple is not None:
            self._ple_prologue()
        pend = None
        for ly in m.layers:
            qn, kn = ly.n_heads * ly.head_dim, ly.n_kv_heads * ly.head_dim
            q, k, v = ly.attn_q, ly.attn_k, ly.attn_v
            mixed = not ly.kv_shared and not (q.qtype == k.qtype == v.qtype)
            src, pro = self._input(pend, ly.input_layernorm, "qkv" in F, xb_out=self.xb if mixed else None)
            if ly.kv_shared:
                d.gemvPro(q.qtype, q.buf, None, src, self.q, qn, H, pro)
            elif not mixed:
                d.gemvQkvPro(q.qtype, q.buf, k.buf, v.buf, src, self.q, self.k, self.v, qn, kn, kn, H, pro)
            else:
                d.gemvPro(q.qtype, q.buf, None, src, self.q, qn, H, pro)
                self._gemv(k, self.xb, self.k)
                self._gemv(v, self.xb, self.v)
            self._attention_core(ly)
            # x += post-attn-norm(ao); act = GeGLU(pre-FFN-norm(x))
            pend = (self.ao, ly.post_attention_layernorm, m.unit_offset, 1.0)
            g, u, I = ly.ffn_gate, ly.ffn_up, ly.intermediate_size
            pair = g.qtype == u.qtype
            src, pro = self._input(pend, ly.pre_feedforward_layernorm, "ffn" in F, xb_out=None if pair else self.xb)
            if pair:
                d.gemvPro(g.qtype, g.buf, u.buf, src, self.act, I, H, pro)
            else:
                d.gemvPro(g.qtype, g.buf, None, src, self.act, I, H, pro)
                self._gemv(u, self.xb, self.up)
                d.geglu(self.act, self.up, self.act, I)
            self._gemv(ly.ffn_down, self.act, self.fo)
            pend = (self.fo, ly.post_feedforward_layernorm, m.unit_offset, 1.0)
            if self.ple is not None and ly.per_layer_input_gate is not None and ly.per_layer_projection is not None:
                # x += post-FFN-norm(fo); gate = W x; d = P (gelu(gate) * ple_l); pending: norm(d)
                t = ly.per_layer_input_gate
                src, pro = self._input(pend, None, "ple" in F)
                d.gemvPro(t.qtype, t.buf, None, src, self.ple_gate, t.rows, H, pro)
                t = ly.per_layer_projection
                ple_l = self.ple.at(4 * ly.index * PLE_DIM)
                if "ple" in F:
                    d.gemvPro(t.qtype, t.buf, None, self.ple_gate, self.fo, t.rows, t.cols,
                              d.prologue(B.PRO_GEGLU, r=ple_l))
                else:
                    d.pleGateGelu(self.ple_gate, ple_l, self.ple_buf, PLE_DIM)
                    self._gemv(t, self.ple_buf, self.fo)
                pend = (self.fo, ly.post_per_layer_input_norm, False, 1.0)
            if ly.layer_scalar != 1.0:
                pend = pend[:3] + (ly.layer_scalar,)
        t = m.lm_head
        src, pro = self._input(pend, m.output_norm, "head" in F)
        d.gemvPro(t.qtype, t.buf, None, src, self.logits, t.rows, t.cols, pro)
        if m.final_softcap > 0.0:
            d.tanhSoftcap(self.logits, m.final_softcap, self.V)
        d.argmax(self.logits, self.V, self.token)

    def _attention_core(self, ly):
        """QK-norm / RoPE / KV append, attention, O projection (q, k, v -> ao). With "attn"
        in the fuse set (and a rotary width the fused kernel takes), one attention launch
        normalises and rotates q and forms, uses and stores the token's K/V row."""
        m, d = self.model, self.dev
        shared = ly.kv_shared
        if "attn" in self.fuse and qk_attention_ok(ly):
            d.attentionDecodeQk(B.F32, self.q, None if shared else self.k, None if shared else self.v,
                                ly.attn_q_norm, None if shared else ly.attn_k_norm, ly.v_norm and not shared,
                                self.kc, self.vc, self.attn, self.cache_rows, self.kv_dim, None,
                                ly.kv_layer * self.max_seq, self.pos, 0, self.max_seq, 1, ly.n_heads, ly.n_kv_heads,
                                ly.head_dim, ly.rotary_dim, ly.rope_theta, m.rope_freq_scale, m.eps, m.unit_offset,
                                ly.attn_scale, m.attn_softcap, ly.sliding_window, self.ws, self.ws_bytes)
            self._gemv(ly.attn_output, self.attn, self.ao)
            return
        d.qkNormRopeKv(B.F32, self.q, None if shared else self.k, None if shared else self.v, ly.attn_q_norm,
                       None if shared else ly.attn_k_norm, ly.v_norm and not shared, self.kc, self.vc,
                       self.cache_rows, ly.index, self.max_seq, self.kv_dim, self.pos, 0, None, 1, ly.n_heads,
                       0 if shared else ly.n_kv_heads, ly.head_dim, ly.rotary_dim, ly.rope_theta, m.rope_freq_scale,
                       m.eps, m.unit_offset)
        d.attentionDecode(B.F32, self.q, self.kc, self.vc, self.attn, self.cache_rows, self.kv_dim, None,
                          ly.kv_layer * self.max_seq, self.pos, 0, self.max_seq, 1, ly.n_heads, ly.n_kv_heads,
                          ly.head_dim, ly.attn_scale, m.attn_softcap, ly.sliding_window, self.ws, self.ws_bytes)
        self._gemv(ly.attn_output, self.attn, self.ao)

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
        bufs = [self.x, self.x2, self.xb, self.q, self.k, self.v, self.attn, self.ao, self.act, self.up, self.fo, self.logits,
                self.kc, self.vc, self.token, self.pos, self.ws]
        if self.ple is not None:
            bufs += [self.ple, self.ple_ctx, self.ple_gate, self.ple_buf]
        for b in bufs:
            b.deinit()
        if self.own_model:
            self.model.free()


def qk_attention_ok(ly):
    """Whether the fused QK + attention kernel takes the layer's RoPE: rotary_dim / 2 a
    multiple of 8 with rotary_dim / 16 a power of two."""
    eff = ly.head_dim if (ly.rotary_dim <= 0 or ly.rotary_dim > ly.head_dim) else ly.rotary_dim
    hl = eff // 2 // 8
    return (eff // 2) % 8 == 0 and hl > 0 and (hl & (hl - 1)) == 0 and ly.head_dim in (64, 128, 256, 512)


def default_fuse(model):
    """Products that take their norms in a prologue by default. Every workgroup of a
    prologue product recomputes the input (norm statistics included) from x, the pending
    branch and both norm weights: worth it where that replaces a launch and the product's
    workgroups are few against its weight stream -- the QKV product (the previous layer's
    post-FFN norm + add and this layer's input norm), the per-layer-embedding gate (256
    rows) and projection (whose prologue is gelu(gate) * ple, no statistics). "attn" puts
    the QK-norm / RoPE / KV append inside the attention launch (one launch fewer per layer).
    Measured, graph decode step of the Gemma-4B-shaped model (34 x 2560, Q4_0), us per token,
    with "ple" and "attn": 1588-1610 alone; + QKV 1520-1534; + gate.up 1598-1610; + QKV and
    gate.up 1557; + those and the LM head 1582 (the gate.up product has 640 workgroups, each
    reading 40 KB of prologue operands beside its 46 KB of weights)."""
    return {"ple", "attn", "qkv"}


def cache_bytes(model, max_seq):
    """Device bytes of the f32 K and V caches for `model` at max_seq positions."""
    return 2 * 4 * len(model.layers) * max_seq * model.max_kv_dim

