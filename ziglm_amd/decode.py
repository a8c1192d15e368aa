"""One greedy decode step of a Gemma-shaped model, enqueued entirely on the device and
captured once as a hipGraph (the reference's graph decode, cuda_model.zig:1008-1080).

Per step, with the token id and position in device buffers:
  x = embedding row of the token * sqrt(H)                       (model.zig:494-503)
  xb = input RMSNorm(x)                                         (first layer only)
  per layer l:
    q, k, v = fused QKV GEMV(xb)                                 (cuda_model.zig:871-899)
    QK-RMSNorm + RoPE(pos) + K/V append to layer l's cache rows   (901-920)
    attn = decode attention over positions [0, pos]              (922-925)
    ao = O GEMV(attn)                                            (926-928)
    x += norm(ao; post_attn); xb = norm(x; pre_ffn)              (930-942)
    act = fused gate.up GeGLU GEMV(xb)                           (946-956)
    fo = down GEMV(act)                                          (958-960)
    x += norm(fo; post_ffn); xb = norm(x; next input norm, or the final norm)
  logits = LM head GEMV(xb) (tied embedding); soft-cap; token = greedy argmax (990-1005)
The argmax writes the token buffer the next step's embedding gather reads, so consecutive
replays decode autoregressively without the host; only the position is uploaded (an
ordered asynchronous copy on the same stream) before each replay.

Weights are synthetic (seeded Q4_0 rows; N(0, 0.1) norm weights), activations f32. This is
the host side of the decode path written over the C-ABI, as ziglm's cuda_model.zig is over
cuda.zig.
"""
import ctypes
import math

import numpy as np

from . import bridge as B
from . import synth
from .device import Graph
from .layer import GEMMA_4B


def q4_0_rows(seed, rows, cols, full=False):
    """Q4_0 bytes [rows, row_bytes]: all rows seeded (full) or 64 seeded rows to tile."""
    return synth.q4_0_table(seed, rows if full else min(rows, 64), cols)


class DecodeModel:
    def __init__(self, dev, shape=GEMMA_4B, n_layers=34, vocab=262144, max_seq=4096, seed=7,
                 final_softcap=30.0, attn_scale=1.0, host_weights=False):
        """host_weights: keep every weight on the host too (small models, for checking)."""
        s = self.shape = shape
        self.dev, self.L, self.V, self.max_seq = dev, n_layers, vocab, max_seq
        self.final_softcap, self.attn_scale = final_softcap, attn_scale
        H, I, qn, kn = s.H, s.I, s.nh * s.D, s.nkv * s.D
        self.host = {} if host_weights else None

        def qmat(name, rows, cols, sd):
            rb = cols // 32 * 18
            buf = dev.alloc(rows * rb)
            src = q4_0_rows(sd, rows, cols, full=host_weights)
            if host_weights:
                buf.upload(src.reshape(-1))
                self.host[name] = src
            else:
                self._tile(buf, src.reshape(-1))
            return buf

        def nvec(name, n, sd):
            w = synth.normal_f32(sd, name, (n,), 0, 0.1)
            if host_weights:
                self.host[name] = w
            return dev.from_numpy(w)

        self.emb = qmat("emb", vocab, H, seed)
        self.layers = []
        for l in range(n_layers):
            sd = seed * 1000 + 10 * l
            self.layers.append({
                "wq": qmat(f"wq{l}", qn, H, sd + 1), "wk": qmat(f"wk{l}", kn, H, sd + 2),
                "wv": qmat(f"wv{l}", kn, H, sd + 3), "wo": qmat(f"wo{l}", H, qn, sd + 4),
                "wg": qmat(f"wg{l}", I, H, sd + 5), "wu": qmat(f"wu{l}", I, H, sd + 6),
                "wd": qmat(f"wd{l}", H, I, sd + 7),
                "in": nvec(f"in{l}", H, sd + 8), "post_attn": nvec(f"post_attn{l}", H, sd + 8),
                "pre_ffn": nvec(f"pre_ffn{l}", H, sd + 8), "post_ffn": nvec(f"post_ffn{l}", H, sd + 8),
                "q_norm": nvec(f"q_norm{l}", s.D, sd + 9), "k_norm": nvec(f"k_norm{l}", s.D, sd + 9),
            })
        self.final_norm = nvec("final_norm", H, seed + 5)
        f4 = lambda n: dev.alloc(n * 4)  # noqa: E731
        self.x, self.xb, self.q, self.k, self.v = f4(H), f4(H), f4(qn), f4(kn), f4(kn)
        self.attn, self.ao, self.act, self.fo, self.logits = f4(qn), f4(H), f4(I), f4(H), f4(vocab)
        self.cache_rows = n_layers * max_seq
        self.kc, self.vc = f4(self.cache_rows * kn), f4(self.cache_rows * kn)
        self.kc.fill(0)
        self.vc.fill(0)
        self.token, self.pos = dev.alloc(16), dev.alloc(16)
        self.ws_bytes = dev.attentionWorkspaceBytes(1, s.nh, s.nkv, s.D, max_seq)
        self.ws = dev.alloc(max(self.ws_bytes, 16))
        self.graph = None

    def _tile(self, buf, src):
        n, first = buf.size_bytes, min(buf.size_bytes, src.nbytes)
        buf.upload(src[:first])
        done = first
        while done < n:
            c = min(done, n - done)
            buf.at(done).copy_from(buf, c)
            done += c

    def step_ops(self):
        """Enqueue one decode step on dev.stream (token and position read from the device)."""
        d, s = self.dev, self.shape
        H, I, qn, kn = s.H, s.I, s.nh * s.D, s.nkv * s.D
        d.embedGather(self.emb, B.Q4_0, self.V, self.token, B.F32, self.x, 1, H, math.sqrt(H))
        d.rmsNormRows(B.F32, self.x, self.layers[0]["in"], self.xb, 1, H, s.eps, s.uo)
        for l, w in enumerate(self.layers):
            d.gemvQkvQ4_0(w["wq"], w["wk"], w["wv"], self.xb, self.q, self.k, self.v, qn, kn, kn, H)
            d.qkNormRopeKv(B.F32, self.q, self.k, self.v, w["q_norm"], w["k_norm"], 0, self.kc, self.vc,
                           self.cache_rows, l, self.max_seq, kn, self.pos, 0, None, 1, s.nh, s.nkv, s.D, 0,
                           s.theta, 1.0, s.eps, s.uo)
            d.attentionDecode(B.F32, self.q, self.kc, self.vc, self.attn, self.cache_rows, kn, None,
                              l * self.max_seq, self.pos, 0, self.max_seq, 1, s.nh, s.nkv, s.D, self.attn_scale,
                              0.0, 0, self.ws, self.ws_bytes)
            d.gemv(B.Q4_0, w["wo"], self.attn, self.ao, H, qn)
            d.rmsNormAddRmsNorm(B.F32, self.x, self.ao, w["post_attn"], w["pre_ffn"], self.xb, 1, H, s.eps, s.uo)
            d.gemvGegluQ4_0(w["wg"], w["wu"], self.xb, self.act, I, H)
            d.gemv(B.Q4_0, w["wd"], self.act, self.fo, H, I)
            nxt = self.layers[l + 1]["in"] if l + 1 < self.L else self.final_norm
            d.rmsNormAddRmsNorm(B.F32, self.x, self.fo, w["post_ffn"], nxt, self.xb, 1, H, s.eps, s.uo)
        d.gemv(B.Q4_0, self.emb, self.xb, self.logits, self.V, H)
        d.tanhSoftcap(self.logits, self.final_softcap, self.V)
        d.argmax(self.logits, self.V, self.token)

    def capture(self):
        self.graph = Graph(self.dev, self.step_ops)
        return self.graph

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
        bufs = [self.emb, self.final_norm, self.x, self.xb, self.q, self.k, self.v, self.attn, self.ao,
                self.act, self.fo, self.logits, self.kc, self.vc, self.token, self.pos, self.ws]
        for w in self.layers:
            bufs.extend(w.values())
        for b in bufs:
            b.deinit()
