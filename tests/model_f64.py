"""An independent float64 forward pass of a Gemma-family GGUF model, from the model's
mathematical definition (not from ziglm's code): block dequantization written out from
the GGUF block layouts, RMSNorm x / sqrt(mean(x^2) + eps) * w (or 1 + w), half-split
RoPE with angle pos * base^(-2i / r), softmax attention over the window, tanh-GELU,
per-layer embeddings, tanh soft-cap. It checks the oracle's f32 restatement
(oracle/model_ref.py) on small models: a dropped norm, a wrong RoPE base or rotary
width, a wrong KV donor or a mis-wired PLE term moves the logits far outside the f32
rounding of a few dozen ops.

The configuration (head sizes, RoPE base / rotary width / window by head size, KV
donors) is taken from a RefModel so that the two differ only in arithmetic.
"""
import numpy as np


def dequant(t, rows=None):
    """f64 values of a tensor record of RefModel.t (rows x cols when rows is given)."""
    raw, typ = t["raw"], t["type"]
    if typ == 0:
        v = raw.view(np.float32).astype(np.float64)
    elif typ == 1:
        v = raw.view(np.float16).astype(np.float64)
    elif typ == 30:
        v = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    elif typ == 8:  # Q8_0: f16 d, 32 x int8
        b = raw.reshape(-1, 34)
        d = b[:, :2].copy().view(np.float16).astype(np.float64)
        v = (b[:, 2:].view(np.int8).astype(np.float64) * d).reshape(-1)
    elif typ == 2:  # Q4_0: f16 d, 16 bytes: low nibbles are elements 0..15, high 16..31, minus 8
        b = raw.reshape(-1, 18)
        d = b[:, :2].copy().view(np.float16).astype(np.float64)
        q = b[:, 2:]
        vals = np.concatenate([(q & 15).astype(np.float64), (q >> 4).astype(np.float64)], axis=1) - 8.0
        v = (vals * d).reshape(-1)
    else:
        raise ValueError(f"type {typ}")
    return v if rows is None else v.reshape(rows, -1)


def rms(x, w, eps, unit_offset):
    y = x / np.sqrt(np.mean(x * x) + eps)
    if w is None:
        return y
    return y * ((1.0 + w) if unit_offset else w)


def rope(h, pos, r, base):
    h = h.copy()
    half = r // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos * base ** (-2.0 * i / r)
    c, s = np.cos(ang), np.sin(ang)
    a, b = h[:half].copy(), h[half:r].copy()
    h[:half] = a * c - b * s
    h[half:r] = a * s + b * c
    return h


def gelu(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


class F64Model:
    def __init__(self, ref):
        """ref: a RefModel over the same file (tensor records and configuration)."""
        self.ref = ref
        L = len(ref.layers)
        self.kc = np.zeros((L, ref.max_seq, ref.kv_dim))
        self.vc = np.zeros_like(self.kc)

    def norm_w(self, w):
        return None if w is None else np.asarray(w, np.float64)

    def forward(self, token, pos):
        r = self.ref
        p, dim, eps, uo = r.p, r.dim, float(r.eps), r.uo
        L = len(r.layers)
        x = dequant(r.token_embd, r.V)[token]
        if r.gemma:
            x = x * np.sqrt(dim)
        ple = None
        if r.ple is not None:
            ple = dequant(r.ple, r.V)[token] * 16.0
            if r.ple_proj is not None:
                ctx = dequant(r.ple_proj, L * 256) @ (x / np.sqrt(dim))
                if r.ple_norm is not None:
                    for l in range(L):
                        s = rms(ctx[l * 256:(l + 1) * 256], self.norm_w(r.ple_norm), eps, False)
                        ple[l * 256:(l + 1) * 256] = (ple[l * 256:(l + 1) * 256] + s) / np.sqrt(2.0)
        for i, ly in enumerate(r.layers):
            hd, nh, nkv = ly["head_dim"], ly["n_heads"], ly["n_kv"]
            W = lambda key, rows: dequant({"raw": ly[key][1].reshape(-1), "type": ly[key][0]}, rows)  # noqa: E731
            xb = rms(x, self.norm_w(ly["in"]), eps, uo) if ly["in"] is not None else x.copy()
            q = (W("q", nh * hd) @ xb).reshape(nh, hd)
            if ly["q_norm"] is not None:
                q = np.stack([rms(h, self.norm_w(ly["q_norm"]), eps, uo) for h in q])
            q = np.stack([rope(h, pos, ly["rotary"], ly["theta"]) for h in q])
            if not ly["shared"]:
                k = (W("k", nkv * hd) @ xb).reshape(nkv, hd)
                v = (W("v", nkv * hd) @ xb).reshape(nkv, hd)
                if ly["k_norm"] is not None:
                    k = np.stack([rms(h, self.norm_w(ly["k_norm"]), eps, uo) for h in k])
                if r.arch == "gemma4":
                    v = np.stack([rms(h, None, eps, uo) for h in v])
                k = np.stack([rope(h, pos, ly["rotary"], ly["theta"]) for h in k])
                self.kc[i, pos, :nkv * hd] = k.reshape(-1)
                self.vc[i, pos, :nkv * hd] = v.reshape(-1)
            scale = 1.0 if r.arch == "gemma4" else 1.0 / np.sqrt(hd)
            start = pos + 1 - ly["window"] if ly["window"] > 0 and pos + 1 > ly["window"] else 0
            d = ly["donor"]
            out = np.zeros((nh, hd))
            for h in range(nh):
                kh = h // (nh // nkv)
                K = self.kc[d, start:pos + 1, kh * hd:(kh + 1) * hd]
                V = self.vc[d, start:pos + 1, kh * hd:(kh + 1) * hd]
                s = (K @ q[h]) * scale
                w = np.exp(s - s.max())
                out[h] = (w / w.sum()) @ V
            ao = W("o", dim) @ out.reshape(-1)
            if ly["post_attn"] is not None:
                ao = rms(ao, self.norm_w(ly["post_attn"]), eps, uo)
            x = x + ao
            xb = rms(x, self.norm_w(ly["pre_ffn"]), eps, uo) if ly["pre_ffn"] is not None else x.copy()
            act = gelu(W("gate", ly["inter"]) @ xb) * (W("up", ly["inter"]) @ xb)
            fo = W("down", dim) @ act
            if ly["post_ffn"] is not None:
                fo = rms(fo, self.norm_w(ly["post_ffn"]), eps, uo)
            x = x + fo
            if ple is not None and ly["ple_gate"] is not None and ly["ple_proj"] is not None:
                g = gelu(W("ple_gate", 256) @ x)
                dx = W("ple_proj", dim) @ (ple[i * 256:(i + 1) * 256] * g)
                if ly["post_ple"] is not None:
                    dx = rms(dx, self.norm_w(ly["post_ple"]), eps, False)
                x = x + dx
            x = x * ly["scalar"]
        xb = rms(x, self.norm_w(r.output_norm), eps, uo)
        head = r.output if r.output is not None else r.token_embd
        logits = dequant(head, r.V) @ xb
        cap = p["final_logit_softcapping"]
        if cap > 0:
            logits = cap * np.tanh(logits / cap)
        return logits
