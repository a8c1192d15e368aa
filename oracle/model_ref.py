"""CPU restatement of ziglm's model load and one-token forward pass (src/model.zig
TransformerModel.load 156-300 and forward 486-812, greedy sampler sampler.zig:158-170)
over a GGUF image parsed by oracle/gguf_ref.py, computed with the oracle's ops
(oracle.py). Test infrastructure only: the decode tests run it beside the device decode
step on the same file.

It reads tensors with the restated parser (not the library's reader) and resolves the
per-layer configuration on its own, so a mistake in the product's loader (a wrong
alternate name, head count, RoPE base, window, KV donor or PLE wiring) shows up as a
different forward pass.
"""
import struct

import numpy as np

from . import gguf_ref as R

PLE_DIM = 256


def _f32(x):
    return float(np.float32(x))


class RefModel:
    def __init__(self, o, data, max_seq):
        """o: Oracle; data: the GGUF bytes; max_seq: KV-cache rows per layer."""
        self.o, self.buf = o, bytes(data)
        f = self.f = R.parse(self.buf)
        p = self.p = f["params"]
        self.tensors = {t[0].decode(): t for t in f["tensors"]}  # last duplicate wins
        dim = self.dim = p["embedding_length"]
        self.arch = p["arch"]
        self.gemma = self.arch in ("gemma", "gemma2", "gemma4")
        self.uo = p["use_gemma_rms_unit_offset"]
        self.eps = np.float32(p["layer_norm_rms_epsilon"])
        self.V = p["vocab_size"]
        self.token_embd = self.t("token_embd.weight")
        self.output = self.t("output.weight")
        self.output_norm = self.norm(self.t("output_norm.weight"), dim)
        self.ple = self.t("per_layer_token_embd.weight", "embed_tokens_per_layer.weight")
        self.ple_proj = self.t("per_layer_model_proj.weight", "per_layer_model_projection.weight")
        self.ple_norm = self.norm(self.t("per_layer_proj_norm.weight", "per_layer_projection_norm.weight"), PLE_DIM)
        self.layers = [self.layer(i) for i in range(p["block_count"])]
        # KV sharing (model.zig:600-616)
        L = len(self.layers)
        if p.get("num_kv_shared_layers", 0) > 0:
            unshared = p["block_count"] - p["num_kv_shared_layers"]
        elif self.arch == "gemma4":
            unshared = 24 if p["block_count"] == 42 else 15
        else:
            unshared = p["block_count"]
        for i, ly in enumerate(self.layers):
            ly["shared"] = self.arch == "gemma4" and (ly["k"] is None or i >= unshared)
            ly["donor"] = i
            if ly["shared"]:
                for l in range(min(unshared, L) - 1, -1, -1):
                    if self.layers[l]["head_dim"] == ly["head_dim"]:
                        ly["donor"] = l
                        break
        self.max_seq = max_seq
        self.kv_dim = max(l["n_kv"] * l["head_dim"] for l in self.layers)
        self.kc = np.zeros((L * max_seq, self.kv_dim), np.float32)
        self.vc = np.zeros_like(self.kc)

    # ---- tensors --------------------------------------------------------------------------
    def t(self, *names):
        """(type, shape, n_dims, raw bytes) of the first present name, or None."""
        for n in names:
            rec = self.tensors.get(n)
            if rec is not None:
                _, typ, nd, shape, off, size = rec
                a = self.f["data_offset"] + off
                return {"type": typ, "shape": shape, "n_dims": nd, "raw": np.frombuffer(self.buf, np.uint8, size, a)}
        return None

    @staticmethod
    def elements(t):
        n = 1
        for d in t["shape"][:t["n_dims"]]:
            n *= d
        return n

    def norm(self, t, n):
        """loadNorm (model.zig:130-137): elements (or n) values dequantized."""
        if t is None:
            return None
        act = self.elements(t) or n
        return self.o.dequantize_row(t["type"], t["raw"], act)

    def mat(self, t, rows):
        return None if t is None else (t["type"], t["raw"].reshape(rows, -1))

    def layer(self, i):
        dim, p = self.dim, self.p
        g = lambda *names: self.t(*[f"blk.{i}.{n}" for n in names])  # noqa: E731
        q_norm_t = g("attn_q_norm.weight")
        head_dim = self.elements(q_norm_t) if q_norm_t is not None else p["head_size"]
        q_t, k_t, gate_t = g("attn_q.weight"), g("attn_k.weight"), g("ffn_gate.weight")
        n_heads = self.elements(q_t) // dim // head_dim if q_t is not None else p["head_count"]
        n_kv = self.elements(k_t) // dim // head_dim if k_t is not None else (p["head_count_kv"] or n_heads)
        inter = self.elements(gate_t) // dim if gate_t is not None else p["feed_forward_length"]
        big = head_dim >= 512
        scalar_t = g("layer_output_scale.weight", "layer_scalar")
        scalar = 1.0
        if scalar_t is not None:  # loadScalar (model.zig:139-154)
            raw = scalar_t["raw"].tobytes()
            if scalar_t["type"] == 30 and len(raw) >= 2:
                scalar = struct.unpack("<f", b"\0\0" + raw[:2])[0]
            elif scalar_t["type"] == 1 and len(raw) >= 2:
                scalar = float(np.frombuffer(raw[:2], np.float16)[0])
            elif scalar_t["type"] == 0 and len(raw) >= 4:
                scalar = struct.unpack("<f", raw[:4])[0]
        return {
            "head_dim": head_dim, "n_heads": n_heads, "n_kv": n_kv, "inter": inter,
            "theta": 1e6 if big else 1e4, "rotary": 128 if big else head_dim, "window": 0 if big else 512,
            "scalar": scalar,
            "in": self.norm(g("attn_norm.weight"), dim),
            "post_attn": self.norm(g("post_attention_norm.weight", "post_attn_norm.weight"), dim),
            "pre_ffn": self.norm(g("ffn_norm.weight"), dim),
            "post_ffn": self.norm(g("post_ffw_norm.weight", "post_ffn_norm.weight"), dim),
            "post_ple": self.norm(g("post_norm.weight", "post_per_layer_input_norm.weight"), dim),
            "q_norm": self.norm(q_norm_t, head_dim), "k_norm": self.norm(g("attn_k_norm.weight"), head_dim),
            "q": self.mat(q_t, n_heads * head_dim), "k": self.mat(k_t, n_kv * head_dim),
            "v": self.mat(g("attn_v.weight"), n_kv * head_dim), "o": self.mat(g("attn_output.weight"), dim),
            "gate": self.mat(gate_t, inter), "up": self.mat(g("ffn_up.weight"), inter),
            "down": self.mat(g("ffn_down.weight"), dim),
            "ple_gate": self.mat(g("inp_gate.weight", "per_layer_input_gate.weight"), PLE_DIM),
            "ple_proj": self.mat(g("proj.weight", "per_layer_projection.weight"), dim),
        }

    # ---- forward (model.zig:486-812) ---------------------------------------------------------
    def gemv(self, m, x):
        return self.o.gemv(m[0], m[1], x)

    def rms(self, x, w, uo=None):
        return self.o.rms_norm(x, w, self.eps, self.uo if uo is None else uo)

    def forward(self, token, pos):
        """Logits (after the final soft-cap) for `token` at `pos`; updates the KV cache."""
        o, dim, p = self.o, self.dim, self.p
        L = len(self.layers)
        e = self.token_embd
        x = o.dequantize_row(e["type"], e["raw"].reshape(self.V, -1)[token], dim)
        if self.gemma:
            x = (x * np.float32(np.sqrt(np.float32(dim)))).astype(np.float32)
        ple = None
        if self.ple is not None:  # model.zig:506-540 (token path)
            n = L * PLE_DIM
            row = o.dequantize_row(self.ple["type"], self.ple["raw"].reshape(self.V, -1)[token], n)
            pq, pw = self.mat(self.ple_proj, n) if self.ple_proj is not None else (None, None)
            ple = o.ple_token_inputs(row, x, pq, pw, self.ple_norm, L, self.eps, ple_dim=PLE_DIM)
        for i, ly in enumerate(self.layers):
            hd, nh, nkv = ly["head_dim"], ly["n_heads"], ly["n_kv"]
            xb = self.rms(x, ly["in"]) if ly["in"] is not None else x.copy()
            q = self.gemv(ly["q"], xb)
            if ly["q_norm"] is not None:
                q = self.rms(q.reshape(nh, hd), ly["q_norm"]).reshape(-1)
            if not ly["shared"]:
                k = self.gemv(ly["k"], xb)
                v = self.gemv(ly["v"], xb)
                q = o.qk_norm_rope_kv(q, k, v, None, ly["k_norm"], self.kc, self.vc, v_norm=self.arch == "gemma4",
                                      layer=i, max_seq=self.max_seq, max_kv_dim=self.kv_dim,
                                      pos=np.array([pos], np.int32), n_heads=nh, n_kv_heads=nkv, head_dim=hd,
                                      rotary_dim=ly["rotary"], base=ly["theta"], freq_scale=p["rope_freq_scale"],
                                      eps=self.eps, unit_offset=self.uo)
            else:
                q, _ = o.apply_rope(q, None, pos, hd, ly["rotary"], nh, 0, ly["theta"], p["rope_freq_scale"])
            scale = 1.0 if self.arch == "gemma4" else _f32(np.float32(1.0) / np.sqrt(np.float32(hd)))
            attn = o.attention(q, self.kc, self.vc, ly["donor"] * self.max_seq, pos, nh, nkv, hd, scale, 0.0,
                               ly["window"])
            ao = self.gemv(ly["o"], attn)
            if ly["post_attn"] is not None:
                ao = self.rms(ao, ly["post_attn"])
            x = (x + ao).astype(np.float32)
            xb = self.rms(x, ly["pre_ffn"]) if ly["pre_ffn"] is not None else x.copy()
            act = o.geglu(self.gemv(ly["gate"], xb), self.gemv(ly["up"], xb))
            fo = self.gemv(ly["down"], act)
            if ly["post_ffn"] is not None:
                fo = self.rms(fo, ly["post_ffn"])
            x = (x + fo).astype(np.float32)
            if ple is not None and ly["ple_gate"] is not None and ly["ple_proj"] is not None:  # 757-781
                x = o.ple_inject(x, ple[i * PLE_DIM:(i + 1) * PLE_DIM], *ly["ple_gate"], *ly["ple_proj"],
                                 ly["post_ple"], self.eps)
            if ly["scalar"] != 1.0:
                x = (x * np.float32(ly["scalar"])).astype(np.float32)
        xb = self.rms(x, self.output_norm)
        head = self.output if self.output is not None else self.token_embd
        logits = self.gemv(self.mat(head, self.V), xb)
        cap = p["final_logit_softcapping"]
        if cap > 0.0:
            logits = o.softcap(logits, cap)
        return logits
