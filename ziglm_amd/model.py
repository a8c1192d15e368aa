"""Model weights as device tables: from a GGUF file (ziglm's TransformerModel.load,
model.zig:156-300, followed by the upload in cuda_model.zig:237-337) or synthetic.

`Model.from_gguf(dev, gguf_file)` resolves everything the decode step needs, with the
reference's rules:
  * tensor names and their alternates (model.zig:157-290): token_embd / output /
    output_norm, blk.N.{attn_norm, post_attention_norm | post_attn_norm, ffn_norm,
    post_ffw_norm | post_ffn_norm, post_norm | post_per_layer_input_norm,
    inp_gate | per_layer_input_gate, proj | per_layer_projection,
    layer_output_scale.weight | layer_scalar, attn_q, attn_k, attn_v, attn_output,
    attn_q_norm, attn_k_norm, ffn_gate, ffn_up, ffn_down}, and the per-layer-embedding
    (PLE) tables per_layer_token_embd | embed_tokens_per_layer, per_layer_model_proj |
    per_layer_model_projection, per_layer_proj_norm | per_layer_projection_norm;
  * per-layer head_dim from attn_q_norm's size, head counts from attn_q / attn_k sizes,
    intermediate size from ffn_gate (model.zig:246-290);
  * RoPE base, rotary dims and sliding window fixed by head_dim (model.zig:270-278):
    head_dim >= 512: base 1e6, 128 rotary dims, no window; else base 1e4, all dims, 512;
  * Gemma-4 cross-layer KV sharing (model.zig:600-616): layers from the unshared count
    on (or without attn_k) read the cache of the last unshared layer of equal head_dim
    and write none; their V gets the no-scale RMSNorm (model.zig:635-640);
  * attention scale 1 for gemma4, else 1/sqrt(head_dim) (model.zig:659); embedding scale
    sqrt(dim) for gemma, gemma2, gemma4 (model.zig:499-502); GeGLU for those, SwiGLU
    otherwise (model.zig:740-744).
Norm weights become f32 device vectors: F32 tensors are copied, other types are
dequantized on the device by the embedding-gather kernel (scale 1, exact), the device
form of model.zig:130-137 loadNorm. Weight matrices are uploaded as raw GGUF rows
(CudaGpuTensor.upload, cuda_model.zig:24-36) through the library's pinned-ring uploader.

Checks the reference does not make (they keep a kernel from reading past a table): every
matrix must hold exactly rows x cols of its type, with the sizes the decode step uses, and
have a type the GEMV and gather kernels take (F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q6_K).
Violations raise ModelError naming the tensor.
"""
import math
from dataclasses import dataclass, field

import numpy as np

from . import bridge as B
from . import gguf as G
from . import synth

GEMV_TYPES = (B.F32, B.F16, B.BF16, B.Q4_0, B.Q8_0, B.Q4_K, B.Q6_K)
GATHER_TYPES = GEMV_TYPES
PLE_DIM = 256  # per-layer embedding width (model.zig:508)


class ModelError(ValueError):
    pass


@dataclass
class Table:
    """A weight matrix on the device in GGUF row layout (CudaGpuTensor)."""
    qtype: int
    rows: int
    cols: int
    buf: object  # DeviceBuffer
    name: str = ""


@dataclass
class Layer:
    """LayerWeights (model.zig:10-45) on the device, with the resolved configuration."""
    index: int
    head_dim: int
    n_heads: int
    n_kv_heads: int
    intermediate_size: int
    rotary_dim: int
    rope_theta: float
    sliding_window: int
    attn_scale: float
    layer_scalar: float = 1.0
    v_norm: bool = False           # Gemma-4 no-scale V norm
    kv_shared: bool = False        # reads kv_layer's cache, writes none
    kv_layer: int = 0              # cache rows used by attention
    input_layernorm: object = None
    post_attention_layernorm: object = None
    pre_feedforward_layernorm: object = None
    post_feedforward_layernorm: object = None
    post_per_layer_input_norm: object = None
    attn_q_norm: object = None
    attn_k_norm: object = None
    attn_q: Table = None
    attn_k: Table = None
    attn_v: Table = None
    attn_output: Table = None
    ffn_gate: Table = None
    ffn_up: Table = None
    ffn_down: Table = None
    per_layer_input_gate: Table = None
    per_layer_projection: Table = None


@dataclass
class Model:
    """Device tables and resolved configuration of one model."""
    dev: object
    arch: str
    dim: int
    vocab: int
    eps: float
    unit_offset: bool
    embed_scale: float
    final_softcap: float
    attn_softcap: float
    rope_freq_scale: float
    activation: str  # "geglu" | "swiglu"
    token_embd: Table
    lm_head: Table
    output_norm: object
    layers: list
    ple_table: Table = None
    ple_proj: Table = None
    ple_proj_norm: object = None
    params: object = None
    host: dict = None  # host copies of the weights (synthetic models built for checking)
    _owned: list = field(default_factory=list)

    @property
    def max_kv_dim(self):
        return max(l.n_kv_heads * l.head_dim for l in self.layers)

    def free(self):
        for b in self._owned:
            b.deinit()
        self._owned = []

    # ---- GGUF -----------------------------------------------------------------------------
    @classmethod
    def from_gguf(cls, dev, f):
        """Resolve and upload the model in GGUFFile `f` (model.zig:156-300,
        cuda_model.zig:237-337)."""
        return _GgufLoader(dev, f).load()

    # ---- synthetic ----------------------------------------------------------------------
    @classmethod
    def synthetic(cls, dev, shape, n_layers, vocab, seed=7, final_softcap=30.0, attn_scale=1.0,
                  host_weights=False):
        """Q4_0 weights from seeded tables (q4_0_table rows; the 64 seeded rows tiled
        over each matrix unless host_weights), N(0, 0.1) norm weights, one RoPE base, no
        window, (1+w) norms: the fixed synthetic Gemma-shaped decode model."""
        s = shape
        H, I, qn, kn = s.H, s.I, s.nh * s.D, s.nkv * s.D
        owned, host = [], ({} if host_weights else None)

        def qmat(name, rows, cols, sd):
            src = synth.q4_0_table(sd, rows if host_weights else min(rows, 64), cols)
            buf = dev.alloc(rows * (cols // 32 * 18))
            owned.append(buf)
            if host_weights:
                buf.upload(src.reshape(-1))
                host[name] = src
            else:
                _tile(buf, src.reshape(-1))
            return Table(B.Q4_0, rows, cols, buf, name)

        def nvec(name, n, sd):
            w = synth.normal_f32(sd, name, (n,), 0, 0.1)
            if host_weights:
                host[name] = w
            buf = dev.from_numpy(w)
            owned.append(buf)
            return buf

        emb = qmat("emb", vocab, H, seed)
        layers = []
        for l in range(n_layers):
            sd = seed * 1000 + 10 * l
            layers.append(Layer(
                index=l, head_dim=s.D, n_heads=s.nh, n_kv_heads=s.nkv, intermediate_size=I, rotary_dim=s.D,
                rope_theta=s.theta, sliding_window=0, attn_scale=attn_scale, kv_layer=l,
                attn_q=qmat(f"wq{l}", qn, H, sd + 1), attn_k=qmat(f"wk{l}", kn, H, sd + 2),
                attn_v=qmat(f"wv{l}", kn, H, sd + 3), attn_output=qmat(f"wo{l}", H, qn, sd + 4),
                ffn_gate=qmat(f"wg{l}", I, H, sd + 5), ffn_up=qmat(f"wu{l}", I, H, sd + 6),
                ffn_down=qmat(f"wd{l}", H, I, sd + 7),
                input_layernorm=nvec(f"in{l}", H, sd + 8), post_attention_layernorm=nvec(f"post_attn{l}", H, sd + 8),
                pre_feedforward_layernorm=nvec(f"pre_ffn{l}", H, sd + 8),
                post_feedforward_layernorm=nvec(f"post_ffn{l}", H, sd + 8),
                attn_q_norm=nvec(f"q_norm{l}", s.D, sd + 9), attn_k_norm=nvec(f"k_norm{l}", s.D, sd + 9)))
        final = nvec("final_norm", H, seed + 5)
        return cls(dev=dev, arch="synthetic", dim=H, vocab=vocab, eps=s.eps, unit_offset=s.uo,
                   embed_scale=float(np.float32(math.sqrt(H))), final_softcap=final_softcap, attn_softcap=0.0,
                   rope_freq_scale=1.0, activation="geglu", token_embd=emb, lm_head=emb, output_norm=final,
                   layers=layers, host=host, _owned=owned)


def _tile(buf, src):
    """Fill `buf` with repeats of `src` (device-side doubling copies)."""
    n, first = buf.size_bytes, min(buf.size_bytes, src.nbytes)
    buf.upload(src[:first])
    done = first
    while done < n:
        c = min(done, n - done)
        buf.at(done).copy_from(buf, c)
        done += c


def _row_bytes(qtype, cols):
    return cols // G.block_size(qtype) * G.type_size(qtype)


class _GgufLoader:
    def __init__(self, dev, f):
        self.dev, self.f = dev, f
        self.owned = []
        self.uploads = []       # (tensor, device buffer)
        self.converts = []      # (raw buffer, qtype, n, f32 buffer): norms to dequantize

    def get(self, *names):
        for n in names:
            t = self.f.getTensor(n)
            if t is not None:
                return t
        return None

    def alloc(self, nbytes):
        b = self.dev.alloc(nbytes)
        self.owned.append(b)
        return b

    def table(self, t, rows, cols, types=GEMV_TYPES):
        """Upload t as a rows x cols matrix, after checking it holds exactly that."""
        if t is None:
            return None
        if t.type not in types:
            raise ModelError(f"{t.name}: GGML type {t.type} is not supported here (supported: {types})")
        if cols % G.block_size(t.type) or t.size_bytes != rows * _row_bytes(t.type, cols) or t.shape[0] != cols:
            raise ModelError(f"{t.name}: shape {t.shape[:t.n_dims]} / {t.size_bytes} bytes is not {rows} x {cols}")
        buf = self.alloc(t.size_bytes)
        self.uploads.append((t, buf))
        return Table(t.type, rows, cols, buf, t.name)

    def norm(self, t, n=None):
        """loadNorm (model.zig:130-137): t dequantized to f32[n or elements]."""
        if t is None:
            return None
        n = n if n is not None else (t.elements() or 1)
        if t.type not in GATHER_TYPES or n % G.block_size(t.type) or \
                t.size_bytes < n // G.block_size(t.type) * G.type_size(t.type):
            raise ModelError(f"{t.name}: norm of type {t.type} with {t.elements()} elements cannot give {n}")
        out = self.alloc(4 * n)
        if t.type == B.F32 and t.size_bytes == 4 * n:
            self.uploads.append((t, out))
        else:  # raw bytes to a scratch buffer, then dequantize the first n elements
            raw = self.dev.alloc(t.size_bytes)
            self.uploads.append((t, raw))
            self.converts.append((raw, t.type, n, out))
        return out

    @staticmethod
    def scalar(t):
        """loadScalar (model.zig:139-154)."""
        if t is None:
            return 1.0
        d = t.data
        if t.type == B.BF16 and d.size >= 2:
            return float((np.frombuffer(d[:2].tobytes(), np.uint16).astype(np.uint32) << 16).view(np.float32)[0])
        if t.type == B.F16 and d.size >= 2:
            return float(np.frombuffer(d[:2].tobytes(), np.float16)[0])
        if t.type == B.F32 and d.size >= 4:
            return float(np.frombuffer(d[:4].tobytes(), np.float32)[0])
        return 1.0

    def load(self):
        f, p = self.f, self.f.params
        dim = p.embedding_length
        emb_t = self.get("token_embd.weight")
        if emb_t is None:
            raise ModelError("MissingTokenEmbeddingTensor")
        out_norm_t = self.get("output_norm.weight")
        if out_norm_t is None:
            raise ModelError("MissingOutputNormTensor")
        gemma = p.arch in G.GEMMA_ARCHS
        try:
            raw_layers = [self._layer_tensors(i) for i in range(p.block_count)]
            layers = self._resolve(raw_layers, p, dim)
            L = len(layers)
            output_t = self.get("output.weight")
            vocab = p.vocab_size
            lm_head = self.table(output_t, vocab, dim) if output_t is not None else None
            emb = self.table(emb_t, vocab, dim, GATHER_TYPES if lm_head is not None else GEMV_TYPES)
            if lm_head is None:
                lm_head = emb  # tied (model.zig:797-800)
            ple_t = self.get("per_layer_token_embd.weight", "embed_tokens_per_layer.weight")
            ple = self.table(ple_t, vocab, L * PLE_DIM, GATHER_TYPES) if ple_t is not None else None
            proj_t = self.get("per_layer_model_proj.weight", "per_layer_model_projection.weight")
            ple_proj = self.table(proj_t, L * PLE_DIM, dim) if proj_t is not None else None
            ple_norm = self.norm(self.get("per_layer_proj_norm.weight", "per_layer_projection_norm.weight"))
            output_norm = self.norm(out_norm_t, dim)
            self._upload()
        except Exception:
            for b in self.owned:
                b.deinit()
            raise
        m = Model(dev=self.dev, arch=p.arch, dim=dim, vocab=p.vocab_size, eps=p.layer_norm_rms_epsilon,
                  unit_offset=p.use_gemma_rms_unit_offset,
                  embed_scale=float(np.sqrt(np.float32(dim))) if gemma else 1.0,
                  final_softcap=p.final_logit_softcapping, attn_softcap=p.attn_logit_softcapping,
                  rope_freq_scale=p.rope_freq_scale, activation="geglu" if gemma else "swiglu",
                  token_embd=emb, lm_head=lm_head, output_norm=output_norm, layers=layers, ple_table=ple,
                  ple_proj=ple_proj, ple_proj_norm=ple_norm, params=p, _owned=self.owned)
        return m

    def _layer_tensors(self, i):
        g = lambda *names: self.get(*[f"blk.{i}.{n}" for n in names])  # noqa: E731
        return {
            "attn_norm": g("attn_norm.weight"), "post_attn": g("post_attention_norm.weight", "post_attn_norm.weight"),
            "ffn_norm": g("ffn_norm.weight"), "post_ffn": g("post_ffw_norm.weight", "post_ffn_norm.weight"),
            "post_ple": g("post_norm.weight", "post_per_layer_input_norm.weight"),
            "ple_gate": g("inp_gate.weight", "per_layer_input_gate.weight"),
            "ple_proj": g("proj.weight", "per_layer_projection.weight"),
            "scalar": g("layer_output_scale.weight", "layer_scalar"),
            "q": g("attn_q.weight"), "k": g("attn_k.weight"), "v": g("attn_v.weight"),
            "o": g("attn_output.weight"), "q_norm": g("attn_q_norm.weight"), "k_norm": g("attn_k_norm.weight"),
            "gate": g("ffn_gate.weight"), "up": g("ffn_up.weight"), "down": g("ffn_down.weight"),
        }

    def _resolve(self, raw, p, dim):
        L = len(raw)
        cfg = []
        for i, t in enumerate(raw):
            head_dim = t["q_norm"].elements() if t["q_norm"] is not None else p.head_size
            if head_dim <= 0:
                raise ModelError(f"blk.{i}: head_dim 0")
            n_heads = t["q"].elements() // dim // head_dim if t["q"] is not None else p.head_count
            if t["k"] is not None:
                n_kv = t["k"].elements() // dim // head_dim
            else:
                n_kv = p.head_count_kv if p.head_count_kv > 0 else n_heads
            inter = t["gate"].elements() // dim if t["gate"] is not None else p.feed_forward_length
            big = head_dim >= 512
            cfg.append((head_dim, n_heads, n_kv, inter, 1e6 if big else 1e4, 128 if big else head_dim,
                        0 if big else 512))
        # cross-layer KV sharing (model.zig:600-616)
        if p.num_kv_shared_layers > 0:
            unshared = p.block_count - p.num_kv_shared_layers
        elif p.arch == "gemma4":
            unshared = 24 if p.block_count == 42 else 15
        else:
            unshared = p.block_count
        gemma4 = p.arch == "gemma4"
        layers = []
        for i, t in enumerate(raw):
            head_dim, n_heads, n_kv, inter, theta, rot, win = cfg[i]
            shared = gemma4 and (t["k"] is None or i >= unshared)
            donor = i
            if shared:
                for l in range(min(unshared, L) - 1, -1, -1):
                    if cfg[l][0] == head_dim:
                        donor = l
                        break
            attn_scale = 1.0 if gemma4 else float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
            qn, kn = n_heads * head_dim, n_kv * head_dim
            ly = Layer(index=i, head_dim=head_dim, n_heads=n_heads, n_kv_heads=n_kv, intermediate_size=inter,
                       rotary_dim=rot, rope_theta=theta, sliding_window=win, attn_scale=attn_scale,
                       layer_scalar=self.scalar(t["scalar"]), v_norm=gemma4, kv_shared=shared, kv_layer=donor)
            ly.input_layernorm = self.norm(t["attn_norm"], None)
            ly.post_attention_layernorm = self.norm(t["post_attn"], None)
            ly.pre_feedforward_layernorm = self.norm(t["ffn_norm"], None)
            ly.post_feedforward_layernorm = self.norm(t["post_ffn"], None)
            ly.post_per_layer_input_norm = self.norm(t["post_ple"], None)
            ly.attn_q_norm = self.norm(t["q_norm"], head_dim)
            ly.attn_k_norm = self.norm(t["k_norm"], None)
            for nm, v in (("input_layernorm", ly.input_layernorm), ("post_attention_layernorm",
                                                                     ly.post_attention_layernorm),
                          ("pre_feedforward_layernorm", ly.pre_feedforward_layernorm),
                          ("post_feedforward_layernorm", ly.post_feedforward_layernorm),
                          ("post_per_layer_input_norm", ly.post_per_layer_input_norm)):
                if v is not None and v.size_bytes < 4 * dim:
                    raise ModelError(f"blk.{i}.{nm}: fewer than {dim} weights")
            if ly.attn_k_norm is not None and ly.attn_k_norm.size_bytes < 4 * head_dim:
                raise ModelError(f"blk.{i}.attn_k_norm: fewer than {head_dim} weights")
            ly.attn_q = self.table(t["q"], qn, dim)
            if not shared:
                ly.attn_k = self.table(t["k"], kn, dim)
                ly.attn_v = self.table(t["v"], kn, dim)
            ly.attn_output = self.table(t["o"], dim, qn)
            ly.ffn_gate = self.table(t["gate"], inter, dim)
            ly.ffn_up = self.table(t["up"], inter, dim)
            ly.ffn_down = self.table(t["down"], dim, inter)
            ly.per_layer_input_gate = self.table(t["ple_gate"], PLE_DIM, dim)
            ly.per_layer_projection = self.table(t["ple_proj"], dim, PLE_DIM)
            layers.append(ly)
        return layers

    def _upload(self):
        if self.uploads:
            self.f.upload([t for t, _ in self.uploads], [b for _, b in self.uploads], self.dev.stream)
        if self.converts:
            ids = self.dev.from_numpy(np.zeros(1, np.int32))
            for raw, qtype, n, out in self.converts:
                self.dev.embedGather(raw, qtype, 1, ids, B.F32, out, 1, n, 1.0)
            self.dev.sync()
            ids.deinit()
            for raw, _, _, _ in self.converts:
                raw.deinit()
        self.dev.sync()
