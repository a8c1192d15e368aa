"""ctypes front end of the CPU oracle (oracle/ziglm_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package. Arrays are numpy; bf16 tensors are
numpy uint16 bit patterns.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30

_fp = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_f = ctypes.c_float
_i = ctypes.c_int

_SIGS = {
    "zo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "zo_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "zo_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
    "zo_bf16_to_f32_n": (None, [_u16p, _fp, _sz]),
    "zo_f32_to_bf16_n": (None, [_fp, _u16p, _sz]),
    "zo_row_bytes": (_sz, [_i, _sz]),
    "zo_dequantize_row": (_i, [_i, _u8p, _fp, _sz]),
    "zo_embed_gather": (_i, [_u8p, _i, _i32p, _sz, _sz, _f, _fp]),
    "zo_rms_norm": (None, [_fp, _fp, _fp, _sz, _f, _i]),
    "zo_rms_norm_no_scale": (None, [_fp, _fp, _sz, _f]),
    "zo_add": (None, [_fp, _fp, _sz]),
    "zo_add_rms_norm": (None, [_fp, _fp, _fp, _fp, _sz, _f, _i]),
    "zo_rms_norm_add": (None, [_fp, _fp, _fp, _sz, _f, _i]),
    "zo_rope_denominator": (ctypes.c_float, [_f, _sz, _sz]),
    "zo_rope_cos_sin": (None, [_f, _f, _fp, _fp]),
    "zo_apply_rope": (None, [_fp, _fp, _sz, _sz, _sz, _sz, _sz, _f, _f, _i]),
    "zo_kv_cache_put": (None, [_fp, _fp, _fp, _fp, _sz, _sz, _sz, _sz, _sz, _sz]),
    "zo_qk_norm_rope_kv_token": (
        None, [_fp, _fp, _fp, _fp, _fp, _i, _sz, _sz, _sz, _sz, _sz, _f, _f, _f, _i]),
    "zo_expm1f": (ctypes.c_float, [_f]),
    "zo_tanhf": (ctypes.c_float, [_f]),
    "zo_gelu": (ctypes.c_float, [_f]),
    "zo_geglu": (None, [_fp, _fp, _fp, _sz]),
    "zo_softcap": (None, [_fp, _f, _sz]),
    "zo_silu": (ctypes.c_float, [_f]),
    "zo_swiglu": (None, [_fp, _fp, _fp, _sz]),
    "zo_swiglu_bf16": (None, [_u16p, _u16p, _u16p, _sz]),
    "zo_ple_gate_gelu": (None, [_fp, _fp, _fp, _sz]),
    "zo_ple_ctx_fuse": (None, [_fp, _fp, _sz, _i]),
    "zo_add_rms_norm_bf16": (None, [_u16p, _u16p, _fp, _u16p, _sz, _sz, _f, _i]),
    "zo_rms_norm_bf16": (None, [_u16p, _fp, _u16p, _sz, _sz, _f, _i]),
    "zo_rms_norm_add_rms_norm_bf16": (None, [_u16p, _u16p, _fp, _fp, _sz, _sz, _f, _i]),
    "zo_rms_norm_add_rms_norm": (None, [_fp, _fp, _fp, _fp, _sz, _sz, _f, _i]),
    "zo_rms_norm_add_bf16": (None, [_u16p, _u16p, _fp, _sz, _sz, _f, _i]),
    "zo_geglu_bf16": (None, [_u16p, _u16p, _u16p, _sz]),
    "zo_dot_f32": (ctypes.c_float, [_fp, _fp, _sz]),
    "zo_dot_q8_0": (ctypes.c_float, [_u8p, _fp, _sz]),
    "zo_dot_q4_0": (ctypes.c_float, [_u8p, _fp, _sz]),
    "zo_dot_q4_k": (ctypes.c_float, [_u8p, _fp, _sz]),
    "zo_dot_q6_k": (ctypes.c_float, [_u8p, _fp, _sz]),
    "zo_dot_row": (ctypes.c_float, [_i, _u8p, _fp, _sz]),
    "zo_gemv": (_i, [_i, _u8p, _fp, _fp, _sz, _sz]),
    "zo_gemm": (_i, [_i, _u8p, _fp, _fp, _sz, _sz, _sz]),
    "zo_argmax": (ctypes.c_uint32, [_fp, _sz]),
    "zo_attention_token": (_i, [_fp, _vp, _vp, _i, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f, _fp]),
    "zo_qk_norm_rope_kv": (
        None,
        [_i, _vp, _vp, _vp, _fp, _fp, _i, _vp, _vp, _sz, _sz, _sz, _i32p, ctypes.c_int64, _i64p,
         _sz, _sz, _sz, _sz, _sz, _f, _f, _f, _i]),
}


class Oracle:
    """Typed handle on one build of the oracle library."""

    def __init__(self, simd=False):
        name = "liboracle_simd.so" if simd else "liboracle.so"
        # ZIGLM_ORACLE_LIB: another build of the same sources (the sanitizer build of
        # tests/asan) for both roles
        path = os.environ.get("ZIGLM_ORACLE_LIB") or os.path.join(_HERE, name)
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        self.lib = ctypes.CDLL(path)
        for fn, (res, args) in _SIGS.items():
            f = getattr(self.lib, fn)
            f.restype = res
            f.argtypes = args

    # -- pointer helpers -------------------------------------------------------------
    @staticmethod
    def _p(a, ptype):
        if a is None:
            return None
        assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
        return a.ctypes.data_as(ptype)

    def fp(self, a):
        if a is not None:
            assert a.dtype == np.float32
        return self._p(a, _fp)

    def u16(self, a):
        if a is not None:
            assert a.dtype == np.uint16
        return self._p(a, _u16p)

    # -- ops -------------------------------------------------------------------------
    def f32_to_bf16(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.zo_f32_to_bf16_n(self.fp(x), self.u16(out), x.size)
        return out

    def bf16_to_f32(self, u):
        u = np.ascontiguousarray(u, dtype=np.uint16)
        out = np.empty(u.shape, np.float32)
        self.lib.zo_bf16_to_f32_n(self.u16(u), self.fp(out), u.size)
        return out

    def row_bytes(self, qtype, n):
        return self.lib.zo_row_bytes(qtype, n)

    def dequantize_row(self, qtype, row, n):
        row = np.ascontiguousarray(row, dtype=np.uint8)
        out = np.empty(n, np.float32)
        rc = self.lib.zo_dequantize_row(qtype, self._p(row, _u8p), self.fp(out), n)
        if rc != 0:
            raise ValueError(f"unsupported qtype {qtype}")
        return out

    def embed_gather(self, table, qtype, ids, dim, scale):
        table = np.ascontiguousarray(table, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((ids.size, dim), np.float32)
        rc = self.lib.zo_embed_gather(self._p(table, _u8p), qtype, self._p(ids, _i32p), ids.size,
                                      dim, scale, self.fp(out))
        if rc != 0:
            raise ValueError(f"unsupported qtype {qtype}")
        return out

    def dot_row(self, qtype, row, x):
        """math.dotRow over one weight row (bytes) and f32 x."""
        row = np.ascontiguousarray(row, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        return float(self.lib.zo_dot_row(qtype, self._p(row, _u8p), self.fp(x), x.size))

    def gemv(self, qtype, w, x):
        """math.gemv: w is [rows, row_bytes] uint8 (or [rows, cols] f32 for F32), x f32[cols]."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        w = np.ascontiguousarray(w).view(np.uint8).reshape(w.shape[0], -1)
        y = np.empty(w.shape[0], np.float32)
        if self.lib.zo_gemv(qtype, self._p(w, _u8p), self.fp(x), self.fp(y), w.shape[0], x.size) != 0:
            raise ValueError(f"unsupported qtype {qtype}")
        return y

    def gemm(self, qtype, w, x):
        """math.gemm: x f32[batch, cols] -> y f32[batch, rows] (batch 1 is gemv)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        w = np.ascontiguousarray(w).view(np.uint8).reshape(w.shape[0], -1)
        y = np.empty((x2.shape[0], w.shape[0]), np.float32)
        rc = self.lib.zo_gemm(qtype, self._p(w, _u8p), self.fp(x2), self.fp(y), x2.shape[0], w.shape[0],
                              x2.shape[1])
        if rc != 0:
            raise ValueError(f"unsupported qtype {qtype}")
        return y

    def argmax(self, logits):
        """sampler.sampleGreedy over one row of logits."""
        x = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
        return int(self.lib.zo_argmax(self.fp(x), x.size))

    def attention(self, q, kc, vc, row0, pos, n_heads, n_kv_heads, head_dim, scale, softcap=0.0,
                  window=0):
        """One query token (q f32[n_heads*head_dim]) over cache rows row0+start .. row0+pos
        of kc / vc ([rows, row_stride] f32 or bf16 uint16)."""
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
        kc = np.ascontiguousarray(kc)
        vc = np.ascontiguousarray(vc)
        kvd = 1 if kc.dtype == np.uint16 else 0
        out = np.empty(n_heads * head_dim, np.float32)
        rc = self.lib.zo_attention_token(self.fp(q), kc.ctypes.data, vc.ctypes.data, kvd, row0, kc.shape[-1],
                                         pos, window, n_heads, n_kv_heads, head_dim, scale, softcap,
                                         self.fp(out))
        if rc != 0:
            raise MemoryError("oracle attention")
        return out

    def rms_norm(self, x, w, eps, unit_offset=True):
        """Row-wise math.rmsNorm over the last axis (w=None -> rmsNormNoScale)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[-1]
        out = np.empty_like(x)
        xr, orr = x.reshape(-1, n), out.reshape(-1, n)
        for r in range(xr.shape[0]):
            if w is None:
                self.lib.zo_rms_norm_no_scale(self.fp(xr[r]), self.fp(orr[r]), n, eps)
            else:
                self.lib.zo_rms_norm(self.fp(xr[r]), self.fp(w), self.fp(orr[r]), n, eps,
                                     int(unit_offset))
        return out

    def add_rms_norm(self, x, r, w, eps, unit_offset=True):
        """Returns (x + r, rmsNorm(x + r)) row-wise (model.zig:714-723)."""
        x = np.array(x, dtype=np.float32, copy=True, order="C")
        r = np.ascontiguousarray(r, dtype=np.float32)
        n = x.shape[-1]
        out = np.empty_like(x)
        xr, rr, orr = x.reshape(-1, n), r.reshape(-1, n), out.reshape(-1, n)
        for i in range(xr.shape[0]):
            self.lib.zo_add_rms_norm(self.fp(xr[i]), self.fp(rr[i]), self.fp(w), self.fp(orr[i]),
                                     n, eps, int(unit_offset))
        return x, out

    def rms_norm_add(self, x, inp, w, eps, unit_offset=True):
        """Returns x + rmsNorm(inp) row-wise (model.zig:748-755); f32 or bf16 (uint16)."""
        if x.dtype == np.uint16:
            x = np.array(x, copy=True, order="C")
            inp = np.ascontiguousarray(inp, dtype=np.uint16)
            n = x.shape[-1]
            self.lib.zo_rms_norm_add_bf16(self.u16(x), self.u16(inp), self.fp(w), x.size // n, n,
                                          eps, int(unit_offset))
            return x
        x = np.array(x, dtype=np.float32, copy=True, order="C")
        inp = np.ascontiguousarray(inp, dtype=np.float32)
        n = x.shape[-1]
        xr, ir = x.reshape(-1, n), inp.reshape(-1, n)
        for i in range(xr.shape[0]):
            self.lib.zo_rms_norm_add(self.fp(xr[i]), self.fp(ir[i]), self.fp(w), n, eps,
                                     int(unit_offset))
        return x

    def rms_norm_add_rms_norm(self, x, xb, w1, w2, eps, unit_offset=True):
        """Returns (x + norm1(xb), norm2(x + norm1(xb))) row-wise; f32 or bf16 (uint16)."""
        n = x.shape[-1]
        rows = x.size // n
        if x.dtype == np.uint16:
            x = np.array(x, copy=True, order="C")
            xb = np.array(xb, copy=True, order="C")
            self.lib.zo_rms_norm_add_rms_norm_bf16(self.u16(x), self.u16(xb), self.fp(w1),
                                                   self.fp(w2), rows, n, eps, int(unit_offset))
        else:
            x = np.array(x, dtype=np.float32, copy=True, order="C")
            xb = np.array(xb, dtype=np.float32, copy=True, order="C")
            self.lib.zo_rms_norm_add_rms_norm(self.fp(x), self.fp(xb), self.fp(w1), self.fp(w2),
                                              rows, n, eps, int(unit_offset))
        return x, xb

    def add_rms_norm_bf16(self, x, r, w, eps, unit_offset=True):
        x = np.array(x, dtype=np.uint16, copy=True, order="C")
        r = np.ascontiguousarray(r, dtype=np.uint16)
        n = x.shape[-1]
        out = np.empty_like(x)
        self.lib.zo_add_rms_norm_bf16(self.u16(x), self.u16(r), self.fp(w), self.u16(out),
                                      x.size // n, n, eps, int(unit_offset))
        return x, out

    def rms_norm_bf16(self, x, w, eps, unit_offset=True):
        x = np.ascontiguousarray(x, dtype=np.uint16)
        n = x.shape[-1]
        out = np.empty_like(x)
        self.lib.zo_rms_norm_bf16(self.u16(x), self.fp(w), self.u16(out), x.size // n, n, eps,
                                  int(unit_offset))
        return out

    def rope_denominator(self, base, i, eff):
        return self.lib.zo_rope_denominator(base, i, eff)

    def rope_cos_sin(self, pos_f, denom):
        c, s = ctypes.c_float(), ctypes.c_float()
        self.lib.zo_rope_cos_sin(pos_f, denom, ctypes.byref(c), ctypes.byref(s))
        return c.value, s.value

    def apply_rope(self, q, k, pos, head_size, rotary_dim, n_heads, n_kv_heads, base,
                   freq_scale=1.0, neox=False):
        q = None if q is None else np.array(q, dtype=np.float32, copy=True, order="C")
        k = None if k is None else np.array(k, dtype=np.float32, copy=True, order="C")
        self.lib.zo_apply_rope(self.fp(q), self.fp(k), pos, head_size, rotary_dim, n_heads,
                               n_kv_heads, base, freq_scale, int(neox))
        return q, k

    def kv_cache_put(self, k_cache, v_cache, k, v, layer, pos, max_seq, n_kv, hd, max_kv_dim):
        self.lib.zo_kv_cache_put(self.fp(k_cache), self.fp(v_cache), self.fp(k), self.fp(v),
                                 layer, pos, max_seq, n_kv, hd, max_kv_dim)

    def qk_norm_rope_kv(self, q, k, v, wq, wk, k_cache, v_cache, *, v_norm=False, layer=0,
                        max_seq, max_kv_dim, pos=None, pos_base=0, slots=None, n_heads,
                        n_kv_heads, head_dim, rotary_dim=0, base=10000.0, freq_scale=1.0,
                        eps=1e-6, unit_offset=True):
        """Token-batched fused op; returns the new q. k_cache/v_cache are updated in place."""
        dtype = 1 if q.dtype == np.uint16 else 0
        q = np.array(q, copy=True, order="C")
        k = np.ascontiguousarray(k)
        v = np.ascontiguousarray(v)
        n_tokens = q.size // (n_heads * head_dim)
        pos_a = None if pos is None else np.ascontiguousarray(pos, dtype=np.int32)
        slot_a = None if slots is None else np.ascontiguousarray(slots, dtype=np.int64)
        self.lib.zo_qk_norm_rope_kv(
            dtype, q.ctypes.data, k.ctypes.data, v.ctypes.data, self.fp(wq), self.fp(wk),
            int(v_norm), k_cache.ctypes.data, v_cache.ctypes.data, layer, max_seq, max_kv_dim,
            self._p(pos_a, _i32p), pos_base, self._p(slot_a, _i64p), n_tokens, n_heads,
            n_kv_heads, head_dim, rotary_dim, base, freq_scale, eps, int(unit_offset))
        return q

    def tanhf(self, x):
        return self.lib.zo_tanhf(x)

    def expm1f(self, x):
        return self.lib.zo_expm1f(x)

    def gelu(self, x):
        return self.lib.zo_gelu(x)

    def geglu(self, gate, up):
        if gate.dtype == np.uint16:
            g = np.ascontiguousarray(gate)
            u = np.ascontiguousarray(up, dtype=np.uint16)
            out = np.empty_like(g)
            self.lib.zo_geglu_bf16(self.u16(g), self.u16(u), self.u16(out), g.size)
            return out
        g = np.ascontiguousarray(gate, dtype=np.float32)
        u = np.ascontiguousarray(up, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.zo_geglu(self.fp(g), self.fp(u), self.fp(out), g.size)
        return out

    def silu(self, x):
        return self.lib.zo_silu(x)

    def swiglu(self, gate, up):
        """math.swiglu: silu(gate) * up; f32, or bf16 (uint16) rounded once."""
        if gate.dtype == np.uint16:
            g = np.ascontiguousarray(gate)
            u = np.ascontiguousarray(up, dtype=np.uint16)
            out = np.empty_like(g)
            self.lib.zo_swiglu_bf16(self.u16(g), self.u16(u), self.u16(out), g.size)
            return out
        g = np.ascontiguousarray(gate, dtype=np.float32)
        u = np.ascontiguousarray(up, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.zo_swiglu(self.fp(g), self.fp(u), self.fp(out), g.size)
        return out

    def ple_gate_gelu(self, gate, ple_slice):
        """model.zig:762-768: ple_slice * gelu(gate)."""
        g = np.ascontiguousarray(gate, dtype=np.float32)
        s_ = np.ascontiguousarray(ple_slice, dtype=np.float32)
        out = np.empty_like(g)
        self.lib.zo_ple_gate_gelu(self.fp(g), self.fp(s_), self.fp(out), g.size)
        return out

    def ple_ctx_fuse(self, ctx, scratch, add_token_embd=True):
        """model.zig:525-535: (ctx + scratch) * f32(1/sqrt 2), or scratch (returns a copy)."""
        c = np.array(ctx, dtype=np.float32, copy=True, order="C")
        s_ = np.ascontiguousarray(scratch, dtype=np.float32)
        self.lib.zo_ple_ctx_fuse(self.fp(c), self.fp(s_), c.size, int(bool(add_token_embd)))
        return c

    def ple_token_inputs(self, ple_row_f32, x, proj_qtype, proj_w, proj_norm, n_layers, eps,
                         token_path=True, ple_dim=256):
        """model.zig:506-540 after the row gather: ple = row * sqrt(256) (token path, else 0);
        ctx = proj(x / sqrt(dim)); per layer l: ctx_l = rmsNorm(ctx_l; proj_norm) (no unit
        offset) and ple_l = (ple_l + ctx_l) * f32(1/sqrt 2) (token path) or ctx_l.
        ple_row_f32: the dequantized PLE row (n_layers * ple_dim), or None when not token_path."""
        n = n_layers * ple_dim
        if token_path:
            ple = (np.asarray(ple_row_f32, np.float32) * np.float32(np.sqrt(np.float32(ple_dim)))).astype(np.float32)
        else:
            ple = np.zeros(n, np.float32)
        if proj_w is None:
            return ple
        x = np.asarray(x, np.float32)
        inv = np.float32(1.0) / np.sqrt(np.float32(x.size))
        xb = (x * inv).astype(np.float32)
        ctx = self.gemv(proj_qtype, proj_w, xb)
        if proj_norm is None:
            return ple
        for l in range(n_layers):
            sl = slice(l * ple_dim, (l + 1) * ple_dim)
            ctx[sl] = self.rms_norm(ctx[sl], proj_norm, eps, unit_offset=False)
            ple[sl] = self.ple_ctx_fuse(ple[sl], ctx[sl], token_path)
        return ple

    def ple_inject(self, x, ple_slice, gate_qtype, gate_w, proj_qtype, proj_w, post_norm, eps):
        """model.zig:757-781 for one layer: gate = gelu(W_gate x); ple = slice * gate;
        d = W_proj ple; d = rmsNorm(d; post_norm) (no unit offset) when present; returns x + d."""
        gate = self.gemv(gate_qtype, gate_w, x)
        pb = self.ple_gate_gelu(gate, ple_slice)
        d = self.gemv(proj_qtype, proj_w, pb)
        if post_norm is not None:
            d = self.rms_norm(d, post_norm, eps, unit_offset=False)
        return (np.asarray(x, np.float32) + d).astype(np.float32)

    def softcap(self, x, cap):
        x = np.array(x, dtype=np.float32, copy=True, order="C")
        self.lib.zo_softcap(self.fp(x), cap, x.size)
        return x

    def tanh_array(self, x):
        """Elementwise zo_tanhf over an array (via soft-cap with cap 1, which is exact:
        1*tanh(x/1) == tanh(x))."""
        return self.softcap(x, 1.0)


_cache = {}


def get(simd=False):
    if simd not in _cache:
        _cache[simd] = Oracle(simd)
    return _cache[simd]
