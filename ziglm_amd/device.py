"""Host-side operator interface over the hip_bridge C-ABI.

`HipDevice` mirrors ziglm's `CudaDevice` (src/cuda.zig:227-751): same method names,
argument order and meaning, one stream created at init, ops enqueued on it and returning
nothing. `DeviceBuffer` mirrors `CudaBuffer` (cuda.zig:187-225). The fused and bf16 entry
points that the reference lacks are added under new names. The parity tests drive the
kernels through this class exactly as cuda_model.zig drives CudaDevice.

Pointer arguments accept a DeviceBuffer, a raw device address (int) or None.
With strict=True (the default) every op checks hip_bridge_last_error() and raises
HipError on an argument error; the reference ignores errors, so strict=False restores that.
"""
import ctypes

import numpy as np

from . import bridge as _b


def _ptr(p):
    if p is None:
        return None
    if isinstance(p, DeviceBuffer):
        return p.ptr
    return int(p)


class DeviceBuffer:
    """Device allocation (cuda.zig:187-225 CudaBuffer): upload / copyFrom / download / deinit."""

    def __init__(self, dev, size_bytes, ptr=None, owner=True):
        self.dev = dev
        self.size_bytes = int(size_bytes)
        self.owner = owner
        if ptr is None:
            p = ctypes.c_void_p()
            dev.b.check(dev.b.hip_malloc(ctypes.byref(p), max(1, self.size_bytes)), "hip_malloc")
            ptr = p.value
        self.ptr = ptr

    def at(self, offset_bytes):
        """Non-owning view at a byte offset."""
        return DeviceBuffer(self.dev, self.size_bytes - offset_bytes, self.ptr + offset_bytes, owner=False)

    def upload(self, host, stream=None):
        host = np.ascontiguousarray(host)
        n = min(self.size_bytes, host.nbytes)
        if n:
            self.dev.b.check(self.dev.b.hip_memcpy_h2d(self.ptr, host.ctypes.data, n, stream), "upload")

    def copy_from(self, other, copy_len, stream=None):
        if copy_len:
            self.dev.b.check(self.dev.b.hip_memcpy_d2d(self.ptr, _ptr(other), copy_len, stream), "copyFrom")

    def download(self, host, stream=None):
        n = min(self.size_bytes, host.nbytes)
        if n:
            self.dev.b.check(self.dev.b.hip_memcpy_d2h(host.ctypes.data, self.ptr, n, stream), "download")
        return host

    def to_numpy(self, shape, dtype):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.size_bytes
        self.dev.sync()
        return self.download(out)

    def fill(self, value=0, stream=None):
        self.dev.b.check(self.dev.b.hip_fill_u8(self.ptr, value, self.size_bytes, stream), "fill")

    def deinit(self):
        if self.owner and self.ptr:
            self.dev.b.hip_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.deinit()
        except Exception:
            pass


class HipDevice:
    """Mirror of ziglm's CudaDevice over libhip_bridge.so (cuda.zig:227-751)."""

    def __init__(self, strict=True):
        self.b = _b.load()
        name = ctypes.create_string_buffer(256)
        vram = ctypes.c_size_t()
        if self.b.hip_device_get_info(0, name, 256, ctypes.byref(vram)) != 0:
            raise _b.HipError("CudaDeviceNotFound equivalent: no HIP device 0")
        s = ctypes.c_void_p()
        self.b.check(self.b.hip_stream_create(ctypes.byref(s)), "hip_stream_create")
        self.stream = s.value
        self.name = name.value.decode(errors="replace")
        self.total_vram_bytes = vram.value
        self.strict = strict

    # -- memory ------------------------------------------------------------------------
    def alloc(self, size_bytes):
        return DeviceBuffer(self, size_bytes)

    def from_numpy(self, arr):
        arr = np.ascontiguousarray(arr)
        buf = DeviceBuffer(self, arr.nbytes)
        buf.upload(arr)
        return buf

    def sync(self):
        self.b.check(self.b.hip_stream_sync(self.stream), "hip_stream_sync")

    def deinit(self):
        if self.stream:
            self.b.hip_stream_destroy(self.stream)
            self.stream = None

    def _done(self, what):
        if self.strict:
            self.b.raise_last_error(what)

    # -- embeddings (cuda.zig:358-380) --------------------------------------------------
    def embedLookup(self, d_weights, qtype, token_id, d_out, dim, scale_factor):
        self.b.hip_embed_lookup(_ptr(d_weights), qtype, token_id, _ptr(d_out), dim, scale_factor, self.stream)
        self._done("embedLookup")

    def embedLookupBatch(self, d_weights, qtype, d_token_ids, d_out, n_tokens, dim, scale_factor):
        self.b.hip_embed_lookup_batch(_ptr(d_weights), qtype, _ptr(d_token_ids), _ptr(d_out),
                                      n_tokens, dim, scale_factor, self.stream)
        self._done("embedLookupBatch")

    def embedGather(self, d_table, qtype, n_rows, d_ids, out_dtype, d_out, n_tokens, dim, scale):
        """new: bounds-checked gather, f32 or bf16 output."""
        self.b.hip_embed_gather(_ptr(d_table), qtype, n_rows, _ptr(d_ids), out_dtype, _ptr(d_out),
                                n_tokens, dim, scale, self.stream)
        self._done("embedGather")

    # -- norms (cuda.zig:383-445) --------------------------------------------------------
    def rmsNorm(self, d_x, d_weight, d_out, n, eps, use_unit_offset):
        self.b.hip_rmsnorm(_ptr(d_x), _ptr(d_weight), _ptr(d_out), n, eps, int(use_unit_offset), self.stream)
        self._done("rmsNorm")

    def rmsNormBatched(self, d_x, d_weight, d_out, head_dim, count, eps, use_unit_offset):
        self.b.hip_rmsnorm_batched(_ptr(d_x), _ptr(d_weight), _ptr(d_out), head_dim, count, eps,
                                   int(use_unit_offset), self.stream)
        self._done("rmsNormBatched")

    def rmsnormAdd(self, d_x, d_in, d_weight, n, eps, use_unit_offset):
        self.b.hip_rmsnorm_add(_ptr(d_x), _ptr(d_in), _ptr(d_weight), n, eps, int(use_unit_offset), self.stream)
        self._done("rmsnormAdd")

    def addRmsNorm(self, d_x, d_residual, d_weight, d_out, n, eps, use_unit_offset):
        self.b.hip_add_rmsnorm(_ptr(d_x), _ptr(d_residual), _ptr(d_weight), _ptr(d_out), n, eps,
                               int(use_unit_offset), self.stream)
        self._done("addRmsNorm")

    def addRmsNormBatched(self, d_x, d_residual, d_weight, d_out, n, batch_size, eps, use_unit_offset):
        self.b.hip_add_rmsnorm_batched(_ptr(d_x), _ptr(d_residual), _ptr(d_weight), _ptr(d_out), n,
                                       batch_size, eps, int(use_unit_offset), self.stream)
        self._done("addRmsNormBatched")

    # new dtype-generic row ops
    def rmsNormRows(self, dtype, d_x, d_weight, d_out, rows, n, eps, use_unit_offset):
        self.b.hip_rmsnorm_rows(dtype, _ptr(d_x), _ptr(d_weight), _ptr(d_out), rows, n, eps,
                                int(use_unit_offset), self.stream)
        self._done("rmsNormRows")

    def addRmsNormRows(self, dtype, d_x, d_residual, d_weight, d_out, rows, n, eps, use_unit_offset):
        self.b.hip_add_rmsnorm_rows(dtype, _ptr(d_x), _ptr(d_residual), _ptr(d_weight), _ptr(d_out),
                                    rows, n, eps, int(use_unit_offset), self.stream)
        self._done("addRmsNormRows")

    def rmsnormAddRows(self, dtype, d_x, d_in, d_weight, rows, n, eps, use_unit_offset):
        self.b.hip_rmsnorm_add_rows(dtype, _ptr(d_x), _ptr(d_in), _ptr(d_weight), rows, n, eps,
                                    int(use_unit_offset), self.stream)
        self._done("rmsnormAddRows")

    def rmsNormAddRmsNorm(self, dtype, d_x, d_xb, d_w1, d_w2, d_out, rows, n, eps, use_unit_offset):
        self.b.hip_rmsnorm_add_rmsnorm(dtype, _ptr(d_x), _ptr(d_xb), _ptr(d_w1), _ptr(d_w2),
                                       _ptr(d_out), rows, n, eps, int(use_unit_offset), self.stream)
        self._done("rmsNormAddRmsNorm")

    # -- RoPE (cuda.zig:447-488) ---------------------------------------------------------
    def rope(self, d_q, d_k, pos, num_heads, num_kv_heads, head_dim, rotary_dim, freq_base):
        self.b.hip_rope(_ptr(d_q), _ptr(d_k), pos, num_heads, num_kv_heads, head_dim, rotary_dim,
                        freq_base, self.stream)
        self._done("rope")

    def ropeInd(self, d_q, d_k, d_pos, num_heads, num_kv_heads, head_dim, rotary_dim, freq_base):
        self.b.hip_rope_ind(_ptr(d_q), _ptr(d_k), _ptr(d_pos), num_heads, num_kv_heads, head_dim,
                            rotary_dim, freq_base, self.stream)
        self._done("ropeInd")

    def ropeBatched(self, d_q, d_k, pos, batch_size, num_heads, num_kv_heads, head_dim, rotary_dim,
                    freq_base):
        self.b.hip_rope_batched(_ptr(d_q), _ptr(d_k), pos, batch_size, num_heads, num_kv_heads,
                                head_dim, rotary_dim, freq_base, self.stream)
        self._done("ropeBatched")

    # -- KV cache (cuda.zig:490-574) -----------------------------------------------------
    def kvCachePut(self, d_k_cache, d_v_cache, d_k, d_v, layer_idx, pos, max_seq, n_kv_heads,
                   head_dim, max_kv_dim):
        self.b.hip_kv_cache_put(_ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_k), _ptr(d_v), layer_idx,
                                pos, max_seq, n_kv_heads, head_dim, max_kv_dim, self.stream)
        self._done("kvCachePut")

    def kvCachePutInd(self, d_k_cache, d_v_cache, d_k, d_v, layer_idx, d_pos, max_seq, n_kv_heads,
                      head_dim, max_kv_dim):
        self.b.hip_kv_cache_put_ind(_ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_k), _ptr(d_v),
                                    layer_idx, _ptr(d_pos), max_seq, n_kv_heads, head_dim,
                                    max_kv_dim, self.stream)
        self._done("kvCachePutInd")

    def kvCachePutBatched(self, d_k_cache, d_v_cache, d_k, d_v, layer_idx, pos, batch_size,
                          max_seq, n_kv_heads, head_dim, max_kv_dim):
        self.b.hip_kv_cache_put_batched(_ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_k), _ptr(d_v),
                                        layer_idx, pos, batch_size, max_seq, n_kv_heads, head_dim,
                                        max_kv_dim, self.stream)
        self._done("kvCachePutBatched")

    # new: fused QK-norm + RoPE + KV append
    def qkNormRopeKv(self, dtype, d_q, d_k, d_v, d_q_norm_w, d_k_norm_w, v_norm, d_k_cache,
                     d_v_cache, cache_rows, layer_idx, max_seq, max_kv_dim, d_pos, pos_base,
                     d_slot, n_tokens, num_heads, num_kv_heads, head_dim, rotary_dim, freq_base,
                     freq_scale, eps, use_unit_offset):
        self.b.hip_qk_norm_rope_kv(dtype, _ptr(d_q), _ptr(d_k), _ptr(d_v), _ptr(d_q_norm_w),
                                   _ptr(d_k_norm_w), int(v_norm), _ptr(d_k_cache), _ptr(d_v_cache),
                                   cache_rows, layer_idx, max_seq, max_kv_dim, _ptr(d_pos), pos_base,
                                   _ptr(d_slot), n_tokens, num_heads, num_kv_heads, head_dim,
                                   rotary_dim, freq_base, freq_scale, eps, int(use_unit_offset),
                                   self.stream)
        self._done("qkNormRopeKv")

    # -- activations & elementwise (cuda.zig:686-750) -------------------------------------
    def geglu(self, d_gate, d_up, d_out, n):
        self.b.hip_geglu(_ptr(d_gate), _ptr(d_up), _ptr(d_out), n, self.stream)
        self._done("geglu")

    def swiglu(self, d_gate, d_up, d_out, n):
        self.b.hip_swiglu(_ptr(d_gate), _ptr(d_up), _ptr(d_out), n, self.stream)
        self._done("swiglu")

    def pleGateGelu(self, d_ple_gate, d_ple_slice, d_ple_buf, ple_dim):
        self.b.hip_ple_gate_gelu(_ptr(d_ple_gate), _ptr(d_ple_slice), _ptr(d_ple_buf), ple_dim, self.stream)
        self._done("pleGateGelu")

    def pleCtxFuse(self, d_ctx_ple_buf, d_ctx_scratch, n, add_token_embd):
        self.b.hip_ple_ctx_fuse(_ptr(d_ctx_ple_buf), _ptr(d_ctx_scratch), n, int(bool(add_token_embd)), self.stream)
        self._done("pleCtxFuse")

    # -- GEMV / GEMM (cuda.zig:281-356) ----------------------------------------------------
    def gemv(self, qtype, d_weights, d_x, d_y, rows, cols):
        self.b.hip_gemv(int(qtype), _ptr(d_weights), _ptr(d_x), _ptr(d_y), rows, cols, self.stream)
        self._done("gemv")

    def gemvGegluQ4_0(self, d_gate_w, d_up_w, d_x, d_act_out, rows, cols):
        self.b.hip_gemv_geglu_q4_0(_ptr(d_gate_w), _ptr(d_up_w), _ptr(d_x), _ptr(d_act_out), rows, cols,
                                   self.stream)
        self._done("gemvGegluQ4_0")

    def gemvQkvQ4_0(self, d_q_w, d_k_w, d_v_w, d_x, d_q_out, d_k_out, d_v_out, q_rows, k_rows, v_rows, cols):
        self.b.hip_gemv_qkv_q4_0(_ptr(d_q_w), _ptr(d_k_w), _ptr(d_v_w), _ptr(d_x), _ptr(d_q_out),
                                 _ptr(d_k_out), _ptr(d_v_out), q_rows, k_rows, v_rows, cols, self.stream)
        self._done("gemvQkvQ4_0")

    @staticmethod
    def prologue(mode=_b.PRO_NORM, r=None, r_weight=None, r_unit_offset=False, scale=1.0, x_out=None,
                 weight=None, unit_offset=False, eps=1e-6, xb_out=None):
        """A HipGemvPrologue (see include/hip_bridge.h). It holds references to the buffers
        it points at, so none is freed while the prologue can still be launched."""
        pro = _b.GemvPrologue(int(mode), _ptr(r), _ptr(r_weight), int(r_unit_offset), float(scale), _ptr(x_out),
                              _ptr(weight), int(unit_offset), float(eps), _ptr(xb_out))
        pro._keep = (r, r_weight, x_out, weight, xb_out)
        return pro

    def gemvPro(self, qtype, d_weights, d_up_weights, d_x, d_y, rows, cols, pro):
        self.b.hip_gemv_pro(int(qtype), _ptr(d_weights), _ptr(d_up_weights), _ptr(d_x), _ptr(d_y), rows, cols,
                            ctypes.byref(pro) if pro is not None else None, self.stream)
        self._done("gemvPro")

    def gemvQkvPro(self, qtype, d_q_w, d_k_w, d_v_w, d_x, d_q_out, d_k_out, d_v_out, q_rows, k_rows, v_rows, cols,
                   pro):
        self.b.hip_gemv_qkv_pro(int(qtype), _ptr(d_q_w), _ptr(d_k_w), _ptr(d_v_w), _ptr(d_x), _ptr(d_q_out),
                                _ptr(d_k_out), _ptr(d_v_out), q_rows, k_rows, v_rows, cols,
                                ctypes.byref(pro) if pro is not None else None, self.stream)
        self._done("gemvQkvPro")

    def gemmQ4_0(self, d_weights, d_x, d_y, batch_size, rows, cols):
        self.b.hip_gemm_q4_0(_ptr(d_weights), _ptr(d_x), _ptr(d_y), batch_size, rows, cols, self.stream)
        self._done("gemmQ4_0")

    def gemm(self, qtype, d_weights, d_x, d_y, batch_size, rows, cols):
        self.b.hip_gemm(int(qtype), _ptr(d_weights), _ptr(d_x), _ptr(d_y), batch_size, rows, cols, self.stream)
        self._done("gemm")

    # new: f32 / bf16 activations and output; with d_up: y = gelu(W x) * (U x)
    def gemmEx(self, qtype, d_weights, d_up, x_dtype, d_x, y_dtype, d_y, batch_size, rows, cols):
        self.b.hip_gemm_ex(int(qtype), _ptr(d_weights), _ptr(d_up), int(x_dtype), _ptr(d_x), int(y_dtype), _ptr(d_y),
                           batch_size, rows, cols, self.stream)
        self._done("gemmEx")

    # new: f32 activations -> three bf16 term planes [3][n] (hip_gemm_ex's F32_TERMS input)
    def splitTerms(self, d_x, d_planes, n):
        self.b.hip_split_terms(_ptr(d_x), _ptr(d_planes), n, self.stream)
        self._done("splitTerms")

    # -- greedy token (cuda.zig:743-750) -------------------------------------------------
    def argmax(self, d_logits, n, d_out_idx):
        self.b.hip_argmax(_ptr(d_logits), n, _ptr(d_out_idx), self.stream)
        self._done("argmax")

    # -- decode attention (cuda.zig:576-684) ---------------------------------------------
    def attentionForward(self, d_q, d_k_cache, d_v_cache, d_out, donor_layer, pos, max_seq, n_heads,
                         n_kv_heads, head_dim, max_kv_dim, attn_scale, softcap, sliding_window):
        self.b.hip_attention_forward(_ptr(d_q), _ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_out), donor_layer, pos,
                                     max_seq, n_heads, n_kv_heads, head_dim, max_kv_dim, attn_scale, softcap,
                                     sliding_window, self.stream)
        self._done("attentionForward")

    def attentionForwardInd(self, d_q, d_k_cache, d_v_cache, d_out, donor_layer, d_pos, max_seq, n_heads,
                            n_kv_heads, head_dim, max_kv_dim, attn_scale, softcap, sliding_window):
        self.b.hip_attention_forward_ind(_ptr(d_q), _ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_out), donor_layer,
                                         _ptr(d_pos), max_seq, n_heads, n_kv_heads, head_dim, max_kv_dim,
                                         attn_scale, softcap, sliding_window, self.stream)
        self._done("attentionForwardInd")

    def attentionBatched(self, d_q, d_k_cache, d_v_cache, d_out, donor_layer, pos, batch_size, max_seq,
                         n_heads, n_kv_heads, head_dim, max_kv_dim, attn_scale, softcap, sliding_window):
        self.b.hip_attention_batched(_ptr(d_q), _ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_out), donor_layer, pos,
                                     batch_size, max_seq, n_heads, n_kv_heads, head_dim, max_kv_dim, attn_scale,
                                     softcap, sliding_window, self.stream)
        self._done("attentionBatched")

    def attentionWorkspaceBytes(self, batch, n_heads, n_kv_heads, head_dim, max_len, sliding_window=0):
        return int(self.b.hip_attention_workspace_bytes(batch, n_heads, n_kv_heads, head_dim, max_len,
                                                        sliding_window))

    def attentionDecode(self, kv_dtype, d_q, d_k_cache, d_v_cache, d_out, cache_rows, row_stride, d_row_base,
                        row_base, d_pos, pos_base, max_len, batch, n_heads, n_kv_heads, head_dim, attn_scale,
                        softcap, sliding_window, d_workspace=None, workspace_bytes=0):
        self.b.hip_attention_decode(int(kv_dtype), _ptr(d_q), _ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_out),
                                    cache_rows, row_stride, _ptr(d_row_base), row_base, _ptr(d_pos), pos_base,
                                    max_len, batch, n_heads, n_kv_heads, head_dim, attn_scale, softcap,
                                    sliding_window, _ptr(d_workspace), workspace_bytes, self.stream)
        self._done("attentionDecode")

    def attentionDecodeNoalloc(self, kv_dtype, d_q, d_k_cache, d_v_cache, d_out, cache_rows, row_stride, d_row_base,
                               row_base, d_pos, pos_base, max_len, batch, n_heads, n_kv_heads, head_dim, attn_scale,
                               softcap, sliding_window):
        """attentionDecode with the split partials in the library's static scratch (no
        workspace, no allocation); calls whose workspace would exceed 32 MiB record ESCRATCH."""
        self.b.hip_attention_decode_noalloc(int(kv_dtype), _ptr(d_q), _ptr(d_k_cache), _ptr(d_v_cache), _ptr(d_out),
                                            cache_rows, row_stride, _ptr(d_row_base), row_base, _ptr(d_pos), pos_base,
                                            max_len, batch, n_heads, n_kv_heads, head_dim, attn_scale, softcap,
                                            sliding_window, self.stream)
        self._done("attentionDecodeNoalloc")

    def attentionDecodeQk(self, kv_dtype, d_q, d_k, d_v, d_q_norm_w, d_k_norm_w, v_norm, d_k_cache, d_v_cache,
                          d_out, cache_rows, row_stride, d_row_base, row_base, d_pos, pos_base, max_len, batch,
                          n_heads, n_kv_heads, head_dim, rotary_dim, freq_base, freq_scale, eps, use_unit_offset,
                          attn_scale, softcap, sliding_window, d_workspace=None, workspace_bytes=0):
        self.b.hip_attention_decode_qk(int(kv_dtype), _ptr(d_q), _ptr(d_k), _ptr(d_v), _ptr(d_q_norm_w),
                                       _ptr(d_k_norm_w), int(bool(v_norm)), _ptr(d_k_cache), _ptr(d_v_cache),
                                       _ptr(d_out), cache_rows, row_stride, _ptr(d_row_base), row_base, _ptr(d_pos),
                                       pos_base, max_len, batch, n_heads, n_kv_heads, head_dim, rotary_dim,
                                       freq_base, freq_scale, eps, int(bool(use_unit_offset)), attn_scale, softcap,
                                       sliding_window, _ptr(d_workspace), workspace_bytes, self.stream)
        self._done("attentionDecodeQk")

    def gegluEx(self, dtype, d_gate, d_up, d_out, n):
        self.b.hip_geglu_ex(dtype, _ptr(d_gate), _ptr(d_up), _ptr(d_out), n, self.stream)
        self._done("gegluEx")

    def add(self, d_x, d_res, n):
        self.b.hip_add(_ptr(d_x), _ptr(d_res), n, self.stream)
        self._done("add")

    def scale(self, d_x, s, n):
        self.b.hip_scale(_ptr(d_x), s, n, self.stream)
        self._done("scale")

    def scaleEx(self, dtype, d_x, s, d_out, n):
        self.b.hip_scale_ex(dtype, _ptr(d_x), s, _ptr(d_out), n, self.stream)
        self._done("scaleEx")

    def swigluEx(self, dtype, d_gate, d_up, d_out, n):
        self.b.hip_swiglu_ex(dtype, _ptr(d_gate), _ptr(d_up), _ptr(d_out), n, self.stream)
        self._done("swigluEx")

    def copyF32(self, d_src, d_dst, n):
        """dst = src (n f32) by a kernel, so it records as a kernel node in a graph."""
        self.scaleEx(_b.F32, d_src, 1.0, d_dst, n)

    def tanhSoftcap(self, d_x, cap, n):
        self.b.hip_tanh_softcap(_ptr(d_x), cap, n, self.stream)
        self._done("tanhSoftcap")

    def tanhSoftcapEx(self, dtype, d_x, cap, n):
        self.b.hip_tanh_softcap_ex(dtype, _ptr(d_x), cap, n, self.stream)
        self._done("tanhSoftcapEx")

    # -- timing ----------------------------------------------------------------------------
    def event(self):
        e = ctypes.c_void_p()
        self.b.check(self.b.hip_event_create(ctypes.byref(e)), "hip_event_create")
        return e.value

    def record(self, ev):
        self.b.check(self.b.hip_event_record(ev, self.stream), "hip_event_record")

    def elapsed_ms(self, start, stop):
        self.b.check(self.b.hip_event_sync(stop), "hip_event_sync")
        ms = ctypes.c_float()
        self.b.check(self.b.hip_event_elapsed_ms(ctypes.byref(ms), start, stop), "hip_event_elapsed_ms")
        return ms.value


class Graph:
    """hipGraph of whatever `body()` enqueues on dev.stream (the reference's graph capture,
    cuda_bridge.h:28-33): capture once, replay with launch()."""

    def __init__(self, dev, body):
        self.dev, b = dev, dev.b
        b.check(b.hip_graph_begin_capture(dev.stream), "begin_capture")
        try:
            body()
        finally:
            g = ctypes.c_void_p()
            b.check(b.hip_graph_end_capture(dev.stream, ctypes.byref(g)), "end_capture")
        ex = ctypes.c_void_p()
        b.check(b.hip_graph_instantiate(ctypes.byref(ex), g), "instantiate")
        self.graph, self.exec = g.value, ex.value

    def launch(self):
        self.dev.b.check(self.dev.b.hip_graph_launch(self.exec, self.dev.stream), "graph_launch")

    def destroy(self):
        self.dev.b.hip_graph_exec_destroy(self.exec)
        self.dev.b.hip_graph_destroy(self.graph)
