"""ctypes binding of libhip_bridge.so: one typed Python callable per C-ABI entry point of
include/hip_bridge.h.

This is the Python side of the drop-in boundary (the Zig host binds the same symbols with
`extern "c"` declarations). There is no fallback: if the library is missing or a symbol is
absent, loading raises.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
# HIP_BRIDGE_LIB selects another build of the same library (e.g. for A/B measurements).
LIB_PATH = os.environ.get("HIP_BRIDGE_LIB") or os.path.join(PKG, "libhip_bridge.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 14, 30
F32_TERMS = 256  # f32 activations as three bf16 term planes (hip_split_terms)
OK, EINVAL, EUNSUPPORTED, ESCRATCH = 0, -1, -2, -3

_v = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t
_pv = ctypes.POINTER(ctypes.c_void_p)

PRO_NORM, PRO_GEGLU = 1, 2


class GemvPrologue(ctypes.Structure):
    """HipGemvPrologue (include/hip_bridge.h)."""
    _fields_ = [("mode", ctypes.c_int), ("r", ctypes.c_void_p), ("r_weight", ctypes.c_void_p),
                ("r_unit_offset", ctypes.c_int), ("scale", ctypes.c_float), ("x_out", ctypes.c_void_p),
                ("weight", ctypes.c_void_p), ("unit_offset", ctypes.c_int), ("eps", ctypes.c_float),
                ("xb_out", ctypes.c_void_p)]


_ppro = ctypes.POINTER(GemvPrologue)

# name -> (restype, argtypes), in header order.
SIGNATURES = {
    # runtime (cuda_bridge.h:15-33)
    "hip_device_get_info": (_i, [_i, ctypes.c_char_p, _sz, ctypes.POINTER(_sz)]),
    "hip_malloc": (_i, [_pv, _sz]),
    "hip_free": (_i, [_v]),
    "hip_malloc_host": (_i, [_pv, _sz]),
    "hip_free_host": (_i, [_v]),
    "hip_memcpy_h2d": (_i, [_v, _v, _sz, _v]),
    "hip_memcpy_d2h": (_i, [_v, _v, _sz, _v]),
    "hip_memcpy_d2d": (_i, [_v, _v, _sz, _v]),
    "hip_stream_create": (_i, [_pv]),
    "hip_stream_destroy": (_i, [_v]),
    "hip_stream_sync": (_i, [_v]),
    "hip_graph_begin_capture": (_i, [_v]),
    "hip_graph_end_capture": (_i, [_v, _pv]),
    "hip_graph_instantiate": (_i, [_pv, _v]),
    "hip_graph_launch": (_i, [_v, _v]),
    "hip_graph_destroy": (_i, [_v]),
    "hip_graph_exec_destroy": (_i, [_v]),
    # new runtime helpers
    "hip_event_create": (_i, [_pv]),
    "hip_event_destroy": (_i, [_v]),
    "hip_event_record": (_i, [_v, _v]),
    "hip_event_sync": (_i, [_v]),
    "hip_event_elapsed_ms": (_i, [ctypes.POINTER(_f), _v, _v]),
    "hip_fill_u8": (_i, [_v, ctypes.c_ubyte, _sz, _v]),
    "hip_bridge_last_error": (_i, []),
    "hip_bridge_error_string": (ctypes.c_char_p, [_i]),
    "hip_bridge_version": (ctypes.c_char_p, []),
    # gather (cuda_bridge.h:53-54 + new)
    "hip_embed_lookup": (None, [_v, _i, _i, _v, _i, _f, _v]),
    "hip_embed_lookup_batch": (None, [_v, _i, _v, _v, _i, _i, _f, _v]),
    "hip_embed_gather": (None, [_v, _i, _i64, _v, _i, _v, _i64, _i, _f, _v]),
    # norms (cuda_bridge.h:55-58, cuda_bridge.cu:2058 + new)
    "hip_rmsnorm": (None, [_v, _v, _v, _i, _f, _i, _v]),
    "hip_rmsnorm_batched": (None, [_v, _v, _v, _i, _i, _f, _i, _v]),
    "hip_add_rmsnorm": (None, [_v, _v, _v, _v, _i, _f, _i, _v]),
    "hip_add_rmsnorm_batched": (None, [_v, _v, _v, _v, _i, _i, _f, _i, _v]),
    "hip_rmsnorm_add": (None, [_v, _v, _v, _i, _f, _i, _v]),
    "hip_rmsnorm_rows": (None, [_i, _v, _v, _v, _i64, _i, _f, _i, _v]),
    "hip_add_rmsnorm_rows": (None, [_i, _v, _v, _v, _v, _i64, _i, _f, _i, _v]),
    "hip_rmsnorm_add_rows": (None, [_i, _v, _v, _v, _i64, _i, _f, _i, _v]),
    "hip_rmsnorm_add_rmsnorm": (None, [_i, _v, _v, _v, _v, _v, _i64, _i, _f, _i, _v]),
    # RoPE (cuda_bridge.h:59-61)
    "hip_rope": (None, [_v, _v, _i, _i, _i, _i, _i, _f, _v]),
    "hip_rope_ind": (None, [_v, _v, _v, _i, _i, _i, _i, _f, _v]),
    "hip_rope_batched": (None, [_v, _v, _i, _i, _i, _i, _i, _i, _f, _v]),
    # KV append (cuda_bridge.h:71-112)
    "hip_kv_cache_put": (None, [_v, _v, _v, _v, _i, _i, _i, _i, _i, _i, _v]),
    "hip_kv_cache_put_ind": (None, [_v, _v, _v, _v, _i, _v, _i, _i, _i, _i, _v]),
    "hip_kv_cache_put_batched": (None, [_v, _v, _v, _v, _i, _i, _i, _i, _i, _i, _i, _v]),
    # fused attention prologue (new)
    "hip_qk_norm_rope_kv": (
        None,
        [_i, _v, _v, _v, _v, _v, _i, _v, _v, _i64, _i, _i, _i, _v, _i, _v, _i, _i, _i, _i, _i,
         _f, _f, _f, _i, _v]),
    # elementwise (cuda_bridge.h:64, 66-68 + new)
    "hip_geglu": (None, [_v, _v, _v, _i, _v]),
    "hip_swiglu": (None, [_v, _v, _v, _i, _v]),
    "hip_add": (None, [_v, _v, _i, _v]),
    "hip_scale": (None, [_v, _f, _i, _v]),
    "hip_tanh_softcap": (None, [_v, _f, _i, _v]),
    # GEMV / GEMM (cuda_bridge.h:36-50)
    "hip_gemv_q4_0": (None, [_v, _v, _v, _i, _i, _v]),
    "hip_gemv_q8_0": (None, [_v, _v, _v, _i, _i, _v]),
    "hip_gemv_q4_k": (None, [_v, _v, _v, _i, _i, _v]),
    "hip_gemv_q6_k": (None, [_v, _v, _v, _i, _i, _v]),
    "hip_gemv_f16": (None, [_v, _v, _v, _i, _i, _v]),
    "hip_gemv_bf16": (None, [_v, _v, _v, _i, _i, _v]),
    "hip_gemv_f32": (None, [_v, _v, _v, _i, _i, _v]),
    "hip_gemv": (None, [_i, _v, _v, _v, _i, _i, _v]),
    "hip_gemv_geglu_q4_0": (None, [_v, _v, _v, _v, _i, _i, _v]),
    "hip_gemv_qkv_q4_0": (None, [_v, _v, _v, _v, _v, _v, _v, _i, _i, _i, _i, _v]),
    "hip_gemv_pro": (None, [_i, _v, _v, _v, _v, _i, _i, _ppro, _v]),
    "hip_gemv_qkv_pro": (None, [_i, _v, _v, _v, _v, _v, _v, _v, _i, _i, _i, _i, _ppro, _v]),
    "hip_gemm_q4_0": (None, [_v, _v, _v, _i, _i, _i, _v]),
    "hip_gemm_q8_0": (None, [_v, _v, _v, _i, _i, _i, _v]),
    "hip_gemm_f16": (None, [_v, _v, _v, _i, _i, _i, _v]),
    "hip_gemm": (None, [_i, _v, _v, _v, _i, _i, _i, _v]),
    "hip_gemm_ex": (None, [_i, _v, _v, _i, _v, _i, _v, _i, _i, _i, _v]),
    "hip_split_terms": (None, [_v, _v, _i64, _v]),
    "hip_argmax": (None, [_v, _i, _v, _v]),
    # decode attention (cuda_bridge.h:115-168)
    "hip_attention_forward": (None, [_v, _v, _v, _v, _i, _i, _i, _i, _i, _i, _i, _f, _f, _i, _v]),
    "hip_attention_forward_ind": (None, [_v, _v, _v, _v, _i, _v, _i, _i, _i, _i, _i, _f, _f, _i, _v]),
    "hip_attention_batched": (None, [_v, _v, _v, _v, _i, _i, _i, _i, _i, _i, _i, _i, _f, _f, _i, _v]),
    "hip_attention_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "hip_attention_decode": (None, [_i, _v, _v, _v, _v, _i64, _i64, _v, _i64, _v, _i, _i, _i, _i, _i, _i,
                                    _f, _f, _i, _v, _sz, _v]),
    "hip_attention_decode_noalloc": (None, [_i, _v, _v, _v, _v, _i64, _i64, _v, _i64, _v, _i, _i, _i, _i, _i, _i,
                                            _f, _f, _i, _v]),
    "hip_attention_decode_qk": (None, [_i, _v, _v, _v, _v, _v, _i, _v, _v, _v, _i64, _i64, _v, _i64, _v, _i, _i,
                                       _i, _i, _i, _i, _i, _f, _f, _f, _i, _f, _f, _i, _v, _sz, _v]),
    "hip_geglu_ex": (None, [_i, _v, _v, _v, _i64, _v]),
    "hip_tanh_softcap_ex": (None, [_i, _v, _f, _i64, _v]),
    "hip_scale_ex": (None, [_i, _v, _f, _v, _i64, _v]),
    "hip_swiglu_ex": (None, [_i, _v, _v, _v, _i64, _v]),
    # measurement: streaming ceiling of a byte mix (new)
    "hip_stream_ref_shapes": (_i, []),
    "hip_stream_ref": (_i, [_i, _i, _v, _v, _v, _v, _i64, _i, _v]),
    "hip_stream_ref_copies": (_i, [_v, _v, _i64, _v, _v, _i64, _v, _v, _i64, _i, _i, _v]),
    # per-layer embedding steps (cuda_bridge.h:171-172)
    "hip_ple_gate_gelu": (None, [_v, _v, _v, _i, _v]),
    "hip_ple_ctx_fuse": (None, [_v, _v, _i, _i, _v]),
}


class HipError(RuntimeError):
    pass


class Bridge:
    """Loaded libhip_bridge.so with typed entry points as attributes."""

    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} not built: run `python -m ziglm_amd.build` (or __graft_entry__.build())")
        self.path = path
        self.lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self.lib, name)  # AttributeError if the symbol is missing
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)

    def version(self):
        return self.hip_bridge_version().decode()

    def check(self, rc, what="hip call"):
        if rc != 0:
            raise HipError(f"{what} failed: {rc} ({self.hip_bridge_error_string(rc).decode()})")

    def last_error(self):
        return self.hip_bridge_last_error()

    def raise_last_error(self, what="op"):
        e = self.hip_bridge_last_error()
        if e != 0:
            raise HipError(f"{what}: {e} ({self.hip_bridge_error_string(e).decode()})")


_bridge = None


def load():
    global _bridge
    if _bridge is None:
        _bridge = Bridge()
    return _bridge
