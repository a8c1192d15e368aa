"""CPU-side checks of the C-ABI boundary (no GPU needed, no compute calls):
every function declared in include/*.h is exported by libhip_bridge.so, every entry point of
the reference ABI (cuda_bridge.h and cuda.zig's extern block) has its hip_ counterpart, the
ctypes bindings (ziglm_amd/bridge.py for hip_bridge.h, ziglm_amd/gguf.py for zl_gguf.h) cover
exactly those functions, the Zig binding (ziglm_amd/zig/hip.zig) declares every hip_bridge.h
function with the header's argument count, and the library loads without initialising a
device."""
import os
import re
import subprocess
import sys

import pytest

from ziglm_amd import bridge, gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {"hip_bridge.h": "hip_", "zl_gguf.h": "zl_"}
HIP_ZIG = os.path.join(ROOT, "ziglm_amd", "zig", "hip.zig")

# The reference's C-ABI: every cuda_* function of src/cuda_bridge.h (lines 15-175) plus the
# two that only cuda.zig's extern block declares (cuda_rmsnorm_add cuda.zig:49,
# cuda_gemv_f32 cuda.zig:39). A drop-in library exports each under the hip_ prefix.
REFERENCE_ABI = """
cuda_device_get_info cuda_malloc cuda_free cuda_malloc_host cuda_free_host cuda_memcpy_h2d
cuda_memcpy_d2h cuda_memcpy_d2d cuda_stream_create cuda_stream_destroy cuda_stream_sync
cuda_graph_begin_capture cuda_graph_end_capture cuda_graph_instantiate cuda_graph_launch
cuda_graph_destroy cuda_graph_exec_destroy
cuda_gemv_q4_0 cuda_gemv_q8_0 cuda_gemv_q4_k cuda_gemv_q6_k cuda_gemv_f16 cuda_gemv_bf16 cuda_gemv
cuda_gemv_geglu_q4_0 cuda_gemv_qkv_q4_0 cuda_gemm_q4_0 cuda_gemm_q8_0 cuda_gemm_f16 cuda_gemm
cuda_embed_lookup cuda_embed_lookup_batch cuda_rmsnorm cuda_rmsnorm_batched cuda_add_rmsnorm
cuda_add_rmsnorm_batched cuda_rope cuda_rope_ind cuda_rope_batched cuda_geglu cuda_swiglu cuda_add
cuda_scale cuda_tanh_softcap cuda_kv_cache_put cuda_kv_cache_put_ind cuda_kv_cache_put_batched
cuda_attention_forward cuda_attention_forward_ind cuda_attention_batched cuda_ple_gate_gelu
cuda_ple_ctx_fuse cuda_argmax
cuda_rmsnorm_add cuda_gemv_f32
""".split()
REF_SRC = "/root/reference/src"


def declared_functions(header=None):
    names = set()
    for h, prefix in HEADERS.items():
        if header and h != header:
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text))
    return sorted(names)


def test_header_parses():
    names = declared_functions()
    assert "hip_qk_norm_rope_kv" in names and "hip_embed_lookup_batch" in names
    assert len(names) >= 50


def test_library_exports_every_declared_symbol():
    if not os.path.exists(bridge.LIB_PATH):
        pytest.fail("libhip_bridge.so is not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", bridge.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT ((?:hip|zl)_\w+)$", out, flags=re.M))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_matches_header():
    assert sorted(bridge.SIGNATURES) == declared_functions("hip_bridge.h")
    assert sorted(gguf.SIGNATURES) == declared_functions("zl_gguf.h")
    gguf.lib()  # binds every zl_ symbol


def test_library_loads_and_binds():
    b = bridge.load()
    assert "gfx950" in b.version()
    assert b.hip_bridge_last_error() == 0
    assert b.hip_bridge_error_string(-2).decode().startswith("unsupported")


def _ref_names(path, pattern):
    text = re.sub(r"/\*.*?\*/|//[^\n]*", "", open(path).read(), flags=re.S)
    return set(re.findall(pattern, text))


def test_reference_abi_list_matches_reference_sources():
    """The committed name list against the reference's own files, where they exist (this
    container only; the list above is what the other tests use)."""
    h, z = os.path.join(REF_SRC, "cuda_bridge.h"), os.path.join(REF_SRC, "cuda.zig")
    if not (os.path.exists(h) and os.path.exists(z)):
        pytest.skip("reference sources not present")
    names = _ref_names(h, r"\b(cuda_\w+)\s*\(") | _ref_names(z, r"extern \"c\" fn (cuda_\w+)")
    assert names == set(REFERENCE_ABI)


def test_every_reference_entry_point_has_a_hip_export():
    declared = set(declared_functions("hip_bridge.h"))
    missing = [n for n in REFERENCE_ABI if "hip_" + n[len("cuda_"):] not in declared]
    assert not missing, f"reference entry points without a hip_ counterpart: {missing}"


def _c_arg_counts():
    text = open(os.path.join(ROOT, "include", "hip_bridge.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(hip_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_zig_binding_declares_every_function():
    """hip.zig's extern block: every hip_bridge.h function, with the same argument count."""
    text = open(HIP_ZIG).read()
    zig = {}
    for m in re.finditer(r"pub extern \"c\" fn (hip_\w+)\((.*?)\)\s*[^;(]+;", text):
        args = m.group(2).strip()
        zig[m.group(1)] = 0 if not args else len([a for a in args.split(",") if a.strip()])
    c = _c_arg_counts()
    assert set(zig) == set(c), (sorted(set(c) - set(zig)), sorted(set(zig) - set(c)))
    bad = {n: (zig[n], c[n]) for n in c if zig[n] != c[n]}
    assert not bad, bad


def test_zig_binding_has_every_cuda_device_method():
    """HipDevice / HipBuffer offer every CudaDevice / CudaBuffer method the reference's callers
    use (cuda.zig:187-751), and the aliases under the reference's names."""
    text = open(HIP_ZIG).read()
    methods = set(re.findall(r"pub (?:inline )?fn (\w+)\(", text))
    need = """upload copyFrom download asF32 asConstF32 deinit init getName alloc sync gemv gemvGegluQ4_0
    gemvQkvQ4_0 gemmQ4_0 gemm embedLookup embedLookupBatch rmsNorm rmsNormBatched rmsnormAdd addRmsNorm
    addRmsNormBatched rope ropeInd ropeBatched kvCachePut kvCachePutInd kvCachePutBatched attentionForward
    attentionForwardInd attentionBatched geglu pleGateGelu pleCtxFuse add scale tanhSoftcap argmax""".split()
    assert not [m for m in need if m not in methods]
    for alias in ("CudaDevice", "CudaBuffer", "CudaStream_t", "CudaGraph_t", "CudaGraphExec_t"):
        assert re.search(r"pub const " + alias + r"\b", text), alias
    for n in REFERENCE_ABI:
        assert re.search(r"pub const " + n + r" = hip_", text), n


# ---- parameter types of hip.zig's externs against include/hip_bridge.h ---------------------

_C_BASE = {"int": "c_int", "unsigned int": "c_uint", "int64_t": "i64", "int32_t": "i32", "size_t": "usize",
           "float": "f32", "double": "f64", "unsigned char": "u8", "char": "u8", "uint32_t": "u32",
           "void": "anyopaque", "HipStream_t": "HipStream_t", "HipGraph_t": "HipGraph_t",
           "HipGraphExec_t": "HipGraphExec_t", "HipEvent_t": "HipEvent_t",
           "HipGemvPrologue": "HipGemvPrologue"}
# handle typedefs: void* in C, an optional opaque pointer in Zig (as cuda.zig's CudaStream_t)
_HANDLES = {"HipStream_t", "HipGraph_t", "HipGraphExec_t", "HipEvent_t"}
# Zig parameters that keep cuda.zig's declared type where the C definition is more specific
# (the same pointer in the ABI): cuda.zig:39 binds cuda_gemv_f32's const float* weights
# (cuda_bridge.cu:1151) as ?*const anyopaque.
_ZIG_AS_REFERENCE = {("hip_gemv_f32", "weights"): "?*const anyopaque"}


def _c_type(decl):
    """'const float* w' -> (pointer levels, const pointee, Zig name of the base type)."""
    t = decl.strip()
    t = t[: len(t) - len(re.search(r"\w+$", t).group(0))].strip()  # drop the parameter name
    parts = [p.strip() for p in t.split("*")]
    words = parts[0].split()
    base = " ".join(w for w in words if w != "const")
    return len(parts) - 1, "const" in words, _C_BASE[base]


def _c_params():
    text = open(os.path.join(ROOT, "include", "hip_bridge.h")).read()
    out = {}
    for m in re.finditer(r"\b(int|void|size_t|const char\*)\s+(hip_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        ret, name, args = m.group(1), m.group(2), m.group(3)
        params = []
        raw = [a for a in args.split(",")] if args.strip() not in ("", "void") else []
        for a in raw:
            nullable = "/*NULL*/" in a
            a = re.sub(r"/\*.*?\*/", "", a, flags=re.S).strip()
            levels, cbase, base = _c_type(a)
            params.append((a.split()[-1].lstrip("*"), levels, cbase, base, nullable))
        out[name] = (ret, params)
    return out


def _zig_type(t):
    """'?[*]const f32' -> (optional, levels, const pointee at the innermost level, base)."""
    t = t.strip()
    opt = t.startswith("?")
    t = t.lstrip("?")
    levels = 0
    inner_opt = False
    const = False
    while True:
        m = re.match(r"^(\[\*c\]|\[\*:0\]|\[\*\]|\*)(const\s+)?(\?)?", t)
        if not m:
            break
        levels += 1
        const = bool(m.group(2))
        inner_opt = inner_opt or bool(m.group(3))
        t = t[m.end():].strip()
    return opt, levels, const, t, inner_opt


def _zig_params():
    text = open(HIP_ZIG).read()
    out = {}
    for m in re.finditer(r"pub extern \"c\" fn (hip_\w+)\((.*?)\)\s*([^;(]+);", text):
        args = [a for a in m.group(2).split(",") if a.strip()]
        params = []
        for a in args:
            nm, ty = a.split(":", 1)
            params.append((nm.strip(), ty.strip()))
        out[m.group(1)] = (m.group(3).strip(), params)
    return out


def test_zig_binding_parameter_types_match_header():
    """Every extern of hip.zig against its C declaration, parameter by parameter: pointer
    depth, constness of the pointee, the scalar type (c_int / i64 / i32 / usize / f32 / u8),
    and optionality: a parameter the header marks NULL is optional (?) in Zig. The header's
    plain pointers may also be optional in Zig (device buffers pass as CudaBuffer.ptr, an
    optional pointer, as in cuda.zig). Handle typedefs (HipStream_t, ...) are pointer types
    in both."""
    c, z = _c_params(), _zig_params()
    assert set(c) == set(z), (sorted(set(c) - set(z)), sorted(set(z) - set(c)))
    ret_map = {"int": "c_int", "void": "void", "size_t": "usize", "const char*": "[*:0]const u8"}
    problems = []
    for name, (cret, cps) in c.items():
        zret, zps = z[name]
        if ret_map[cret] != zret:
            problems.append((name, "return", cret, zret))
        if len(cps) != len(zps):
            problems.append((name, "arity", len(cps), len(zps)))
            continue
        for (cn, lv, cconst, base, nullable), (zn, zt) in zip(cps, zps):
            opt, zlv, zconst, zbase, _ = _zig_type(zt)
            where = (name, cn, zt)
            if (name, cn) in _ZIG_AS_REFERENCE:
                if zt != _ZIG_AS_REFERENCE[(name, cn)]:
                    problems.append(where + ("cuda.zig form",))
                continue
            if base in _HANDLES:
                if lv == 0 and zbase != base or lv == 1 and not (zlv == 1 and zbase == base):
                    problems.append(where + ("handle",))
                continue
            if zlv != lv or zbase != base:
                problems.append(where + (f"C {lv}x* {base}",))
            elif lv == 1 and zconst != cconst:
                problems.append(where + ("const" if cconst else "mutable",))
            elif lv == 0 and opt:
                problems.append(where + ("optional scalar",))
            if nullable and not opt:
                problems.append(where + ("NULL allowed in C, not optional in Zig",))
    assert not problems, problems


def test_zig_type_check_catches_planted_mistakes(tmp_path, monkeypatch):
    """The check above against copies of hip.zig with one planted mistake each: a const
    pointee made mutable, an i64 narrowed to c_int, a NULL-able pointer made non-optional, a
    pointer made a double pointer."""
    src = open(HIP_ZIG).read()
    mutations = [
        ("hip_rmsnorm(x: [*]const f32", "hip_rmsnorm(x: [*]f32"),
        ("n_rows: i64, ids: [*]const i32", "n_rows: c_int, ids: [*]const i32"),
        ("hip_rmsnorm_add_rmsnorm(dtype: c_int, x: *anyopaque, xb: *const anyopaque, w1: ?[*]const f32",
         "hip_rmsnorm_add_rmsnorm(dtype: c_int, x: *anyopaque, xb: *const anyopaque, w1: [*]const f32"),
        ("hip_event_elapsed_ms(ms: *f32", "hip_event_elapsed_ms(ms: **f32"),
    ]
    for old, new in mutations:
        assert src.count(old) == 1, old
        p = tmp_path / "hip.zig"
        p.write_text(src.replace(old, new))
        monkeypatch.setattr(sys.modules[__name__], "HIP_ZIG", str(p))
        with pytest.raises(AssertionError):
            test_zig_binding_parameter_types_match_header()
