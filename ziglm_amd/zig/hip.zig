//! hip.zig: ziglm's device binding for AMD Instinct MI355X (gfx950) over libhip_bridge.so.
//!
//! This is a drop-in for ziglm's src/cuda.zig. Put the file at src/hip.zig, then replace
//! `@import("cuda.zig")` with `@import("hip.zig")` in backend.zig:8, cuda_model.zig:8,
//! engine.zig:20 and root.zig:17. Nothing else in those files changes: the file exports
//! `CudaDevice`, `CudaBuffer`, `CudaStream_t`, `CudaGraph_t`, `CudaGraphExec_t` and every
//! `cuda_*` function that cuda.zig declares (cuda.zig:13-181) as aliases of the hip_ names.
//! The C-ABI is include/hip_bridge.h. Every extern below has that header's argument list,
//! which tests/test_abi_cpu.py checks.
//!
//! Differences from cuda.zig that a caller can see:
//!   * `gemv` and `gemm` pass the GGML type id to the library's dispatcher. An unsupported
//!     type is a no-op that hip_bridge_last_error() reports. cuda.zig:299 runs every
//!     unknown type as F32.
//!   * Numerics follow ziglm's CPU path (math.zig, quant.zig), not the CUDA kernels.
//!     Gathers are bit-exact with the CPU, and norms use 1/sqrt.
//!   * Errors are named Hip* (HipMemcpyFailed, ...). ziglm's callers only propagate them
//!     with `try` or `catch |err|`, so the inferred error sets change but no call site does.
//! New methods below the reference set cover the fused and bf16 entry points.
const std = @import("std");
const types = @import("types.zig");
const GGMLType = types.GGMLType;

pub const HipStream_t = ?*anyopaque;
pub const HipGraph_t = ?*anyopaque;
pub const HipGraphExec_t = ?*anyopaque;
pub const HipEvent_t = ?*anyopaque;

/// Activation / table dtypes of the new entry points (GGML type ids, hip_bridge.h).
pub const dtype_f32: c_int = 0;
pub const dtype_bf16: c_int = 30;
/// f32 activations as three bf16 term planes (splitTerms), an input form of gemmEx.
pub const dtype_f32_terms: c_int = 256;

// ---------------------------------------------------------------------------------------
// C-ABI (include/hip_bridge.h)
// ---------------------------------------------------------------------------------------

// runtime
pub extern "c" fn hip_device_get_info(device_id: c_int, name: [*c]u8, name_len: usize, total_vram_bytes: *usize) c_int;
pub extern "c" fn hip_malloc(ptr: *?*anyopaque, bytes: usize) c_int;
pub extern "c" fn hip_free(ptr: ?*anyopaque) c_int;
pub extern "c" fn hip_malloc_host(ptr: *?*anyopaque, bytes: usize) c_int;
pub extern "c" fn hip_free_host(ptr: ?*anyopaque) c_int;
pub extern "c" fn hip_memcpy_h2d(dst: ?*anyopaque, src: ?*const anyopaque, bytes: usize, stream: HipStream_t) c_int;
pub extern "c" fn hip_memcpy_d2h(dst: ?*anyopaque, src: ?*const anyopaque, bytes: usize, stream: HipStream_t) c_int;
pub extern "c" fn hip_memcpy_d2d(dst: ?*anyopaque, src: ?*const anyopaque, bytes: usize, stream: HipStream_t) c_int;
pub extern "c" fn hip_stream_create(stream: *HipStream_t) c_int;
pub extern "c" fn hip_stream_destroy(stream: HipStream_t) c_int;
pub extern "c" fn hip_stream_sync(stream: HipStream_t) c_int;
pub extern "c" fn hip_graph_begin_capture(stream: HipStream_t) c_int;
pub extern "c" fn hip_graph_end_capture(stream: HipStream_t, graph_out: *HipGraph_t) c_int;
pub extern "c" fn hip_graph_instantiate(exec_out: *HipGraphExec_t, graph: HipGraph_t) c_int;
pub extern "c" fn hip_graph_launch(exec: HipGraphExec_t, stream: HipStream_t) c_int;
pub extern "c" fn hip_graph_destroy(graph: HipGraph_t) c_int;
pub extern "c" fn hip_graph_exec_destroy(exec: HipGraphExec_t) c_int;
pub extern "c" fn hip_event_create(event: *HipEvent_t) c_int;
pub extern "c" fn hip_event_destroy(event: HipEvent_t) c_int;
pub extern "c" fn hip_event_record(event: HipEvent_t, stream: HipStream_t) c_int;
pub extern "c" fn hip_event_sync(event: HipEvent_t) c_int;
pub extern "c" fn hip_event_elapsed_ms(ms: *f32, start: HipEvent_t, stop: HipEvent_t) c_int;
pub extern "c" fn hip_fill_u8(ptr: ?*anyopaque, value: u8, bytes: usize, stream: HipStream_t) c_int;
pub extern "c" fn hip_bridge_last_error() c_int;
pub extern "c" fn hip_bridge_error_string(code: c_int) [*:0]const u8;
pub extern "c" fn hip_bridge_version() [*:0]const u8;

// embedding gather
pub extern "c" fn hip_embed_lookup(emb_weights: ?*const anyopaque, qtype: c_int, token_id: c_int, out: [*]f32, dim: c_int, scale: f32, stream: HipStream_t) void;
pub extern "c" fn hip_embed_lookup_batch(emb_weights: ?*const anyopaque, qtype: c_int, token_ids: [*]const c_int, out: [*]f32, n_tokens: c_int, dim: c_int, scale: f32, stream: HipStream_t) void;
pub extern "c" fn hip_embed_gather(table: ?*const anyopaque, qtype: c_int, n_rows: i64, ids: [*]const i32, out_dtype: c_int, out: *anyopaque, n_tokens: i64, dim: c_int, scale: f32, stream: HipStream_t) void;

// RMSNorm family
pub extern "c" fn hip_rmsnorm(x: [*]const f32, weight: ?[*]const f32, out: [*]f32, n: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_rmsnorm_batched(x: [*]f32, weight: ?[*]const f32, out: [*]f32, head_dim: c_int, count: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_add_rmsnorm(x: [*]f32, residual: [*]const f32, weight: ?[*]const f32, out: [*]f32, n: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_add_rmsnorm_batched(x: [*]f32, residual: [*]const f32, weight: ?[*]const f32, out: [*]f32, n: c_int, batch_size: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_rmsnorm_add(x: [*]f32, in: [*]const f32, weight: ?[*]const f32, n: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_rmsnorm_rows(dtype: c_int, x: *const anyopaque, weight: ?[*]const f32, out: *anyopaque, rows: i64, n: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_add_rmsnorm_rows(dtype: c_int, x: *anyopaque, residual: *const anyopaque, weight: ?[*]const f32, out: *anyopaque, rows: i64, n: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_rmsnorm_add_rows(dtype: c_int, x: *anyopaque, in: *const anyopaque, weight: ?[*]const f32, rows: i64, n: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_rmsnorm_add_rmsnorm(dtype: c_int, x: *anyopaque, xb: *const anyopaque, w1: ?[*]const f32, w2: ?[*]const f32, out: *anyopaque, rows: i64, n: c_int, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;

// RoPE and KV-cache append
pub extern "c" fn hip_rope(q: ?[*]f32, k: ?[*]f32, pos: c_int, num_heads: c_int, num_kv_heads: c_int, head_dim: c_int, rotary_dim: c_int, freq_base: f32, stream: HipStream_t) void;
pub extern "c" fn hip_rope_ind(q: ?[*]f32, k: ?[*]f32, d_pos: [*]const c_int, num_heads: c_int, num_kv_heads: c_int, head_dim: c_int, rotary_dim: c_int, freq_base: f32, stream: HipStream_t) void;
pub extern "c" fn hip_rope_batched(q: ?[*]f32, k: ?[*]f32, pos: c_int, batch_size: c_int, num_heads: c_int, num_kv_heads: c_int, head_dim: c_int, rotary_dim: c_int, freq_base: f32, stream: HipStream_t) void;
pub extern "c" fn hip_kv_cache_put(k_cache: [*]f32, v_cache: [*]f32, k: [*]const f32, v: [*]const f32, layer_idx: c_int, pos: c_int, max_seq: c_int, n_kv_heads: c_int, head_dim: c_int, max_kv_dim: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_kv_cache_put_ind(k_cache: [*]f32, v_cache: [*]f32, k: [*]const f32, v: [*]const f32, layer_idx: c_int, d_pos: [*]const c_int, max_seq: c_int, n_kv_heads: c_int, head_dim: c_int, max_kv_dim: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_kv_cache_put_batched(k_cache: [*]f32, v_cache: [*]f32, k: [*]const f32, v: [*]const f32, layer_idx: c_int, pos: c_int, batch_size: c_int, max_seq: c_int, n_kv_heads: c_int, head_dim: c_int, max_kv_dim: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_qk_norm_rope_kv(dtype: c_int, q: ?*anyopaque, k: ?*const anyopaque, v: ?*const anyopaque, q_norm_w: ?[*]const f32, k_norm_w: ?[*]const f32, v_norm: c_int, k_cache: ?*anyopaque, v_cache: ?*anyopaque, cache_rows: i64, layer_idx: c_int, max_seq: c_int, max_kv_dim: c_int, d_pos: ?[*]const i32, pos_base: c_int, d_slot: ?[*]const i64, n_tokens: c_int, num_heads: c_int, num_kv_heads: c_int, head_dim: c_int, rotary_dim: c_int, freq_base: f32, freq_scale: f32, eps: f32, use_unit_offset: c_int, stream: HipStream_t) void;

// GEMV / GEMM
pub const HipGemvPrologue = extern struct {
    mode: c_int, // pro_norm or pro_geglu
    r: ?[*]const f32 = null,
    r_weight: ?[*]const f32 = null,
    r_unit_offset: c_int = 0,
    scale: f32 = 1.0,
    x_out: ?[*]f32 = null,
    weight: ?[*]const f32 = null,
    unit_offset: c_int = 0,
    eps: f32 = 1e-6,
    xb_out: ?[*]f32 = null,
};
pub const pro_norm: c_int = 1;
pub const pro_geglu: c_int = 2;
pub extern "c" fn hip_gemv_q4_0(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_q8_0(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_q4_k(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_q6_k(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_f16(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_bf16(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_f32(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv(qtype: c_int, weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_geglu_q4_0(gate_w: ?*const anyopaque, up_w: ?*const anyopaque, x: [*]const f32, act_out: [*]f32, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_qkv_q4_0(q_w: ?*const anyopaque, k_w: ?*const anyopaque, v_w: ?*const anyopaque, x: [*]const f32, q_out: [*]f32, k_out: [*]f32, v_out: [*]f32, q_rows: c_int, k_rows: c_int, v_rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_pro(qtype: c_int, weights: ?*const anyopaque, up_weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, rows: c_int, cols: c_int, pro: ?*const HipGemvPrologue, stream: HipStream_t) void;
pub extern "c" fn hip_gemv_qkv_pro(qtype: c_int, q_w: ?*const anyopaque, k_w: ?*const anyopaque, v_w: ?*const anyopaque, x: [*]const f32, q_out: [*]f32, k_out: [*]f32, v_out: [*]f32, q_rows: c_int, k_rows: c_int, v_rows: c_int, cols: c_int, pro: ?*const HipGemvPrologue, stream: HipStream_t) void;
pub extern "c" fn hip_gemm_q4_0(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, batch_size: c_int, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemm_q8_0(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, batch_size: c_int, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemm_f16(weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, batch_size: c_int, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_gemm(qtype: c_int, weights: ?*const anyopaque, x: [*]const f32, y: [*]f32, batch_size: c_int, rows: c_int, cols: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_split_terms(x: [*]const f32, planes: ?*anyopaque, n: i64, stream: HipStream_t) void;
pub extern "c" fn hip_gemm_ex(qtype: c_int, weights: ?*const anyopaque, up_weights: ?*const anyopaque, x_dtype: c_int, x: ?*const anyopaque, y_dtype: c_int, y: ?*anyopaque, batch_size: c_int, rows: c_int, cols: c_int, stream: HipStream_t) void;

// decode attention
pub extern "c" fn hip_attention_forward(q: [*]const f32, k_cache: [*]const f32, v_cache: [*]const f32, out: [*]f32, donor_layer: c_int, pos: c_int, max_seq: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, max_kv_dim: c_int, attn_scale: f32, softcap: f32, sliding_window: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_attention_forward_ind(q: [*]const f32, k_cache: [*]const f32, v_cache: [*]const f32, out: [*]f32, donor_layer: c_int, d_pos: [*]const c_int, max_seq: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, max_kv_dim: c_int, attn_scale: f32, softcap: f32, sliding_window: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_attention_batched(q: [*]const f32, k_cache: [*]const f32, v_cache: [*]const f32, out: [*]f32, donor_layer: c_int, pos: c_int, batch_size: c_int, max_seq: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, max_kv_dim: c_int, attn_scale: f32, softcap: f32, sliding_window: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_attention_workspace_bytes(batch: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, max_len: c_int, sliding_window: c_int) usize;
pub extern "c" fn hip_attention_decode(kv_dtype: c_int, q: [*]const f32, k_cache: ?*const anyopaque, v_cache: ?*const anyopaque, out: [*]f32, cache_rows: i64, row_stride: i64, d_row_base: ?[*]const i64, row_base: i64, d_pos: ?[*]const i32, pos_base: c_int, max_len: c_int, batch: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, attn_scale: f32, softcap: f32, sliding_window: c_int, workspace: ?*anyopaque, workspace_bytes: usize, stream: HipStream_t) void;
pub extern "c" fn hip_attention_decode_noalloc(kv_dtype: c_int, q: [*]const f32, k_cache: ?*const anyopaque, v_cache: ?*const anyopaque, out: [*]f32, cache_rows: i64, row_stride: i64, d_row_base: ?[*]const i64, row_base: i64, d_pos: ?[*]const i32, pos_base: c_int, max_len: c_int, batch: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, attn_scale: f32, softcap: f32, sliding_window: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_attention_decode_qk(kv_dtype: c_int, q: [*]const f32, k: ?[*]const f32, v: ?[*]const f32, q_norm_w: ?[*]const f32, k_norm_w: ?[*]const f32, v_norm: c_int, k_cache: *anyopaque, v_cache: *anyopaque, out: [*]f32, cache_rows: i64, row_stride: i64, d_row_base: ?[*]const i64, row_base: i64, d_pos: ?[*]const i32, pos_base: c_int, max_len: c_int, batch: c_int, n_heads: c_int, n_kv_heads: c_int, head_dim: c_int, rotary_dim: c_int, freq_base: f32, freq_scale: f32, eps: f32, use_unit_offset: c_int, attn_scale: f32, softcap: f32, sliding_window: c_int, workspace: ?*anyopaque, workspace_bytes: usize, stream: HipStream_t) void;

// greedy token selection
pub extern "c" fn hip_argmax(logits: [*]const f32, n: c_int, out_idx: [*]c_uint, stream: HipStream_t) void;

// activations and elementwise
pub extern "c" fn hip_geglu(gate: [*]const f32, up: [*]const f32, out: [*]f32, n: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_swiglu(gate: [*]const f32, up: [*]const f32, out: [*]f32, n: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_add(x: [*]f32, residual: [*]const f32, n: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_scale(x: [*]f32, scale: f32, n: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_tanh_softcap(x: [*]f32, cap: f32, n: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_geglu_ex(dtype: c_int, gate: *const anyopaque, up: *const anyopaque, out: *anyopaque, n: i64, stream: HipStream_t) void;
pub extern "c" fn hip_tanh_softcap_ex(dtype: c_int, x: *anyopaque, cap: f32, n: i64, stream: HipStream_t) void;
pub extern "c" fn hip_scale_ex(dtype: c_int, x: *const anyopaque, scale: f32, out: *anyopaque, n: i64, stream: HipStream_t) void;
pub extern "c" fn hip_swiglu_ex(dtype: c_int, gate: *const anyopaque, up: *const anyopaque, out: *anyopaque, n: i64, stream: HipStream_t) void;

// per-layer embedding steps
pub extern "c" fn hip_ple_gate_gelu(ple_gate_in: [*]const f32, ple_slice: [*]const f32, ple_buf_out: [*]f32, ple_dim: c_int, stream: HipStream_t) void;
pub extern "c" fn hip_ple_ctx_fuse(ctx_ple_buf: [*]f32, ctx_scratch: [*]const f32, n: c_int, add_token_embd: c_int, stream: HipStream_t) void;

// measurement: the streaming ceiling of a byte mix
pub extern "c" fn hip_stream_ref_shapes() c_int;
pub extern "c" fn hip_stream_ref(n_in: c_int, n_out: c_int, in0: ?*const anyopaque, in1: ?*const anyopaque, out0: ?*anyopaque, out1: ?*anyopaque, bytes: i64, shape: c_int, stream: HipStream_t) c_int;
pub extern "c" fn hip_stream_ref_copies(src0: ?*const anyopaque, dst0: ?*anyopaque, bytes0: i64, src1: ?*const anyopaque, dst1: ?*anyopaque, bytes1: i64, src2: ?*const anyopaque, dst2: ?*anyopaque, bytes2: i64, interleave: c_int, shape: c_int, stream: HipStream_t) c_int;

// ---------------------------------------------------------------------------------------
// Reference names (cuda.zig:5-181): what cuda_model.zig, engine.zig, backend.zig and
// root.zig refer to.
// ---------------------------------------------------------------------------------------
pub const CudaStream_t = HipStream_t;
pub const CudaGraph_t = HipGraph_t;
pub const CudaGraphExec_t = HipGraphExec_t;
pub const CudaDevice = HipDevice;
pub const CudaBuffer = HipBuffer;

pub const cuda_device_get_info = hip_device_get_info;
pub const cuda_malloc = hip_malloc;
pub const cuda_free = hip_free;
pub const cuda_malloc_host = hip_malloc_host;
pub const cuda_free_host = hip_free_host;
pub const cuda_memcpy_h2d = hip_memcpy_h2d;
pub const cuda_memcpy_d2h = hip_memcpy_d2h;
pub const cuda_memcpy_d2d = hip_memcpy_d2d;
pub const cuda_stream_create = hip_stream_create;
pub const cuda_stream_destroy = hip_stream_destroy;
pub const cuda_stream_sync = hip_stream_sync;
pub const cuda_graph_begin_capture = hip_graph_begin_capture;
pub const cuda_graph_end_capture = hip_graph_end_capture;
pub const cuda_graph_instantiate = hip_graph_instantiate;
pub const cuda_graph_launch = hip_graph_launch;
pub const cuda_graph_destroy = hip_graph_destroy;
pub const cuda_graph_exec_destroy = hip_graph_exec_destroy;
pub const cuda_gemv_q4_0 = hip_gemv_q4_0;
pub const cuda_gemv_q8_0 = hip_gemv_q8_0;
pub const cuda_gemv_q4_k = hip_gemv_q4_k;
pub const cuda_gemv_q6_k = hip_gemv_q6_k;
pub const cuda_gemv_f16 = hip_gemv_f16;
pub const cuda_gemv_bf16 = hip_gemv_bf16;
pub const cuda_gemv_f32 = hip_gemv_f32;
pub const cuda_gemv = hip_gemv;
pub const cuda_gemv_geglu_q4_0 = hip_gemv_geglu_q4_0;
pub const cuda_gemv_qkv_q4_0 = hip_gemv_qkv_q4_0;
pub const cuda_gemm_q4_0 = hip_gemm_q4_0;
pub const cuda_gemm_q8_0 = hip_gemm_q8_0;
pub const cuda_gemm_f16 = hip_gemm_f16;
pub const cuda_gemm = hip_gemm;
pub const cuda_embed_lookup = hip_embed_lookup;
pub const cuda_embed_lookup_batch = hip_embed_lookup_batch;
pub const cuda_rmsnorm = hip_rmsnorm;
pub const cuda_rmsnorm_batched = hip_rmsnorm_batched;
pub const cuda_add_rmsnorm = hip_add_rmsnorm;
pub const cuda_add_rmsnorm_batched = hip_add_rmsnorm_batched;
pub const cuda_rmsnorm_add = hip_rmsnorm_add;
pub const cuda_rope = hip_rope;
pub const cuda_rope_ind = hip_rope_ind;
pub const cuda_rope_batched = hip_rope_batched;
pub const cuda_geglu = hip_geglu;
pub const cuda_swiglu = hip_swiglu;
pub const cuda_add = hip_add;
pub const cuda_scale = hip_scale;
pub const cuda_tanh_softcap = hip_tanh_softcap;
pub const cuda_kv_cache_put = hip_kv_cache_put;
pub const cuda_kv_cache_put_ind = hip_kv_cache_put_ind;
pub const cuda_kv_cache_put_batched = hip_kv_cache_put_batched;
pub const cuda_attention_forward = hip_attention_forward;
pub const cuda_attention_forward_ind = hip_attention_forward_ind;
pub const cuda_attention_batched = hip_attention_batched;
pub const cuda_ple_gate_gelu = hip_ple_gate_gelu;
pub const cuda_ple_ctx_fuse = hip_ple_ctx_fuse;
pub const cuda_argmax = hip_argmax;

// ---------------------------------------------------------------------------------------
// Conversions used by every wrapper
// ---------------------------------------------------------------------------------------
inline fn int(v: usize) c_int {
    return @intCast(v);
}
inline fn flag(b: bool) c_int {
    return @intFromBool(b);
}
inline fn qt(t: GGMLType) c_int {
    return @intCast(@intFromEnum(t));
}

// ---------------------------------------------------------------------------------------
// HipBuffer (the reference's CudaBuffer, cuda.zig:187-225)
// ---------------------------------------------------------------------------------------
pub const HipBuffer = struct {
    ptr: ?*anyopaque,
    size_bytes: usize,

    fn copied(rc: c_int) !void {
        if (rc != 0) return error.HipMemcpyFailed;
    }

    /// Host -> device, at most size_bytes (stream null: synchronous).
    pub fn upload(self: *const HipBuffer, host_src: []const u8, stream: HipStream_t) !void {
        const n = @min(self.size_bytes, host_src.len);
        if (n != 0) try copied(hip_memcpy_h2d(self.ptr, host_src.ptr, n, stream));
    }

    pub fn copyFrom(self: *const HipBuffer, other: HipBuffer, copy_len: usize, stream: HipStream_t) !void {
        if (copy_len != 0) try copied(hip_memcpy_d2d(self.ptr, other.ptr, copy_len, stream));
    }

    /// Device -> host, at most size_bytes.
    pub fn download(self: *const HipBuffer, host_dst: []u8, stream: HipStream_t) !void {
        const n = @min(self.size_bytes, host_dst.len);
        if (n != 0) try copied(hip_memcpy_d2h(host_dst.ptr, self.ptr, n, stream));
    }

    pub inline fn asF32(self: *const HipBuffer) [*]f32 {
        return @ptrCast(@alignCast(self.ptr.?));
    }

    pub inline fn asConstF32(self: *const HipBuffer) [*]const f32 {
        return @ptrCast(@alignCast(self.ptr.?));
    }

    pub fn deinit(self: *HipBuffer) void {
        const p = self.ptr orelse return;
        _ = hip_free(p);
        self.ptr = null;
    }
};

// ---------------------------------------------------------------------------------------
// HipDevice (the reference's CudaDevice, cuda.zig:227-751): one device, one stream; every
// op is enqueued on `stream` and never synchronises, so a decode step can be captured.
// ---------------------------------------------------------------------------------------
pub const HipDevice = struct {
    allocator: std.mem.Allocator,
    stream: HipStream_t,
    name: [256]u8,
    name_len: usize,
    total_vram_bytes: usize,

    pub fn init(allocator: std.mem.Allocator) !*HipDevice {
        var name: [256]u8 = [_]u8{0} ** 256;
        var vram: usize = 0;
        if (hip_device_get_info(0, &name, name.len, &vram) != 0) return error.HipDeviceNotFound;
        var stream: HipStream_t = null;
        if (hip_stream_create(&stream) != 0) return error.HipStreamCreateFailed;
        errdefer _ = hip_stream_destroy(stream);
        const self = try allocator.create(HipDevice);
        self.* = .{
            .allocator = allocator,
            .stream = stream,
            .name = name,
            .name_len = std.mem.indexOfScalar(u8, &name, 0) orelse name.len,
            .total_vram_bytes = vram,
        };
        return self;
    }

    pub fn deinit(self: *HipDevice) void {
        _ = hip_stream_destroy(self.stream);
        self.allocator.destroy(self);
    }

    pub fn getName(self: *const HipDevice) []const u8 {
        return self.name[0..self.name_len];
    }

    pub fn alloc(self: *const HipDevice, size_bytes: usize) !HipBuffer {
        _ = self;
        var p: ?*anyopaque = null;
        if (hip_malloc(&p, size_bytes) != 0 or p == null) return error.HipOutOfMemory;
        return .{ .ptr = p, .size_bytes = size_bytes };
    }

    pub fn sync(self: *const HipDevice) void {
        _ = hip_stream_sync(self.stream);
    }

    // ---- GEMV / GEMM (cuda.zig:281-356) -------------------------------------------------
    pub fn gemv(self: *const HipDevice, qtype: GGMLType, d_weights: ?*const anyopaque, d_x: [*]const f32, d_y: [*]f32, rows: usize, cols: usize) void {
        hip_gemv(qt(qtype), d_weights, d_x, d_y, int(rows), int(cols), self.stream);
    }

    pub inline fn gemvGegluQ4_0(self: *const HipDevice, d_gate_w: ?*const anyopaque, d_up_w: ?*const anyopaque, d_x: [*]const f32, d_act_out: [*]f32, rows: usize, cols: usize) void {
        hip_gemv_geglu_q4_0(d_gate_w, d_up_w, d_x, d_act_out, int(rows), int(cols), self.stream);
    }

    pub inline fn gemvQkvQ4_0(self: *const HipDevice, d_q_w: ?*const anyopaque, d_k_w: ?*const anyopaque, d_v_w: ?*const anyopaque, d_x: [*]const f32, d_q_out: [*]f32, d_k_out: [*]f32, d_v_out: [*]f32, q_rows: usize, k_rows: usize, v_rows: usize, cols: usize) void {
        hip_gemv_qkv_q4_0(d_q_w, d_k_w, d_v_w, d_x, d_q_out, d_k_out, d_v_out, int(q_rows), int(k_rows), int(v_rows), int(cols), self.stream);
    }

    pub fn gemmQ4_0(self: *const HipDevice, d_weights: ?*const anyopaque, d_x: [*]const f32, d_y: [*]f32, batch_size: usize, rows: usize, cols: usize) void {
        hip_gemm_q4_0(d_weights, d_x, d_y, int(batch_size), int(rows), int(cols), self.stream);
    }

    pub fn gemm(self: *const HipDevice, qtype: GGMLType, d_weights: ?*const anyopaque, d_x: [*]const f32, d_y: [*]f32, batch_size: usize, rows: usize, cols: usize) void {
        hip_gemm(qt(qtype), d_weights, d_x, d_y, int(batch_size), int(rows), int(cols), self.stream);
    }

    /// New: the prefill product with f32 or bf16 activations (x_dtype) and output (y_dtype:
    /// dtype_f32 / dtype_bf16); with d_up_weights, y = gelu(W x) * (U x) (gate.up GeGLU).
    /// New: f32 activations -> three bf16 term planes [3][n], gemmEx's dtype_f32_terms input.
    pub fn splitTerms(self: *const HipDevice, d_x: [*]const f32, d_planes: ?*anyopaque, n: usize) void {
        hip_split_terms(d_x, d_planes, @intCast(n), self.stream);
    }

    pub fn gemmEx(self: *const HipDevice, qtype: GGMLType, d_weights: ?*const anyopaque, d_up_weights: ?*const anyopaque, x_dtype: c_int, d_x: ?*const anyopaque, y_dtype: c_int, d_y: ?*anyopaque, batch_size: usize, rows: usize, cols: usize) void {
        hip_gemm_ex(qt(qtype), d_weights, d_up_weights, x_dtype, d_x, y_dtype, d_y, int(batch_size), int(rows), int(cols), self.stream);
    }

    // ---- embeddings (cuda.zig:358-380) --------------------------------------------------
    pub fn embedLookup(self: *const HipDevice, d_weights: ?*const anyopaque, qtype: GGMLType, token_id: u32, d_out: [*]f32, dim: usize, scale_factor: f32) void {
        hip_embed_lookup(d_weights, qt(qtype), @intCast(token_id), d_out, int(dim), scale_factor, self.stream);
    }

    pub fn embedLookupBatch(self: *const HipDevice, d_weights: ?*const anyopaque, qtype: GGMLType, d_token_ids: [*]const c_int, d_out: [*]f32, n_tokens: usize, dim: usize, scale_factor: f32) void {
        hip_embed_lookup_batch(d_weights, qt(qtype), d_token_ids, d_out, int(n_tokens), int(dim), scale_factor, self.stream);
    }

    // ---- norms (cuda.zig:382-445) -------------------------------------------------------
    pub fn rmsNorm(self: *const HipDevice, d_x: [*]const f32, d_weight: ?[*]const f32, d_out: [*]f32, n: usize, eps: f32, use_unit_offset: bool) void {
        hip_rmsnorm(d_x, d_weight, d_out, int(n), eps, flag(use_unit_offset), self.stream);
    }

    pub fn rmsNormBatched(self: *const HipDevice, d_x: [*]f32, d_weight: ?[*]const f32, d_out: [*]f32, head_dim: usize, count: usize, eps: f32, use_unit_offset: bool) void {
        hip_rmsnorm_batched(d_x, d_weight, d_out, int(head_dim), int(count), eps, flag(use_unit_offset), self.stream);
    }

    pub fn rmsnormAdd(self: *const HipDevice, d_x: [*]f32, d_in: [*]const f32, d_weight: ?[*]const f32, n: usize, eps: f32, use_unit_offset: bool) void {
        hip_rmsnorm_add(d_x, d_in, d_weight, int(n), eps, flag(use_unit_offset), self.stream);
    }

    pub fn addRmsNorm(self: *const HipDevice, d_x: [*]f32, d_residual: [*]const f32, d_weight: ?[*]const f32, d_out: [*]f32, n: usize, eps: f32, use_unit_offset: bool) void {
        hip_add_rmsnorm(d_x, d_residual, d_weight, d_out, int(n), eps, flag(use_unit_offset), self.stream);
    }

    pub fn addRmsNormBatched(self: *const HipDevice, d_x: [*]f32, d_residual: [*]const f32, d_weight: ?[*]const f32, d_out: [*]f32, n: usize, batch_size: usize, eps: f32, use_unit_offset: bool) void {
        hip_add_rmsnorm_batched(d_x, d_residual, d_weight, d_out, int(n), int(batch_size), eps, flag(use_unit_offset), self.stream);
    }

    // ---- RoPE (cuda.zig:447-488) --------------------------------------------------------
    pub fn rope(self: *const HipDevice, d_q: ?[*]f32, d_k: ?[*]f32, pos: usize, num_heads: usize, num_kv_heads: usize, head_dim: usize, rotary_dim: usize, freq_base: f32) void {
        hip_rope(d_q, d_k, int(pos), int(num_heads), int(num_kv_heads), int(head_dim), int(rotary_dim), freq_base, self.stream);
    }

    pub fn ropeInd(self: *const HipDevice, d_q: ?[*]f32, d_k: ?[*]f32, d_pos: [*]const c_int, num_heads: usize, num_kv_heads: usize, head_dim: usize, rotary_dim: usize, freq_base: f32) void {
        hip_rope_ind(d_q, d_k, d_pos, int(num_heads), int(num_kv_heads), int(head_dim), int(rotary_dim), freq_base, self.stream);
    }

    pub fn ropeBatched(self: *const HipDevice, d_q: ?[*]f32, d_k: ?[*]f32, pos: usize, batch_size: usize, num_heads: usize, num_kv_heads: usize, head_dim: usize, rotary_dim: usize, freq_base: f32) void {
        hip_rope_batched(d_q, d_k, int(pos), int(batch_size), int(num_heads), int(num_kv_heads), int(head_dim), int(rotary_dim), freq_base, self.stream);
    }

    // ---- KV-cache append (cuda.zig:490-574) ---------------------------------------------
    pub fn kvCachePut(self: *const HipDevice, d_k_cache: [*]f32, d_v_cache: [*]f32, d_k: [*]const f32, d_v: [*]const f32, layer_idx: usize, pos: usize, max_seq: usize, n_kv_heads: usize, head_dim: usize, max_kv_dim: usize) void {
        hip_kv_cache_put(d_k_cache, d_v_cache, d_k, d_v, int(layer_idx), int(pos), int(max_seq), int(n_kv_heads), int(head_dim), int(max_kv_dim), self.stream);
    }

    pub fn kvCachePutInd(self: *const HipDevice, d_k_cache: [*]f32, d_v_cache: [*]f32, d_k: [*]const f32, d_v: [*]const f32, layer_idx: usize, d_pos: [*]const c_int, max_seq: usize, n_kv_heads: usize, head_dim: usize, max_kv_dim: usize) void {
        hip_kv_cache_put_ind(d_k_cache, d_v_cache, d_k, d_v, int(layer_idx), d_pos, int(max_seq), int(n_kv_heads), int(head_dim), int(max_kv_dim), self.stream);
    }

    pub fn kvCachePutBatched(self: *const HipDevice, d_k_cache: [*]f32, d_v_cache: [*]f32, d_k: [*]const f32, d_v: [*]const f32, layer_idx: usize, pos: usize, batch_size: usize, max_seq: usize, n_kv_heads: usize, head_dim: usize, max_kv_dim: usize) void {
        hip_kv_cache_put_batched(d_k_cache, d_v_cache, d_k, d_v, int(layer_idx), int(pos), int(batch_size), int(max_seq), int(n_kv_heads), int(head_dim), int(max_kv_dim), self.stream);
    }

    // ---- decode attention (cuda.zig:576-684) --------------------------------------------
    pub fn attentionForward(self: *const HipDevice, d_q: [*]const f32, d_k_cache: [*]const f32, d_v_cache: [*]const f32, d_out: [*]f32, donor_layer: usize, pos: usize, max_seq: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, max_kv_dim: usize, attn_scale: f32, softcap: f32, sliding_window: usize) void {
        hip_attention_forward(d_q, d_k_cache, d_v_cache, d_out, int(donor_layer), int(pos), int(max_seq), int(n_heads), int(n_kv_heads), int(head_dim), int(max_kv_dim), attn_scale, softcap, int(sliding_window), self.stream);
    }

    pub fn attentionForwardInd(self: *const HipDevice, d_q: [*]const f32, d_k_cache: [*]const f32, d_v_cache: [*]const f32, d_out: [*]f32, donor_layer: usize, d_pos: [*]const c_int, max_seq: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, max_kv_dim: usize, attn_scale: f32, softcap: f32, sliding_window: usize) void {
        hip_attention_forward_ind(d_q, d_k_cache, d_v_cache, d_out, int(donor_layer), d_pos, int(max_seq), int(n_heads), int(n_kv_heads), int(head_dim), int(max_kv_dim), attn_scale, softcap, int(sliding_window), self.stream);
    }

    pub fn attentionBatched(self: *const HipDevice, d_q: [*]const f32, d_k_cache: [*]const f32, d_v_cache: [*]const f32, d_out: [*]f32, donor_layer: usize, pos: usize, batch_size: usize, max_seq: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, max_kv_dim: usize, attn_scale: f32, softcap: f32, sliding_window: usize) void {
        hip_attention_batched(d_q, d_k_cache, d_v_cache, d_out, int(donor_layer), int(pos), int(batch_size), int(max_seq), int(n_heads), int(n_kv_heads), int(head_dim), int(max_kv_dim), attn_scale, softcap, int(sliding_window), self.stream);
    }

    // ---- activations, PLE, elementwise, argmax (cuda.zig:686-750) -----------------------
    pub fn geglu(self: *const HipDevice, d_gate: [*]const f32, d_up: [*]const f32, d_out: [*]f32, n: usize) void {
        hip_geglu(d_gate, d_up, d_out, int(n), self.stream);
    }

    pub fn swiglu(self: *const HipDevice, d_gate: [*]const f32, d_up: [*]const f32, d_out: [*]f32, n: usize) void {
        hip_swiglu(d_gate, d_up, d_out, int(n), self.stream);
    }

    pub fn pleGateGelu(self: *const HipDevice, d_ple_gate: [*]const f32, d_ple_slice: [*]const f32, d_ple_buf: [*]f32, ple_dim: usize) void {
        hip_ple_gate_gelu(d_ple_gate, d_ple_slice, d_ple_buf, int(ple_dim), self.stream);
    }

    pub fn pleCtxFuse(self: *const HipDevice, d_ctx_ple_buf: [*]f32, d_ctx_scratch: [*]const f32, n: usize, add_token_embd: bool) void {
        hip_ple_ctx_fuse(d_ctx_ple_buf, d_ctx_scratch, int(n), flag(add_token_embd), self.stream);
    }

    pub fn add(self: *const HipDevice, d_x: [*]f32, d_res: [*]const f32, n: usize) void {
        hip_add(d_x, d_res, int(n), self.stream);
    }

    pub fn scale(self: *const HipDevice, d_x: [*]f32, s: f32, n: usize) void {
        hip_scale(d_x, s, int(n), self.stream);
    }

    pub fn tanhSoftcap(self: *const HipDevice, d_x: [*]f32, cap: f32, n: usize) void {
        hip_tanh_softcap(d_x, cap, int(n), self.stream);
    }

    pub fn argmax(self: *const HipDevice, d_logits: [*]const f32, n: usize, d_out_idx: [*]c_uint) void {
        hip_argmax(d_logits, int(n), d_out_idx, self.stream);
    }

    // ---- new entry points (no CudaDevice counterpart) -----------------------------------

    /// Per-head Q/K RMSNorm, RoPE, Q written in place, rotated K and (optionally
    /// normalised) V written to the cache, for n_tokens tokens in one launch. Replaces
    /// rmsNormBatched(Q), rmsNormBatched(K), [rmsNormBatched(V)], rope(K), kvCachePut,
    /// rope(Q) (cuda_model.zig:643-662). cache_rows = rows the caller allocated
    /// (n_layers * max_seq in the reference layout); position of token t: d_pos[t], or
    /// pos_base + t when d_pos is null; cache row: d_slot[t], or layer_idx * max_seq +
    /// position when d_slot is null.
    pub fn qkNormRopeKv(self: *const HipDevice, dtype: c_int, d_q: ?*anyopaque, d_k: ?*const anyopaque, d_v: ?*const anyopaque, q_norm: ?[*]const f32, k_norm: ?[*]const f32, v_norm: bool, d_k_cache: ?*anyopaque, d_v_cache: ?*anyopaque, cache_rows: usize, layer_idx: usize, max_seq: usize, max_kv_dim: usize, d_pos: ?[*]const i32, pos_base: usize, d_slot: ?[*]const i64, n_tokens: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, rotary_dim: usize, theta: f32, freq_scale: f32, eps: f32, unit_offset: bool) void {
        hip_qk_norm_rope_kv(dtype, d_q, d_k, d_v, q_norm, k_norm, flag(v_norm), d_k_cache, d_v_cache, @intCast(cache_rows), int(layer_idx), int(max_seq), int(max_kv_dim), d_pos, int(pos_base), d_slot, int(n_tokens), int(n_heads), int(n_kv_heads), int(head_dim), int(rotary_dim), theta, freq_scale, eps, flag(unit_offset), self.stream);
    }

    /// x += norm(xb; w1); out = norm(x; w2), row-wise. The post-attention norm + addRmsNorm
    /// pair (cuda_model.zig:674-679), or the post-FFN rmsnormAdd + next input norm
    /// (cuda_model.zig:706, 583) with out = xb.
    pub fn rmsNormAddRmsNorm(self: *const HipDevice, dtype: c_int, d_x: *anyopaque, d_xb: *const anyopaque, w1: ?[*]const f32, w2: ?[*]const f32, d_out: *anyopaque, rows: usize, n: usize, eps: f32, unit_offset: bool) void {
        hip_rmsnorm_add_rmsnorm(dtype, d_x, d_xb, w1, w2, d_out, @intCast(rows), int(n), eps, flag(unit_offset), self.stream);
    }

    pub fn rmsNormRows(self: *const HipDevice, dtype: c_int, d_x: *const anyopaque, d_weight: ?[*]const f32, d_out: *anyopaque, rows: usize, n: usize, eps: f32, unit_offset: bool) void {
        hip_rmsnorm_rows(dtype, d_x, d_weight, d_out, @intCast(rows), int(n), eps, flag(unit_offset), self.stream);
    }

    pub fn addRmsNormRows(self: *const HipDevice, dtype: c_int, d_x: *anyopaque, d_residual: *const anyopaque, d_weight: ?[*]const f32, d_out: *anyopaque, rows: usize, n: usize, eps: f32, unit_offset: bool) void {
        hip_add_rmsnorm_rows(dtype, d_x, d_residual, d_weight, d_out, @intCast(rows), int(n), eps, flag(unit_offset), self.stream);
    }

    pub fn rmsnormAddRows(self: *const HipDevice, dtype: c_int, d_x: *anyopaque, d_in: *const anyopaque, d_weight: ?[*]const f32, rows: usize, n: usize, eps: f32, unit_offset: bool) void {
        hip_rmsnorm_add_rows(dtype, d_x, d_in, d_weight, @intCast(rows), int(n), eps, flag(unit_offset), self.stream);
    }

    pub fn gegluEx(self: *const HipDevice, dtype: c_int, d_gate: *const anyopaque, d_up: *const anyopaque, d_out: *anyopaque, n: usize) void {
        hip_geglu_ex(dtype, d_gate, d_up, d_out, @intCast(n), self.stream);
    }

    pub fn swigluEx(self: *const HipDevice, dtype: c_int, d_gate: *const anyopaque, d_up: *const anyopaque, d_out: *anyopaque, n: usize) void {
        hip_swiglu_ex(dtype, d_gate, d_up, d_out, @intCast(n), self.stream);
    }

    pub fn tanhSoftcapEx(self: *const HipDevice, dtype: c_int, d_x: *anyopaque, cap: f32, n: usize) void {
        hip_tanh_softcap_ex(dtype, d_x, cap, @intCast(n), self.stream);
    }

    /// out = x * s; s = 1 copies with a kernel (no memcpy node inside a captured graph).
    pub fn scaleEx(self: *const HipDevice, dtype: c_int, d_x: *const anyopaque, s: f32, d_out: *anyopaque, n: usize) void {
        hip_scale_ex(dtype, d_x, s, d_out, @intCast(n), self.stream);
    }

    /// Bounds-checked gather (ids outside [0, n_rows) give a zero row), f32 or bf16 out.
    pub fn embedGather(self: *const HipDevice, d_table: ?*const anyopaque, qtype: GGMLType, n_rows: usize, d_ids: [*]const i32, out_dtype: c_int, d_out: *anyopaque, n_tokens: usize, dim: usize, scale_factor: f32) void {
        hip_embed_gather(d_table, qt(qtype), @intCast(n_rows), d_ids, out_dtype, d_out, @intCast(n_tokens), int(dim), scale_factor, self.stream);
    }

    pub fn attentionWorkspaceBytes(self: *const HipDevice, batch: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, max_len: usize, sliding_window: usize) usize {
        _ = self;
        return hip_attention_workspace_bytes(int(batch), int(n_heads), int(n_kv_heads), int(head_dim), int(max_len), int(sliding_window));
    }

    /// Batched decode attention with per-token positions and cache row bases, f32 or bf16
    /// caches, split over the sequence when a workspace of attentionWorkspaceBytes is given.
    pub fn attentionDecode(self: *const HipDevice, kv_dtype: c_int, d_q: [*]const f32, d_k_cache: ?*const anyopaque, d_v_cache: ?*const anyopaque, d_out: [*]f32, cache_rows: usize, row_stride: usize, d_row_base: ?[*]const i64, row_base: usize, d_pos: ?[*]const i32, pos_base: usize, max_len: usize, batch: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, attn_scale: f32, softcap: f32, sliding_window: usize, workspace: ?HipBuffer) void {
        const ws_ptr: ?*anyopaque = if (workspace) |w| w.ptr else null;
        const ws_len: usize = if (workspace) |w| w.size_bytes else 0;
        hip_attention_decode(kv_dtype, d_q, d_k_cache, d_v_cache, d_out, @intCast(cache_rows), @intCast(row_stride), d_row_base, @intCast(row_base), d_pos, int(pos_base), int(max_len), int(batch), int(n_heads), int(n_kv_heads), int(head_dim), attn_scale, softcap, int(sliding_window), ws_ptr, ws_len, self.stream);
    }

    /// attentionDecode for callers that cannot allocate (graph capture, serving loops): the
    /// split partials live in the library's static 32 MiB device scratch; a call needing more
    /// is not launched (lastError() = -3). Calls overlapping in time on one GPU race.
    pub fn attentionDecodeNoalloc(self: *const HipDevice, kv_dtype: c_int, d_q: [*]const f32, d_k_cache: ?*const anyopaque, d_v_cache: ?*const anyopaque, d_out: [*]f32, cache_rows: usize, row_stride: usize, d_row_base: ?[*]const i64, row_base: usize, d_pos: ?[*]const i32, pos_base: usize, max_len: usize, batch: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, attn_scale: f32, softcap: f32, sliding_window: usize) void {
        hip_attention_decode_noalloc(kv_dtype, d_q, d_k_cache, d_v_cache, d_out, @intCast(cache_rows), @intCast(row_stride), d_row_base, @intCast(row_base), d_pos, int(pos_base), int(max_len), int(batch), int(n_heads), int(n_kv_heads), int(head_dim), attn_scale, softcap, int(sliding_window), self.stream);
    }

    /// attentionDecode with the QK-norm, RoPE and KV append of the token's own row folded in
    /// (raw q / k / v in; k = v = null for KV-shared layers).
    pub fn attentionDecodeQk(self: *const HipDevice, kv_dtype: c_int, d_q: [*]const f32, d_k: ?[*]const f32, d_v: ?[*]const f32, q_norm: ?[*]const f32, k_norm: ?[*]const f32, v_norm: bool, d_k_cache: *anyopaque, d_v_cache: *anyopaque, d_out: [*]f32, cache_rows: usize, row_stride: usize, d_row_base: ?[*]const i64, row_base: usize, d_pos: ?[*]const i32, pos_base: usize, max_len: usize, batch: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize, rotary_dim: usize, theta: f32, freq_scale: f32, eps: f32, unit_offset: bool, attn_scale: f32, softcap: f32, sliding_window: usize, workspace: ?HipBuffer) void {
        const ws_ptr: ?*anyopaque = if (workspace) |w| w.ptr else null;
        const ws_len: usize = if (workspace) |w| w.size_bytes else 0;
        hip_attention_decode_qk(kv_dtype, d_q, d_k, d_v, q_norm, k_norm, flag(v_norm), d_k_cache, d_v_cache, d_out, @intCast(cache_rows), @intCast(row_stride), d_row_base, @intCast(row_base), d_pos, int(pos_base), int(max_len), int(batch), int(n_heads), int(n_kv_heads), int(head_dim), int(rotary_dim), theta, freq_scale, eps, flag(unit_offset), attn_scale, softcap, int(sliding_window), ws_ptr, ws_len, self.stream);
    }

    /// GEMV with an input prologue (norm / residual / gelu(x) * r built in the product's
    /// workgroups); up_weights non-null makes it a gate.up GeGLU product.
    pub fn gemvPro(self: *const HipDevice, qtype: GGMLType, d_weights: ?*const anyopaque, d_up_weights: ?*const anyopaque, d_x: [*]const f32, d_y: [*]f32, rows: usize, cols: usize, pro: ?*const HipGemvPrologue) void {
        hip_gemv_pro(qt(qtype), d_weights, d_up_weights, d_x, d_y, int(rows), int(cols), pro, self.stream);
    }

    pub fn gemvQkvPro(self: *const HipDevice, qtype: GGMLType, d_q_w: ?*const anyopaque, d_k_w: ?*const anyopaque, d_v_w: ?*const anyopaque, d_x: [*]const f32, d_q_out: [*]f32, d_k_out: [*]f32, d_v_out: [*]f32, q_rows: usize, k_rows: usize, v_rows: usize, cols: usize, pro: ?*const HipGemvPrologue) void {
        hip_gemv_qkv_pro(qt(qtype), d_q_w, d_k_w, d_v_w, d_x, d_q_out, d_k_out, d_v_out, int(q_rows), int(k_rows), int(v_rows), int(cols), pro, self.stream);
    }

    /// Byte fill by a kernel (safe inside a captured graph, unlike a memset node).
    pub fn fill(self: *const HipDevice, buf: HipBuffer, value: u8) !void {
        if (hip_fill_u8(buf.ptr, value, buf.size_bytes, self.stream) != 0) return error.HipFillFailed;
    }

    /// The first op error recorded on this thread since the last call (0 = none).
    pub fn lastError(self: *const HipDevice) c_int {
        _ = self;
        return hip_bridge_last_error();
    }
};
