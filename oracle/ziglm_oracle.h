/*
 * ziglm CPU oracle: a plain-C restatement of ziglm's CPU arithmetic for the fused
 * per-layer ops (reference: simonproyt/ziglm, src/math.zig, src/quant.zig,
 * src/model.zig, src/kv_cache.zig).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels and the
 * timed CPU baseline in bench.py. Nothing in the product library (libhip_bridge.so)
 * links, loads or calls it, and no product code path falls back to it.
 *
 * Every function cites the reference lines it restates. Parity status per function is
 * stated at its definition in ziglm_oracle.c ("pinned by ..." / "parity unpinned").
 */
#ifndef ZIGLM_ORACLE_H
#define ZIGLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (types.zig:4-31). */
enum {
    ZO_F32 = 0,
    ZO_F16 = 1,
    ZO_Q4_0 = 2,
    ZO_Q8_0 = 8,
    ZO_Q4_K = 12,
    ZO_Q6_K = 14,
    ZO_BF16 = 30,
};

/* ---- scalar conversions (quant.zig:22-40) ---- */
float zo_f16_to_f32(uint16_t h);
float zo_bf16_to_f32(uint16_t u);
uint16_t zo_f32_to_bf16(float f);
void zo_bf16_to_f32_n(const uint16_t* src, float* dst, size_t n);
void zo_f32_to_bf16_n(const float* src, uint16_t* dst, size_t n);

/* ---- quant rows + embedding gather (quant.zig:73-130, 357-385, 413-607; model.zig:494-503) ---- */
size_t zo_row_bytes(int qtype, size_t n_elements);
int zo_dequantize_row(int qtype, const uint8_t* src, float* dst, size_t n_elements);
int zo_embed_gather(const uint8_t* table, int qtype, const int32_t* ids, size_t n_tokens,
                    size_t dim, float scale, float* out);

/* ---- RMSNorm (math.zig:850-988) and residual adds (model.zig:714-716, 753-755) ---- */
void zo_rms_norm(const float* x, const float* w, float* out, size_t n, float eps, int unit_offset);
void zo_rms_norm_no_scale(const float* x, float* out, size_t n, float eps);
void zo_add(float* x, const float* r, size_t n);
void zo_add_rms_norm(float* x, const float* r, const float* w, float* out, size_t n, float eps,
                     int unit_offset);
void zo_rms_norm_add(float* x, const float* in, const float* w, size_t n, float eps, int unit_offset);

/* ---- RoPE (math.zig:1019-1078) with the explicit frequency recipe ---- */
float zo_rope_denominator(float base, size_t i, size_t eff_rotary);
void zo_rope_cos_sin(float pos_f, float denom, float* c, float* s);
void zo_apply_rope(float* q, float* k, size_t pos, size_t head_size, size_t rotary_dim,
                   size_t n_heads, size_t n_kv_heads, float freq_base, float freq_scale, int neox);

/* ---- KV append (kv_cache.zig:63-85, logical layout [layer][max_seq][max_kv_dim]) ---- */
void zo_kv_cache_put(float* k_cache, float* v_cache, const float* k, const float* v,
                     size_t layer, size_t pos, size_t max_seq, size_t n_kv_heads, size_t head_dim,
                     size_t max_kv_dim);

/* ---- Per-token QK-norm + RoPE + KV append (model.zig:562-597, 628-655) ---- */
void zo_qk_norm_rope_kv_token(float* q, float* k, float* v, const float* q_norm_w,
                              const float* k_norm_w, int v_norm, size_t pos, size_t n_heads,
                              size_t n_kv_heads, size_t head_dim, size_t rotary_dim,
                              float freq_base, float freq_scale, float eps, int unit_offset);

/* ---- tanh family (std.math.tanh f32 = musl tanhf/expm1f), GeGLU, soft-cap ---- */
float zo_expm1f(float x);
float zo_tanhf(float x);
float zo_gelu(float x);
void zo_geglu(const float* gate, const float* up, float* out, size_t n);
void zo_softcap(float* x, float cap, size_t n);
float zo_silu(float x);
void zo_swiglu(const float* gate, const float* up, float* out, size_t n);
void zo_ple_gate_gelu(const float* gate, const float* slice, float* out, size_t n);
void zo_ple_ctx_fuse(float* ctx, const float* s, size_t n, int add_token_embd);

/* ---- bf16 activation variants: upconvert, run the f32 op, round once (quant.zig:30-40) ---- */
void zo_add_rms_norm_bf16(uint16_t* x, const uint16_t* r, const float* w, uint16_t* out,
                          size_t rows, size_t n, float eps, int unit_offset);
void zo_rms_norm_bf16(const uint16_t* x, const float* w, uint16_t* out, size_t rows, size_t n,
                      float eps, int unit_offset);
void zo_rms_norm_add_rms_norm_bf16(uint16_t* x, uint16_t* xb, const float* w1, const float* w2,
                                   size_t rows, size_t n, float eps, int unit_offset);
void zo_rms_norm_add_rms_norm(float* x, float* xb, const float* w1, const float* w2, size_t rows,
                              size_t n, float eps, int unit_offset);
void zo_rms_norm_add_bf16(uint16_t* x, const uint16_t* in, const float* w, size_t rows, size_t n,
                          float eps, int unit_offset);
void zo_geglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n);
void zo_swiglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n);

/* Token-batched fused QK-norm + RoPE + KV append, f32 or bf16 (dtype: 0 f32, 1 bf16).
 * q: [T][nh][d] updated in place; k, v: [T][nkv][d] read only; the rotated K and the
 * (optionally normalised) V go to cache row slot(t) = slots ? slots[t] : layer*max_seq+pos(t),
 * pos(t) = pos ? pos[t] : pos_base + t. */
void zo_qk_norm_rope_kv(int dtype, void* q, const void* k, const void* v, const float* q_norm_w,
                        const float* k_norm_w, int v_norm, void* k_cache, void* v_cache,
                        size_t layer, size_t max_seq, size_t max_kv_dim, const int32_t* pos,
                        int64_t pos_base, const int64_t* slots, size_t n_tokens, size_t n_heads,
                        size_t n_kv_heads, size_t head_dim, size_t rotary_dim, float freq_base,
                        float freq_scale, float eps, int unit_offset);

/* ---- dot products, GEMV, GEMM (math.zig:25-330, 652-846; ziglm_oracle_gemv.c) ---- */
float zo_dot_f32(const float* a, const float* b, size_t n);
float zo_dot_q8_0(const uint8_t* row, const float* x, size_t n);
float zo_dot_q4_0(const uint8_t* row, const float* x, size_t n);
float zo_dot_q4_k(const uint8_t* row, const float* x, size_t n);
float zo_dot_q6_k(const uint8_t* row, const float* x, size_t n);
float zo_dot_row(int qtype, const uint8_t* row, const float* x, size_t cols);
/* y[r] = dotRow(W[r], x), rows of zo_row_bytes(qtype, cols) bytes. */
int zo_gemv(int qtype, const uint8_t* w, const float* x, float* y, size_t rows, size_t cols);
/* Y[b*rows + r] for X[b*cols + c]; batch 1 is zo_gemv. */
int zo_gemm(int qtype, const uint8_t* w, const float* x, float* y, size_t batch, size_t rows,
            size_t cols);

/* ---- decode attention, one query token (model.zig:658-700; ziglm_oracle_gemv.c) ---- */
int zo_attention_token(const float* q, const void* k_cache, const void* v_cache, int kv_dtype,
                       size_t row0, size_t row_stride, size_t pos, size_t window, size_t n_heads,
                       size_t n_kv_heads, size_t head_dim, float scale, float softcap, float* out);

/* ---- greedy sampling (sampler.zig:158-170) ---- */
uint32_t zo_argmax(const float* logits, size_t n);

#ifdef __cplusplus
}
#endif
#endif
