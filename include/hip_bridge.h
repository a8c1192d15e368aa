/*
 * hip_bridge -- C-ABI of ziglm's fused per-layer ops on AMD Instinct MI355X (gfx950).
 *
 * Drop-in replacement for ziglm's src/cuda_bridge.h (reference: simonproyt/ziglm). Every
 * entry point with a reference counterpart cites the declaration it replaces as
 * "replaces cuda_bridge.h:LINE" (or cuda_bridge.cu:LINE / cuda.zig:LINE where the
 * reference declares it only there). Entry points marked "new" have no counterpart: they
 * carry the bf16-activation and fused variants and the per-row position/slot addressing.
 *
 * Conventions (as the reference):
 *   - plain pointers and sizes only; the caller owns every device buffer (hip_malloc),
 *     the bridge borrows pointers and keeps no global state on the op path;
 *   - runtime calls return int: 0 = success, otherwise a hipError_t value;
 *   - ops return void, are stream-ordered on `stream` (NULL = the null stream), never
 *     allocate or synchronise (so they can be captured into a hipGraph), and return early
 *     without launching when a size is <= 0;
 *   - unsupported qtype / dtype / shape: no launch (the reference silently no-ops); the
 *     reason is recorded for hip_bridge_last_error();
 *   - in-place aliasing is allowed where the reference relies on it (noted per op);
 *   - a pointer parameter marked NULL may be NULL (its meaning is stated per op); every
 *     other pointer must point to a buffer of the stated size.
 * Numerics follow ziglm's CPU path (src/math.zig, src/quant.zig), not its CUDA kernels:
 *   - gathers are bit-exact: out = (f32(q) * d) * scale, one rounding;
 *   - RMSNorm: inv = 1/sqrt(mean + eps), out = (x*inv)*(1+w); the register-row kernels
 *     (rows of up to 16 16-byte chunks per lane, 16-byte aligned) take 1/sqrt from the
 *     hardware reciprocal square root, within 1 ulp of the reference's IEEE sqrt and
 *     divide; other rows take the IEEE form;
 *   - RoPE angles: theta = f32(pos)*freq_scale / D_i (IEEE f32 division) with
 *     D_i = f32(pow(base, f32(2i)/f32(r))) evaluated in double precision; cos/sin within
 *     1.3 ulp of the correctly rounded values (an exact double-precision reduction by pi/2,
 *     then fitted f32 polynomials);
 *   - bf16 activations: upconvert, compute in f32, round to nearest even once.
 */
#ifndef HIP_BRIDGE_H
#define HIP_BRIDGE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* HipStream_t;    /* replaces CudaStream_t    (cuda_bridge.h:10) */
typedef void* HipGraph_t;     /* replaces CudaGraph_t     (cuda_bridge.h:11) */
typedef void* HipGraphExec_t; /* replaces CudaGraphExec_t (cuda_bridge.h:12) */
typedef void* HipEvent_t;     /* new: event handle for stream timing */

/* Activation / table element types: GGML type ids (reference types.zig:4-31). */
#define HIP_BRIDGE_F32 0
#define HIP_BRIDGE_F16 1
#define HIP_BRIDGE_Q4_0 2
#define HIP_BRIDGE_Q8_0 8
#define HIP_BRIDGE_Q4_K 12
#define HIP_BRIDGE_Q6_K 14
#define HIP_BRIDGE_BF16 30
/* new: f32 activations as three bf16 term planes (hip_split_terms), an input form of
 * hip_gemm_ex only */
#define HIP_BRIDGE_F32_TERMS 256

/* hip_bridge_last_error() codes (positive values are hipError_t launch errors). */
#define HIP_BRIDGE_OK 0
#define HIP_BRIDGE_EINVAL (-1)       /* bad argument (NULL buffer, bad size); no launch */
#define HIP_BRIDGE_EUNSUPPORTED (-2) /* qtype / dtype / shape not supported; no launch */
#define HIP_BRIDGE_ESCRATCH (-3)     /* call exceeds a no-allocation entry point's static
                                        scratch; no launch */

/* ---------------------------------------------------------------------------------- */
/* Device & memory management (replaces cuda_bridge.h:15-25)                          */
/* ---------------------------------------------------------------------------------- */
int hip_device_get_info(int device_id, char* name, size_t name_len, size_t* total_vram_bytes); /* cuda_bridge.h:15 */
int hip_malloc(void** ptr, size_t bytes);                                            /* cuda_bridge.h:16 */
int hip_free(void* ptr /*NULL*/);                                                    /* cuda_bridge.h:17 */
int hip_malloc_host(void** ptr, size_t bytes);                                       /* cuda_bridge.h:18 */
int hip_free_host(void* ptr /*NULL*/);                                               /* cuda_bridge.h:19 */
int hip_memcpy_h2d(void* dst, const void* src, size_t bytes, HipStream_t stream);    /* cuda_bridge.h:20 */
int hip_memcpy_d2h(void* dst, const void* src, size_t bytes, HipStream_t stream);    /* cuda_bridge.h:21 */
int hip_memcpy_d2d(void* dst, const void* src, size_t bytes, HipStream_t stream);    /* cuda_bridge.h:22 */
int hip_stream_create(HipStream_t* stream);                                          /* cuda_bridge.h:23 */
int hip_stream_destroy(HipStream_t stream);                                          /* cuda_bridge.h:24 */
int hip_stream_sync(HipStream_t stream);                                             /* cuda_bridge.h:25 */

/* ---------------------------------------------------------------------------------- */
/* Graph management (replaces cuda_bridge.h:28-33)                                    */
/* ---------------------------------------------------------------------------------- */
int hip_graph_begin_capture(HipStream_t stream);                      /* cuda_bridge.h:28 */
int hip_graph_end_capture(HipStream_t stream, HipGraph_t* graph_out); /* cuda_bridge.h:29 */
int hip_graph_instantiate(HipGraphExec_t* exec_out, HipGraph_t graph);/* cuda_bridge.h:30 */
int hip_graph_launch(HipGraphExec_t exec, HipStream_t stream);        /* cuda_bridge.h:31 */
int hip_graph_destroy(HipGraph_t graph);                              /* cuda_bridge.h:32 */
int hip_graph_exec_destroy(HipGraphExec_t exec);                      /* cuda_bridge.h:33 */

/* ---------------------------------------------------------------------------------- */
/* New runtime helpers: events (timing), fill, error reporting                         */
/* ---------------------------------------------------------------------------------- */
int hip_event_create(HipEvent_t* event);
int hip_event_destroy(HipEvent_t event);
int hip_event_record(HipEvent_t event, HipStream_t stream);
int hip_event_sync(HipEvent_t event);
int hip_event_elapsed_ms(float* ms, HipEvent_t start, HipEvent_t stop);
/* Byte fill by a kernel (not hipMemsetAsync, so it is safe inside a captured graph). */
int hip_fill_u8(void* ptr, unsigned char value, size_t bytes, HipStream_t stream);
/* Last recorded op error on this host thread (HIP_BRIDGE_* or hipError_t); reading it
 * clears it. */
int hip_bridge_last_error(void);
const char* hip_bridge_error_string(int code);
/* Build identification string (architecture, compile flags). */
const char* hip_bridge_version(void);

/* ---------------------------------------------------------------------------------- */
/* Embedding gather + dequant + scale (replaces cuda_bridge.h:53-54)                    */
/* qtype in {F32, F16, Q4_0, Q8_0, Q6_K, BF16}; row r of the table starts at           */
/* r * row_bytes(qtype, dim). out[t][i] = dequant(table[ids[t]])[i] * scale, bit-exact  */
/* to quant.zig + model.zig:494-503.                                                   */
/* ---------------------------------------------------------------------------------- */
void hip_embed_lookup(const void* emb_weights, int qtype, int token_id, float* out, int dim,
                      float scale, HipStream_t stream);                      /* cuda_bridge.h:53 */
void hip_embed_lookup_batch(const void* emb_weights, int qtype, const int* token_ids, float* out,
                            int n_tokens, int dim, float scale, HipStream_t stream); /* cuda_bridge.h:54 */
/* new: 64-bit sizes, bounds-checked ids (ids outside [0, n_rows) give a zero row),
 * f32 or bf16 output (out_dtype). */
void hip_embed_gather(const void* table, int qtype, int64_t n_rows, const int32_t* ids,
                      int out_dtype, void* out, int64_t n_tokens, int dim, float scale,
                      HipStream_t stream);

/* ---------------------------------------------------------------------------------- */
/* RMSNorm family, f32 (replaces cuda_bridge.h:55-58, cuda_bridge.cu:2058)             */
/* weight may be NULL (scale 1, reference's no-scale norm); use_unit_offset: (1+w).     */
/* ---------------------------------------------------------------------------------- */
void hip_rmsnorm(const float* x, const float* weight /*NULL*/, float* out, int n, float eps,
                 int use_unit_offset, HipStream_t stream);                   /* cuda_bridge.h:55 */
/* count rows of head_dim; weight shared by all rows; x == out allowed. */
void hip_rmsnorm_batched(float* x, const float* weight /*NULL*/, float* out, int head_dim, int count,
                         float eps, int use_unit_offset, HipStream_t stream); /* cuda_bridge.h:56 */
/* x += residual (written back), out = norm(x); out may alias residual. */
void hip_add_rmsnorm(float* x, const float* residual, const float* weight /*NULL*/, float* out, int n,
                     float eps, int use_unit_offset, HipStream_t stream);     /* cuda_bridge.h:57 */
void hip_add_rmsnorm_batched(float* x, const float* residual, const float* weight /*NULL*/, float* out,
                             int n, int batch_size, float eps, int use_unit_offset,
                             HipStream_t stream);                            /* cuda_bridge.h:58 */
/* x += norm(in). */
void hip_rmsnorm_add(float* x, const float* in, const float* weight /*NULL*/, int n, float eps,
                     int use_unit_offset, HipStream_t stream); /* cuda_bridge.cu:2058, cuda.zig:49 */

/* new: dtype-generic row variants (dtype HIP_BRIDGE_F32 or HIP_BRIDGE_BF16 for x, residual,
 * out; weights always f32), `rows` rows of n. Semantics as the f32 ops above. */
void hip_rmsnorm_rows(int dtype, const void* x, const float* weight /*NULL*/, void* out, int64_t rows,
                      int n, float eps, int use_unit_offset, HipStream_t stream);
void hip_add_rmsnorm_rows(int dtype, void* x, const void* residual, const float* weight /*NULL*/,
                          void* out, int64_t rows, int n, float eps, int use_unit_offset,
                          HipStream_t stream);
void hip_rmsnorm_add_rows(int dtype, void* x, const void* in, const float* weight /*NULL*/,
                          int64_t rows, int n, float eps, int use_unit_offset,
                          HipStream_t stream);
/* new, fused: xb' = norm(xb; w1); x += xb'; out = norm(x; w2). This is the reference's
 * post-attention norm + addRmsNorm pair (cuda_model.zig:930-942) and also the post-FFN
 * rmsnormAdd followed by the next layer's input norm (cuda_model.zig:962-967, 840-845).
 * out may alias xb. */
void hip_rmsnorm_add_rmsnorm(int dtype, void* x, const void* xb, const float* w1 /*NULL*/,
                             const float* w2 /*NULL*/, void* out, int64_t rows, int n, float eps,
                             int use_unit_offset, HipStream_t stream);

/* ---------------------------------------------------------------------------------- */
/* RoPE, half-split (ziglm RoPEType.normal), f32, in place (replaces cuda_bridge.h:59-61) */
/* q or k may be NULL. rotary_dim 0 or > head_dim means head_dim.                       */
/* ---------------------------------------------------------------------------------- */
void hip_rope(float* q /*NULL*/, float* k /*NULL*/, int pos, int num_heads, int num_kv_heads, int head_dim,
              int rotary_dim, float freq_base, HipStream_t stream);          /* cuda_bridge.h:59 */
void hip_rope_ind(float* q /*NULL*/, float* k /*NULL*/, const int* d_pos, int num_heads, int num_kv_heads,
                  int head_dim, int rotary_dim, float freq_base, HipStream_t stream); /* cuda_bridge.h:60 */
/* token b of batch_size at position pos + b */
void hip_rope_batched(float* q /*NULL*/, float* k /*NULL*/, int pos, int batch_size, int num_heads,
                      int num_kv_heads, int head_dim, int rotary_dim, float freq_base,
                      HipStream_t stream);                                   /* cuda_bridge.h:61 */

/* ---------------------------------------------------------------------------------- */
/* KV-cache append, f32, cache layout [layer][max_seq][max_kv_dim] (cuda_bridge.h:71-112) */
/* Rows with pos outside [0, max_seq) are skipped.                                      */
/* ---------------------------------------------------------------------------------- */
void hip_kv_cache_put(float* k_cache, float* v_cache, const float* k, const float* v,
                      int layer_idx, int pos, int max_seq, int n_kv_heads, int head_dim,
                      int max_kv_dim, HipStream_t stream);                    /* cuda_bridge.h:71-83 */
void hip_kv_cache_put_ind(float* k_cache, float* v_cache, const float* k, const float* v,
                          int layer_idx, const int* d_pos, int max_seq, int n_kv_heads,
                          int head_dim, int max_kv_dim, HipStream_t stream);  /* cuda_bridge.h:85-97 */
void hip_kv_cache_put_batched(float* k_cache, float* v_cache, const float* k, const float* v,
                              int layer_idx, int pos, int batch_size, int max_seq,
                              int n_kv_heads, int head_dim, int max_kv_dim,
                              HipStream_t stream);                           /* cuda_bridge.h:99-112 */

/* ---------------------------------------------------------------------------------- */
/* new, fused attention prologue: per-head Q RMSNorm -> RoPE -> Q written in place;     */
/* per-head K RMSNorm -> RoPE -> written to the K cache; V (optionally Gemma-4 no-scale */
/* norm, v_norm=1) -> written to the V cache. Replaces the reference sequence           */
/* rmsNormBatched(Q), rmsNormBatched(K), [rmsNormBatched(V, NULL)], rope(K),            */
/* kvCachePut, rope(Q) (cuda_model.zig:643-662, 901-920, 1268-1327) with one launch.    */
/*   q: [n_tokens][num_heads][head_dim], k, v: [n_tokens][num_kv_heads][head_dim],      */
/*   dtype HIP_BRIDGE_F32 or HIP_BRIDGE_BF16 (activations and caches);                  */
/*   q_norm_w / k_norm_w: f32[head_dim] or NULL (no norm); q may be NULL (K/V only);     */
/*   k or v NULL: that cache is not written (its cache pointer is then unused; given k   */
/*   or v, k_cache or v_cache must not be NULL: EINVAL, no launch);                     */
/*   position of token t: d_pos ? d_pos[t] : pos_base + t;                              */
/*   cache row of token t: d_slot ? d_slot[t] : layer_idx*max_seq + position;           */
/*   rows outside [0, cache_rows) are not written; element (t, h, j) of K goes to        */
/*   k_cache[row*max_kv_dim + h*head_dim + j].                                          */
/* ---------------------------------------------------------------------------------- */
void hip_qk_norm_rope_kv(int dtype, void* q /*NULL*/, const void* k /*NULL*/, const void* v /*NULL*/,
                         const float* q_norm_w /*NULL*/, const float* k_norm_w /*NULL*/, int v_norm,
                         void* k_cache, void* v_cache, int64_t cache_rows, int layer_idx,
                         int max_seq, int max_kv_dim, const int32_t* d_pos /*NULL*/, int pos_base,
                         const int64_t* d_slot /*NULL*/, int n_tokens, int num_heads, int num_kv_heads,
                         int head_dim, int rotary_dim, float freq_base, float freq_scale,
                         float eps, int use_unit_offset, HipStream_t stream);

/* ---------------------------------------------------------------------------------- */
/* GEMV / small-batch GEMM, f32 activations (replaces cuda_bridge.h:36-50)              */
/* y[r] = sum_c W[r][c] * x[c]; W: rows x cols in GGML layout (Q4_0, Q8_0: cols % 32    */
/* == 0, rows of (cols/32)*18 or *34 bytes; F16/BF16/F32 rows of cols elements).        */
/* Arithmetic is ziglm's CPU definition (math.zig:25-330, 652-846): exact dequantisation */
/* and f32 sums with x kept in f32 (no Q8_1 activation quantisation as in the CUDA       */
/* kernels); the summation order differs from the CPU's.                                 */
/* ---------------------------------------------------------------------------------- */
void hip_gemv_q4_0(const void* weights, const float* x, float* y, int rows, int cols,
                   HipStream_t stream);                                     /* cuda_bridge.h:36 */
void hip_gemv_q8_0(const void* weights, const float* x, float* y, int rows, int cols,
                   HipStream_t stream);                                     /* cuda_bridge.h:37 */
void hip_gemv_q4_k(const void* weights, const float* x, float* y, int rows, int cols,
                   HipStream_t stream);                                     /* cuda_bridge.h:38 */
void hip_gemv_q6_k(const void* weights, const float* x, float* y, int rows, int cols,
                   HipStream_t stream);                                     /* cuda_bridge.h:39 */
void hip_gemv_f16(const void* weights, const float* x, float* y, int rows, int cols,
                  HipStream_t stream);                                      /* cuda_bridge.h:40 */
void hip_gemv_bf16(const void* weights, const float* x, float* y, int rows, int cols,
                   HipStream_t stream);                                     /* cuda_bridge.h:41 */
void hip_gemv_f32(const float* weights, const float* x, float* y, int rows, int cols,
                  HipStream_t stream);                       /* cuda_bridge.cu:1151, cuda.zig:39 */
/* qtype dispatch (F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q6_K); other types are a no-op +
 * EUNSUPPORTED (the reference treats every unknown type as F32). */
void hip_gemv(int qtype, const void* weights, const float* x, float* y, int rows, int cols,
              HipStream_t stream);                                          /* cuda_bridge.h:42 */
/* act_out[r] = gelu_tanh(gate_r . x) * (up_r . x) */
void hip_gemv_geglu_q4_0(const void* gate_w, const void* up_w, const float* x, float* act_out,
                         int rows, int cols, HipStream_t stream);           /* cuda_bridge.h:43 */
/* three products over one x in one launch; any of the row counts may be 0 */
void hip_gemv_qkv_q4_0(const void* q_w, const void* k_w, const void* v_w, const float* x,
                       float* q_out, float* k_out, float* v_out, int q_rows, int k_rows,
                       int v_rows, int cols, HipStream_t stream);            /* cuda_bridge.h:44 */
/* new: GEMV with an input prologue (batch 1), so the norm / residual step before a product
 * needs no launch of its own. Every workgroup builds the product's input v from x:
 *   mode HIP_GEMV_PRO_NORM:  x1 = (x + [RMSNorm(r; r_weight, r_unit_offset)]) * scale
 *                            (r NULL: x1 = x * scale; r_weight NULL: r added as is),
 *                            v = RMSNorm(x1; weight, unit_offset) (weight NULL: v = x1);
 *   mode HIP_GEMV_PRO_GEGLU: v = gelu_tanh(x) * r.
 * Workgroup 0 stores x1 to x_out and v to xb_out when they are not NULL; neither may alias
 * x or r (other workgroups are still reading them). RMSNorm is the norm kernels'
 * arithmetic: inv = 1/sqrt(mean(v^2) + eps), (v * inv) * (1 + w) or (v * inv) * w.
 * cols <= 16384, cols % 8 == 0, every vector 16-byte aligned; else EUNSUPPORTED. */
#define HIP_GEMV_PRO_NORM 1
#define HIP_GEMV_PRO_GEGLU 2
typedef struct {
    int mode;
    const float* r;
    const float* r_weight;
    int r_unit_offset;
    float scale;
    float* x_out;
    const float* weight;
    int unit_offset;
    float eps;
    float* xb_out;
} HipGemvPrologue;
/* y = W . v, or with up_weights: y[r] = gelu_tanh(W_r . v) * (U_r . v); any GEMV qtype. */
void hip_gemv_pro(int qtype, const void* weights, const void* up_weights /*NULL*/, const float* x, float* y,
                  int rows, int cols, const HipGemvPrologue* pro, HipStream_t stream);
/* Q, K, V of one qtype over one v in one launch (hip_gemv_qkv_q4_0 for any qtype). */
void hip_gemv_qkv_pro(int qtype, const void* q_w, const void* k_w, const void* v_w, const float* x,
                      float* q_out, float* k_out, float* v_out, int q_rows, int k_rows, int v_rows,
                      int cols, const HipGemvPrologue* pro, HipStream_t stream);
/* Y[b*rows + r] = W[r] . X[b*cols ...], b < batch_size (batch 1 is the GEMV). y must not
 * overlap x or the weights: deep products and small batches of long rows clear y and add two
 * halves of each dot product into it (0 + a + b, the same bits in either order) while other
 * workgroups still read x; y in device memory (float atomics). */
void hip_gemm_q4_0(const void* weights, const float* x, float* y, int batch_size, int rows,
                   int cols, HipStream_t stream);                           /* cuda_bridge.h:47 */
void hip_gemm_q8_0(const void* weights, const float* x, float* y, int batch_size, int rows,
                   int cols, HipStream_t stream);                           /* cuda_bridge.h:48 */
void hip_gemm_f16(const void* weights, const float* x, float* y, int batch_size, int rows,
                  int cols, HipStream_t stream);                            /* cuda_bridge.h:49 */
void hip_gemm(int qtype, const void* weights, const float* x, float* y, int batch_size,
              int rows, int cols, HipStream_t stream);                      /* cuda_bridge.h:50 */
/* new: the prefill product with f32, bf16 or split f32 (HIP_BRIDGE_F32_TERMS) activations
 * (x_dtype) and f32 or bf16 output (y_dtype), and
 * the gate.up GeGLU pair: with up_weights (same type and shape), y[b][r] =
 * gelu_tanh(W_r . x_b) * (U_r . x_b), the reference's two prefill GEMMs and k_geglu
 * (cuda_model.zig:1372-1387) in one launch. bf16 activations are exact matrix-core operands
 * (one term), so a bf16 norm output feeds the product directly. Q4_0, Q8_0, F16, BF16, F32
 * weights with cols % 32 == 0, Q4_K and Q6_K with cols % 256 == 0; x 16-byte aligned;
 * 128 * cols * sizeof(x element) < 4 GiB; else EUNSUPPORTED. f32 x and y without
 * up_weights is hip_gemm, which takes the matrix cores from 96 tokens for 8192 rows or more,
 * 64 for fewer rows at least 4096 deep, else 128 (Q4_K 128 / 96 / 96, Q6_K 64 / 96 / 96), and
 * the small-batch or vector kernels below. */
void hip_gemm_ex(int qtype, const void* weights, const void* up_weights /*NULL*/, int x_dtype,
                 const void* x, int y_dtype, void* y, int batch_size, int rows, int cols,
                 HipStream_t stream);
/* new: f32 activations x[n] -> three bf16 planes planes[u][n] (u = 0, 1, 2: h = bf16(x),
 * m = bf16(x - h), l = bf16(x - h - m); h + m + l carries x's 24 significant bits), the
 * HIP_BRIDGE_F32_TERMS input of hip_gemm_ex: split once and shared by every product of the
 * same activations (QKV, gate and up), the K loop then converts weights only. The products
 * equal hip_gemm's on the f32 activations bit for bit where hip_gemm runs on the matrix cores
 * (Q4_K: within f32 rounding, its min term summing the planes rather than x). n % 4 == 0, x
 * 16-byte and planes 8-byte aligned; else EUNSUPPORTED. */
void hip_split_terms(const float* x, void* planes, int64_t n, HipStream_t stream);

/* ---------------------------------------------------------------------------------- */
/* Decode attention, f32 q/out (replaces cuda_bridge.h:115-168)                         */
/* Query token b at position p attends to positions [max(0, p+1-window), p] (window 0: */
/* all): score = (q_h . k_t) * attn_scale, softcap * tanh(score / softcap) when         */
/* softcap > 0, softmax, out_h = sum_t w_t v_t; kv head of query head h is              */
/* h / (n_heads / n_kv_heads) (1, 2, 4 or 8 query heads per kv head;                    */
/* head_dim 64, 128, 256 or 512).                                                       */
/* Key of (position t, kv head j) at k_cache[(row0 + t) * row_stride + j * head_dim].   */
/* ---------------------------------------------------------------------------------- */
/* reference layout, f32 cache: row0 = donor_layer * max_seq, row_stride = max_kv_dim */
void hip_attention_forward(const float* q, const float* k_cache, const float* v_cache, float* out,
                           int donor_layer, int pos, int max_seq, int n_heads, int n_kv_heads,
                           int head_dim, int max_kv_dim, float attn_scale, float softcap,
                           int sliding_window, HipStream_t stream);        /* cuda_bridge.h:115-131 */
void hip_attention_forward_ind(const float* q, const float* k_cache, const float* v_cache,
                               float* out, int donor_layer, const int* d_pos, int max_seq,
                               int n_heads, int n_kv_heads, int head_dim, int max_kv_dim,
                               float attn_scale, float softcap, int sliding_window,
                               HipStream_t stream);                        /* cuda_bridge.h:133-149 */
/* token b of batch_size at position pos + b (causal chunk of one sequence) */
void hip_attention_batched(const float* q, const float* k_cache, const float* v_cache, float* out,
                           int donor_layer, int pos, int batch_size, int max_seq, int n_heads,
                           int n_kv_heads, int head_dim, int max_kv_dim, float attn_scale,
                           float softcap, int sliding_window, HipStream_t stream); /* cuda_bridge.h:151-168 */
/* new: batched decode with per-token positions (d_pos ? d_pos[b] : pos_base + b) and cache
 * row bases (d_row_base ? d_row_base[b] : row_base), f32 or bf16 caches (kv_dtype), cache
 * bounds (cache_rows > 0; positions must also be < max_len; tokens outside give zeros) and
 * a split over the sequence when the caller passes a workspace of at least
 * hip_attention_workspace_bytes(...) bytes (16-byte aligned); with none it runs unsplit. */
size_t hip_attention_workspace_bytes(int batch, int n_heads, int n_kv_heads, int head_dim,
                                     int max_len, int sliding_window);
void hip_attention_decode(int kv_dtype, const float* q, const void* k_cache, const void* v_cache,
                          float* out, int64_t cache_rows, int64_t row_stride,
                          const int64_t* d_row_base /*NULL*/, int64_t row_base, const int32_t* d_pos /*NULL*/,
                          int pos_base, int max_len, int batch, int n_heads, int n_kv_heads,
                          int head_dim, float attn_scale, float softcap, int sliding_window,
                          void* workspace /*NULL*/, size_t workspace_bytes, HipStream_t stream);
/* new, no counterpart in the reference: hip_attention_decode for callers that cannot
 * allocate (code under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The split partials live in a static 32 MiB device array of the library, one per
 * GPU, instead of a workspace; the call allocates nothing. A call whose
 * hip_attention_workspace_bytes(batch, n_heads, n_kv_heads, head_dim, max_len,
 * sliding_window) exceeds 32 MiB is not launched and records HIP_BRIDGE_ESCRATCH (e.g. 256
 * sequences of Gemma-4B heads over 32768 positions need 68 MB: use hip_attention_decode).
 * Every call on one GPU shares that GPU's array: calls that overlap in time on one GPU
 * (different streams, or host threads) race. Nothing in the array needs to start at zero
 * (every partial the merge uses is written by the same call). The first call on a device
 * looks up the array's device address (hipGetSymbolAddress); make it outside stream capture. */
void hip_attention_decode_noalloc(int kv_dtype, const float* q, const void* k_cache, const void* v_cache,
                                  float* out, int64_t cache_rows, int64_t row_stride,
                                  const int64_t* d_row_base /*NULL*/, int64_t row_base, const int32_t* d_pos /*NULL*/,
                                  int pos_base, int max_len, int batch, int n_heads, int n_kv_heads,
                                  int head_dim, float attn_scale, float softcap, int sliding_window,
                                  HipStream_t stream);
/* new: the same call with the decode step's QK-norm + RoPE + KV append folded in (no
 * counterpart in the reference, which runs hip_qk_norm_rope_kv's three steps as separate
 * launches before attention): q holds the raw query heads (read only; not rewritten), and
 * each token's own K / V row is formed from the raw k, v [batch][n_kv_heads][head_dim]
 * (norm with k_norm_w, RoPE, v no-scale norm when v_norm) and written to its cache row
 * (row base + position), the same computation as hip_qk_norm_rope_kv's except for the order
 * of the per-head sum of squares and the inverse square root (IEEE sqrt and divide here, the
 * hardware reciprocal square root there, within 1 ulp of each other): the rows agree within
 * the oracle's tolerance, not bit for bit. Attention uses the row directly. k = v = NULL: the layer reads rows written earlier (KV-shared layers); only
 * q is normalised and rotated. Norm weights may be NULL (no norm). rotary_dim / 2 must be a
 * multiple of 8 with rotary_dim / 16 a power of two (or rotary_dim 0 = head_dim such);
 * other shapes report HIP_BRIDGE_EUNSUPPORTED. Same workspace rule as hip_attention_decode. */
void hip_attention_decode_qk(int kv_dtype, const float* q, const float* k /*NULL*/, const float* v /*NULL*/,
                             const float* q_norm_w /*NULL*/, const float* k_norm_w /*NULL*/, int v_norm,
                             void* k_cache, void* v_cache, float* out, int64_t cache_rows,
                             int64_t row_stride, const int64_t* d_row_base /*NULL*/, int64_t row_base,
                             const int32_t* d_pos /*NULL*/, int pos_base, int max_len, int batch,
                             int n_heads, int n_kv_heads, int head_dim, int rotary_dim,
                             float freq_base, float freq_scale, float eps, int use_unit_offset,
                             float attn_scale, float softcap, int sliding_window,
                             void* workspace /*NULL*/, size_t workspace_bytes, HipStream_t stream);

/* ---------------------------------------------------------------------------------- */
/* Greedy token selection (replaces cuda_bridge.h:175) with ziglm's CPU definition      */
/* (sampler.zig:158-170): *out_idx = first index of the greatest logit in [1, n) (index 0, */
/* the pad token, is never chosen; NaN never compares greater; n <= 1 gives 0).          */
/* Partials live in device globals: calls on different streams must not overlap.        */
/* ---------------------------------------------------------------------------------- */
void hip_argmax(const float* logits, int n, unsigned int* out_idx, HipStream_t stream); /* cuda_bridge.h:175 */

/* ---------------------------------------------------------------------------------- */
/* Activations & elementwise (replaces cuda_bridge.h:64, 66-68)                         */
/* ---------------------------------------------------------------------------------- */
/* out = gelu_tanh(gate) * up; out may alias gate or up. */
void hip_geglu(const float* gate, const float* up, float* out, int n, HipStream_t stream); /* cuda_bridge.h:64 */
/* out = silu(gate) * up, silu(x) = x / (1 + exp(-x)) (math.zig:1108-1117); out may alias gate
 * or up. */
void hip_swiglu(const float* gate, const float* up, float* out, int n, HipStream_t stream); /* cuda_bridge.h:65 */
void hip_add(float* x, const float* residual, int n, HipStream_t stream);              /* cuda_bridge.h:66 */
void hip_scale(float* x, float scale, int n, HipStream_t stream);                      /* cuda_bridge.h:67 */
/* x = cap * tanh(x / cap), in place. */
void hip_tanh_softcap(float* x, float cap, int n, HipStream_t stream);                 /* cuda_bridge.h:68 */
/* new: dtype-generic, 64-bit sizes. */
void hip_geglu_ex(int dtype, const void* gate, const void* up, void* out, int64_t n,
                  HipStream_t stream);
void hip_tanh_softcap_ex(int dtype, void* x, float cap, int64_t n, HipStream_t stream);
/* new: out[i] = x[i] * scale (x == out allowed; scale 1 copies exactly). */
void hip_scale_ex(int dtype, const void* x, float scale, void* out, int64_t n, HipStream_t stream);
void hip_swiglu_ex(int dtype, const void* gate, const void* up, void* out, int64_t n,
                   HipStream_t stream);

/* ---------------------------------------------------------------------------------- */
/* Per-layer embedding (Gemma-4 PLE) steps (replaces cuda_bridge.h:171-172)             */
/* ---------------------------------------------------------------------------------- */
/* ple_buf_out[i] = gelu_tanh(ple_gate_in[i]) * ple_slice[i] (model.zig:762-768). */
void hip_ple_gate_gelu(const float* ple_gate_in, const float* ple_slice, float* ple_buf_out,
                       int ple_dim, HipStream_t stream);                     /* cuda_bridge.h:171 */
/* add_token_embd != 0: ctx_ple_buf[i] = (ctx_ple_buf[i] + ctx_scratch[i]) * f32(1/sqrt(2));
 * else ctx_ple_buf[i] = ctx_scratch[i] (model.zig:525-535; n = n_layers * 256 per token). */
void hip_ple_ctx_fuse(float* ctx_ple_buf, const float* ctx_scratch, int n, int add_token_embd,
                      HipStream_t stream);                                   /* cuda_bridge.h:172 */

/* ---------------------------------------------------------------------------------- */
/* new, measurement only (no counterpart in the reference): the practical HBM ceiling of  */
/* an op's byte mix. Reads n_in (1 or 2) streams and writes n_out (1 or 2) streams of      */
/* `bytes` each (a multiple of 16, 16-byte aligned buffers) with launch shape `shape` in   */
/* [0, hip_stream_ref_shapes()); returns 0 or an error code. out0 may equal in0 (a read-   */
/* modify-write in place, like the residual-stream updates). Shapes differ in workgroup    */
/* size, chunks per thread, load/store cache policy and store form (buffer or global      */
/* stores). The fastest shape at a given size and mix is the ceiling a fused op of that    */
/* mix is compared with.                                                                   */
/* ---------------------------------------------------------------------------------- */
int hip_stream_ref_shapes(void);
int hip_stream_ref(int n_in, int n_out, const void* in0, const void* in1 /*NULL*/, void* out0, void* out1 /*NULL*/,
                   int64_t bytes, int shape, HipStream_t stream);
/* The same kernel copying up to three pairs in one launch, dst_p = src_p over bytes_p      */
/* (a multiple of 16, 16-byte aligned buffers; bytes_p == 0: pair unused, pointers may be */
/* NULL; dst_p may equal src_p), for byte mixes whose streams differ in size (the QK op:  */
/* Q in place, K and V into the caches). interleave != 0: the pairs' workgroups are       */
/* interleaved in proportion to their sizes, else pair by pair. Returns 0 or an error.    */
int hip_stream_ref_copies(const void* src0, void* dst0, int64_t bytes0, const void* src1 /*NULL*/,
                          void* dst1 /*NULL*/, int64_t bytes1, const void* src2 /*NULL*/, void* dst2 /*NULL*/,
                          int64_t bytes2, int interleave, int shape, HipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* HIP_BRIDGE_H */
