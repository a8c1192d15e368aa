// hip_device.hpp -- C++ host interface over the hip_bridge C-ABI, for C++ hosts.
//
// Mirrors ziglm's Zig host wrapper src/cuda.zig: HipBuffer follows CudaBuffer
// (cuda.zig:187-225: upload / copyFrom / download / deinit) and HipDevice follows
// CudaDevice (cuda.zig:227-751): same method names, argument order and meaning, one stream
// created at init, ops enqueued on it and returning nothing (launch problems are recorded
// for hip_bridge_last_error(), as the reference ignores them). Runtime failures throw
// HipBridgeError where the Zig code returns an error (CudaDeviceNotFound,
// CudaStreamCreateFailed, CudaMemcpyFailed). Header-only; link libhip_bridge.so.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "hip_bridge.h"

namespace ziglm {

enum class GGMLType : int { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q6_K = 14, BF16 = 30 };

struct HipBridgeError : std::runtime_error {
    int code;
    HipBridgeError(const std::string& what, int c)
        : std::runtime_error(what + ": " + hip_bridge_error_string(c)), code(c) {}
};

inline void check(int rc, const char* what) {
    if (rc != 0) throw HipBridgeError(what, rc);
}

// cuda.zig:187-225
struct HipBuffer {
    void* ptr = nullptr;
    size_t size_bytes = 0;

    static HipBuffer alloc(size_t bytes) {
        HipBuffer b;
        check(hip_malloc(&b.ptr, bytes), "hip_malloc");
        b.size_bytes = bytes;
        return b;
    }
    void upload(const void* host_src, size_t len, HipStream_t stream) const {
        const size_t n = len < size_bytes ? len : size_bytes;
        if (n) check(hip_memcpy_h2d(ptr, host_src, n, stream), "CudaMemcpyFailed (upload)");
    }
    void copyFrom(const HipBuffer& other, size_t copy_len, HipStream_t stream) const {
        if (copy_len) check(hip_memcpy_d2d(ptr, other.ptr, copy_len, stream), "CudaMemcpyFailed (copyFrom)");
    }
    void download(void* host_dst, size_t len, HipStream_t stream) const {
        const size_t n = len < size_bytes ? len : size_bytes;
        if (n) check(hip_memcpy_d2h(host_dst, ptr, n, stream), "CudaMemcpyFailed (download)");
    }
    float* asF32() const { return static_cast<float*>(ptr); }
    const float* asConstF32() const { return static_cast<const float*>(ptr); }
    void deinit() {
        if (ptr) hip_free(ptr);
        ptr = nullptr;
    }
};

// cuda.zig:227-751 (the fused-op surface; GEMV/GEMM/attention are not part of this library)
class HipDevice {
public:
    HipStream_t stream = nullptr;
    char name[256] = {0};
    size_t total_vram_bytes = 0;

    // cuda.zig:234-255
    HipDevice() {
        check(hip_device_get_info(0, name, sizeof(name), &total_vram_bytes), "CudaDeviceNotFound");
        check(hip_stream_create(&stream), "CudaStreamCreateFailed");
    }
    ~HipDevice() { hip_stream_destroy(stream); }
    HipDevice(const HipDevice&) = delete;
    HipDevice& operator=(const HipDevice&) = delete;

    void sync() const { check(hip_stream_sync(stream), "hip_stream_sync"); }

    // cuda.zig:281-356
    void gemv(GGMLType qtype, const void* d_weights, const float* d_x, float* d_y, size_t rows,
              size_t cols) const {
        hip_gemv((int)qtype, d_weights, d_x, d_y, (int)rows, (int)cols, stream);
    }
    void gemvGegluQ4_0(const void* d_gate_w, const void* d_up_w, const float* d_x, float* d_act_out,
                       size_t rows, size_t cols) const {
        hip_gemv_geglu_q4_0(d_gate_w, d_up_w, d_x, d_act_out, (int)rows, (int)cols, stream);
    }
    void gemvQkvQ4_0(const void* d_q_w, const void* d_k_w, const void* d_v_w, const float* d_x, float* d_q_out,
                     float* d_k_out, float* d_v_out, size_t q_rows, size_t k_rows, size_t v_rows,
                     size_t cols) const {
        hip_gemv_qkv_q4_0(d_q_w, d_k_w, d_v_w, d_x, d_q_out, d_k_out, d_v_out, (int)q_rows, (int)k_rows,
                          (int)v_rows, (int)cols, stream);
    }
    void gemmQ4_0(const void* d_weights, const float* d_x, float* d_y, size_t batch_size, size_t rows,
                  size_t cols) const {
        hip_gemm_q4_0(d_weights, d_x, d_y, (int)batch_size, (int)rows, (int)cols, stream);
    }
    void gemm(GGMLType qtype, const void* d_weights, const float* d_x, float* d_y, size_t batch_size,
              size_t rows, size_t cols) const {
        hip_gemm((int)qtype, d_weights, d_x, d_y, (int)batch_size, (int)rows, (int)cols, stream);
    }
    // new: f32 activations -> three bf16 term planes [3][n] (gemmEx's HIP_BRIDGE_F32_TERMS input)
    void splitTerms(const float* d_x, void* d_planes, size_t n) const {
        hip_split_terms(d_x, d_planes, (int64_t)n, stream);
    }
    // new: f32 / bf16 activations and output; with d_up_weights, y = gelu(W x) * (U x)
    void gemmEx(GGMLType qtype, const void* d_weights, const void* d_up_weights, int x_dtype, const void* d_x,
                int y_dtype, void* d_y, size_t batch_size, size_t rows, size_t cols) const {
        hip_gemm_ex((int)qtype, d_weights, d_up_weights, x_dtype, d_x, y_dtype, d_y, (int)batch_size, (int)rows,
                    (int)cols, stream);
    }
    // new: products with an input prologue (norm / residual add / gelu(x) * r), batch 1
    void gemvPro(GGMLType qtype, const void* d_weights, const void* d_up_weights, const float* d_x, float* d_y,
                 size_t rows, size_t cols, const HipGemvPrologue* pro) const {
        hip_gemv_pro((int)qtype, d_weights, d_up_weights, d_x, d_y, (int)rows, (int)cols, pro, stream);
    }
    void gemvQkvPro(GGMLType qtype, const void* d_q_w, const void* d_k_w, const void* d_v_w, const float* d_x,
                    float* d_q_out, float* d_k_out, float* d_v_out, size_t q_rows, size_t k_rows, size_t v_rows,
                    size_t cols, const HipGemvPrologue* pro) const {
        hip_gemv_qkv_pro((int)qtype, d_q_w, d_k_w, d_v_w, d_x, d_q_out, d_k_out, d_v_out, (int)q_rows,
                         (int)k_rows, (int)v_rows, (int)cols, pro, stream);
    }

    // cuda.zig:358-380
    void embedLookup(const void* d_weights, GGMLType qtype, uint32_t token_id, float* d_out, size_t dim,
                     float scale_factor) const {
        hip_embed_lookup(d_weights, (int)qtype, (int)token_id, d_out, (int)dim, scale_factor, stream);
    }
    void embedLookupBatch(const void* d_weights, GGMLType qtype, const int* d_token_ids, float* d_out,
                          size_t n_tokens, size_t dim, float scale_factor) const {
        hip_embed_lookup_batch(d_weights, (int)qtype, d_token_ids, d_out, (int)n_tokens, (int)dim,
                               scale_factor, stream);
    }

    // cuda.zig:383-445
    void rmsNorm(const float* d_x, const float* d_weight, float* d_out, size_t n, float eps,
                 bool use_unit_offset) const {
        hip_rmsnorm(d_x, d_weight, d_out, (int)n, eps, use_unit_offset ? 1 : 0, stream);
    }
    void rmsNormBatched(float* d_x, const float* d_weight, float* d_out, size_t head_dim, size_t count,
                        float eps, bool use_unit_offset) const {
        hip_rmsnorm_batched(d_x, d_weight, d_out, (int)head_dim, (int)count, eps, use_unit_offset ? 1 : 0, stream);
    }
    void rmsnormAdd(float* d_x, const float* d_in, const float* d_weight, size_t n, float eps,
                    bool use_unit_offset) const {
        hip_rmsnorm_add(d_x, d_in, d_weight, (int)n, eps, use_unit_offset ? 1 : 0, stream);
    }
    void addRmsNorm(float* d_x, const float* d_residual, const float* d_weight, float* d_out, size_t n,
                    float eps, bool use_unit_offset) const {
        hip_add_rmsnorm(d_x, d_residual, d_weight, d_out, (int)n, eps, use_unit_offset ? 1 : 0, stream);
    }
    void addRmsNormBatched(float* d_x, const float* d_residual, const float* d_weight, float* d_out,
                           size_t n, size_t batch_size, float eps, bool use_unit_offset) const {
        hip_add_rmsnorm_batched(d_x, d_residual, d_weight, d_out, (int)n, (int)batch_size, eps,
                                use_unit_offset ? 1 : 0, stream);
    }

    // cuda.zig:447-488
    void rope(float* d_q, float* d_k, size_t pos, size_t num_heads, size_t num_kv_heads, size_t head_dim,
              size_t rotary_dim, float freq_base) const {
        hip_rope(d_q, d_k, (int)pos, (int)num_heads, (int)num_kv_heads, (int)head_dim, (int)rotary_dim,
                 freq_base, stream);
    }
    void ropeInd(float* d_q, float* d_k, const int* d_pos, size_t num_heads, size_t num_kv_heads,
                 size_t head_dim, size_t rotary_dim, float freq_base) const {
        hip_rope_ind(d_q, d_k, d_pos, (int)num_heads, (int)num_kv_heads, (int)head_dim, (int)rotary_dim,
                     freq_base, stream);
    }
    void ropeBatched(float* d_q, float* d_k, size_t pos, size_t batch_size, size_t num_heads,
                     size_t num_kv_heads, size_t head_dim, size_t rotary_dim, float freq_base) const {
        hip_rope_batched(d_q, d_k, (int)pos, (int)batch_size, (int)num_heads, (int)num_kv_heads, (int)head_dim,
                         (int)rotary_dim, freq_base, stream);
    }

    // cuda.zig:490-574
    void kvCachePut(float* d_k_cache, float* d_v_cache, const float* d_k, const float* d_v, size_t layer_idx,
                    size_t pos, size_t max_seq, size_t n_kv_heads, size_t head_dim, size_t max_kv_dim) const {
        hip_kv_cache_put(d_k_cache, d_v_cache, d_k, d_v, (int)layer_idx, (int)pos, (int)max_seq, (int)n_kv_heads,
                         (int)head_dim, (int)max_kv_dim, stream);
    }
    void kvCachePutInd(float* d_k_cache, float* d_v_cache, const float* d_k, const float* d_v, size_t layer_idx,
                       const int* d_pos, size_t max_seq, size_t n_kv_heads, size_t head_dim,
                       size_t max_kv_dim) const {
        hip_kv_cache_put_ind(d_k_cache, d_v_cache, d_k, d_v, (int)layer_idx, d_pos, (int)max_seq,
                             (int)n_kv_heads, (int)head_dim, (int)max_kv_dim, stream);
    }
    void kvCachePutBatched(float* d_k_cache, float* d_v_cache, const float* d_k, const float* d_v,
                           size_t layer_idx, size_t pos, size_t batch_size, size_t max_seq, size_t n_kv_heads,
                           size_t head_dim, size_t max_kv_dim) const {
        hip_kv_cache_put_batched(d_k_cache, d_v_cache, d_k, d_v, (int)layer_idx, (int)pos, (int)batch_size,
                                 (int)max_seq, (int)n_kv_heads, (int)head_dim, (int)max_kv_dim, stream);
    }

    // cuda.zig:576-684
    void attentionForward(const float* d_q, const float* d_k_cache, const float* d_v_cache, float* d_out,
                          size_t donor_layer, size_t pos, size_t max_seq, size_t n_heads, size_t n_kv_heads,
                          size_t head_dim, size_t max_kv_dim, float attn_scale, float softcap,
                          size_t sliding_window) const {
        hip_attention_forward(d_q, d_k_cache, d_v_cache, d_out, (int)donor_layer, (int)pos, (int)max_seq,
                              (int)n_heads, (int)n_kv_heads, (int)head_dim, (int)max_kv_dim, attn_scale, softcap,
                              (int)sliding_window, stream);
    }
    void attentionForwardInd(const float* d_q, const float* d_k_cache, const float* d_v_cache, float* d_out,
                             size_t donor_layer, const int* d_pos, size_t max_seq, size_t n_heads,
                             size_t n_kv_heads, size_t head_dim, size_t max_kv_dim, float attn_scale,
                             float softcap, size_t sliding_window) const {
        hip_attention_forward_ind(d_q, d_k_cache, d_v_cache, d_out, (int)donor_layer, d_pos, (int)max_seq,
                                  (int)n_heads, (int)n_kv_heads, (int)head_dim, (int)max_kv_dim, attn_scale,
                                  softcap, (int)sliding_window, stream);
    }
    void attentionBatched(const float* d_q, const float* d_k_cache, const float* d_v_cache, float* d_out,
                          size_t donor_layer, size_t pos, size_t batch_size, size_t max_seq, size_t n_heads,
                          size_t n_kv_heads, size_t head_dim, size_t max_kv_dim, float attn_scale, float softcap,
                          size_t sliding_window) const {
        hip_attention_batched(d_q, d_k_cache, d_v_cache, d_out, (int)donor_layer, (int)pos, (int)batch_size,
                              (int)max_seq, (int)n_heads, (int)n_kv_heads, (int)head_dim, (int)max_kv_dim,
                              attn_scale, softcap, (int)sliding_window, stream);
    }

    // cuda.zig:743-750
    void argmax(const float* d_logits, size_t n, unsigned int* d_out_idx) const {
        hip_argmax(d_logits, (int)n, d_out_idx, stream);
    }

    // cuda.zig:686-750
    void geglu(const float* d_gate, const float* d_up, float* d_out, size_t n) const {
        hip_geglu(d_gate, d_up, d_out, (int)n, stream);
    }
    void swiglu(const float* d_gate, const float* d_up, float* d_out, size_t n) const {
        hip_swiglu(d_gate, d_up, d_out, (int)n, stream);
    }
    // cuda.zig:696-714
    void pleGateGelu(const float* d_ple_gate, const float* d_ple_slice, float* d_ple_buf, size_t ple_dim) const {
        hip_ple_gate_gelu(d_ple_gate, d_ple_slice, d_ple_buf, (int)ple_dim, stream);
    }
    void pleCtxFuse(float* d_ctx_ple_buf, const float* d_ctx_scratch, size_t n, bool add_token_embd) const {
        hip_ple_ctx_fuse(d_ctx_ple_buf, d_ctx_scratch, (int)n, add_token_embd ? 1 : 0, stream);
    }
    void add(float* d_x, const float* d_res, size_t n) const { hip_add(d_x, d_res, (int)n, stream); }
    void scale(float* d_x, float s, size_t n) const { hip_scale(d_x, s, (int)n, stream); }
    void tanhSoftcap(float* d_x, float cap, size_t n) const { hip_tanh_softcap(d_x, cap, (int)n, stream); }

    // ---- new entry points (no CudaDevice counterpart) ----------------------------------
    void qkNormRopeKv(int dtype, void* d_q, const void* d_k, const void* d_v, const float* d_q_norm_w,
                      const float* d_k_norm_w, bool v_norm, void* d_k_cache, void* d_v_cache,
                      int64_t cache_rows, size_t layer_idx, size_t max_seq, size_t max_kv_dim,
                      const int32_t* d_pos, int pos_base, const int64_t* d_slot, size_t n_tokens,
                      size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t rotary_dim,
                      float freq_base, float freq_scale, float eps, bool use_unit_offset) const {
        hip_qk_norm_rope_kv(dtype, d_q, d_k, d_v, d_q_norm_w, d_k_norm_w, v_norm ? 1 : 0, d_k_cache, d_v_cache,
                            cache_rows, (int)layer_idx, (int)max_seq, (int)max_kv_dim, d_pos, pos_base, d_slot,
                            (int)n_tokens, (int)num_heads, (int)num_kv_heads, (int)head_dim, (int)rotary_dim,
                            freq_base, freq_scale, eps, use_unit_offset ? 1 : 0, stream);
    }
    void rmsNormAddRmsNorm(int dtype, void* d_x, const void* d_xb, const float* d_w1, const float* d_w2,
                           void* d_out, int64_t rows, size_t n, float eps, bool use_unit_offset) const {
        hip_rmsnorm_add_rmsnorm(dtype, d_x, d_xb, d_w1, d_w2, d_out, rows, (int)n, eps, use_unit_offset ? 1 : 0,
                                stream);
    }
    void gegluEx(int dtype, const void* d_gate, const void* d_up, void* d_out, int64_t n) const {
        hip_geglu_ex(dtype, d_gate, d_up, d_out, n, stream);
    }
    void embedGather(const void* d_table, GGMLType qtype, int64_t n_rows, const int32_t* d_ids, int out_dtype,
                     void* d_out, int64_t n_tokens, size_t dim, float scale) const {
        hip_embed_gather(d_table, (int)qtype, n_rows, d_ids, out_dtype, d_out, n_tokens, (int)dim, scale, stream);
    }
};

}  // namespace ziglm
