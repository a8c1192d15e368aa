/*
 * ziglm CPU oracle, part 2: dot products, GEMV, GEMM and decode attention (reference:
 * simonproyt/ziglm, src/math.zig:25-330, 440-496, 556-616, 652-846, 1088-1106;
 * src/model.zig:658-700). TEST INFRASTRUCTURE ONLY (see ziglm_oracle.h): the
 * checker for the HIP GEMV kernels; nothing in the product library uses it.
 *
 * Zig's @Vector(8|16, f32) arithmetic is restated with GCC vector extensions, built with
 * -ffp-contract=off (Zig does not contract a*b + c to an FMA in its default float mode).
 *
 * Parity status. The dot products are sums of exactly representable products in a fixed
 * f32 order; every function here is pinned in tests/test_oracle_cpu.py by
 *   - closed forms: integer-valued inputs whose every partial sum is exact in f32, so the
 *     result must equal the exact integer dot product bit for bit (a dropped block, a
 *     wrong nibble order, sign or scale index fails);
 *   - float64: random rows within 2^-20 * sum|w_i x_i| of the exact dot product;
 *   - gemv / gemm agree with the row-wise dequantise-then-dot definition in float64.
 * What stays unpinned at the last bit is @reduce(.Add)'s lane order (restated here as
 * lane 0..N-1 in sequence, as for the norms).
 */
#include "ziglm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef float v8f __attribute__((vector_size(32)));
typedef float v16f __attribute__((vector_size(64)));

static inline v8f ld8(const float* p) {
    v8f v;
    memcpy(&v, p, sizeof(v));
    return v;
}

static inline v16f ld16f(const float* p) {
    v16f v;
    memcpy(&v, p, sizeof(v));
    return v;
}

static inline float red8(v8f v) {
    float s = v[0];
    for (int j = 1; j < 8; ++j) s += v[j];
    return s;
}

static inline float red16(v16f v) {
    float s = v[0];
    for (int j = 1; j < 16; ++j) s += v[j];
    return s;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static inline float bf16f(uint16_t u) {
    uint32_t b = (uint32_t)u << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* math.zig:25-67 dotF32F32: four 8-wide accumulators over 32-element steps, 8-wide
 * remainder into sum0, @reduce((s0+s1)+(s2+s3)), scalar tail. */
float zo_dot_f32(const float* a, const float* b, size_t n) {
    v8f s0 = {0}, s1 = {0}, s2 = {0}, s3 = {0};
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        s0 += ld8(a + i) * ld8(b + i);
        s1 += ld8(a + i + 8) * ld8(b + i + 8);
        s2 += ld8(a + i + 16) * ld8(b + i + 16);
        s3 += ld8(a + i + 24) * ld8(b + i + 24);
    }
    for (; i + 8 <= n; i += 8) s0 += ld8(a + i) * ld8(b + i);
    float total = red8((s0 + s1) + (s2 + s3));
    for (; i < n; ++i) total += a[i] * b[i];
    return total;
}

/* Rows of 16-bit floats (math.zig:69-119 dotF16F32, 121-176 dotBf16F32): the same
 * structure as dotF32F32 with each 8-element group converted exactly to f32 first. */
static float dot_half(const uint8_t* a, const float* b, size_t n, int bf) {
    v8f s0 = {0}, s1 = {0}, s2 = {0}, s3 = {0};
    float t[32];
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        for (int j = 0; j < 32; ++j) {
            const uint16_t u = rd16(a + 2 * (i + j));
            t[j] = bf ? bf16f(u) : zo_f16_to_f32(u);
        }
        s0 += ld8(t) * ld8(b + i);
        s1 += ld8(t + 8) * ld8(b + i + 8);
        s2 += ld8(t + 16) * ld8(b + i + 16);
        s3 += ld8(t + 24) * ld8(b + i + 24);
    }
    for (; i + 8 <= n; i += 8) {
        for (int j = 0; j < 8; ++j) {
            const uint16_t u = rd16(a + 2 * (i + j));
            t[j] = bf ? bf16f(u) : zo_f16_to_f32(u);
        }
        s0 += ld8(t) * ld8(b + i);
    }
    float total = red8((s0 + s1) + (s2 + s3));
    for (; i < n; ++i) {
        const uint16_t u = rd16(a + 2 * i);
        total += (bf ? bf16f(u) : zo_f16_to_f32(u)) * b[i];
    }
    return total;
}

/* math.zig:178-235 dotQ8_0F32: two 16-wide accumulators; per pair of blocks
 * sum_k += (q[0:16]*x[0:16] + q[16:32]*x[16:32]) * d_k; odd last block into sum0;
 * @reduce(sum0 + sum1). */
float zo_dot_q8_0(const uint8_t* row, const float* x, size_t n) {
    const size_t nb = n / 32;
    v16f s0 = {0}, s1 = {0};
    size_t b = 0;
    for (; b < nb; ++b) {
        const uint8_t* blk = row + b * 34;
        const float d = zo_f16_to_f32(rd16(blk));
        v16f q0, q1, vd;
        for (int j = 0; j < 16; ++j) {
            q0[j] = (float)(int8_t)blk[2 + j];
            q1[j] = (float)(int8_t)blk[2 + 16 + j];
            vd[j] = d;
        }
        const v16f acc = (q0 * ld16f(x + 32 * b) + q1 * ld16f(x + 32 * b + 16)) * vd;
        /* blocks 2k and 2k+1 go to sum0 and sum1; an odd last block to sum0 */
        if ((b & 1) == 0) s0 += acc;
        else s1 += acc;
    }
    return red16(s0 + s1);
}

/* math.zig:265-326 dotQ4_0F32: low nibbles are elements 0..15, high nibbles 16..31;
 * acc = (lo*x[0:16] + hi*x[16:32]) - 8*(x[0:16] + x[16:32]); sum_k += acc * d_k. */
float zo_dot_q4_0(const uint8_t* row, const float* x, size_t n) {
    const size_t nb = n / 32;
    v16f s0 = {0}, s1 = {0};
    v16f eight;
    for (int j = 0; j < 16; ++j) eight[j] = 8.0f;
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* blk = row + b * 18;
        const float d = zo_f16_to_f32(rd16(blk));
        v16f lo, hi, vd;
        for (int j = 0; j < 16; ++j) {
            lo[j] = (float)(blk[2 + j] & 0x0F);
            hi[j] = (float)(blk[2 + j] >> 4);
            vd[j] = d;
        }
        const v16f xa = ld16f(x + 32 * b), xb = ld16f(x + 32 * b + 16);
        const v16f acc = (lo * xa + hi * xb) - eight * (xa + xb);
        if ((b & 1) == 0) s0 += acc * vd;
        else s1 += acc * vd;
    }
    return red16(s0 + s1);
}

/* Q4_K 6-bit scale / min unpacking of a 144-byte super-block (math.zig:453-458,
 * quant.zig:285-290). */
static void q4k_scales(const uint8_t* sc, uint8_t* scales, uint8_t* mins) {
    for (int j = 0; j < 4; ++j) {
        scales[j] = sc[j] & 63;
        mins[j] = sc[j + 4] & 63;
        scales[j + 4] = (uint8_t)((sc[j + 8] & 0x0F) | ((sc[j] >> 6) << 4));
        mins[j + 4] = (uint8_t)((sc[j + 8] >> 4) | ((sc[j + 4] >> 6) << 4));
    }
}

/* math.zig:440-496 dotQ4_KF32: 144-byte super-blocks {f16 d, f16 dmin, scales[12], qs[128]};
 * 16-lane accumulator: total += (q0*(d*sc) - dmin*m) * b0 + (q1*(d*sc') - dmin*m') * b1. */
float zo_dot_q4_k(const uint8_t* row, const float* x, size_t n) {
    v16f total = {0};
    for (size_t b = 0; b < n / 256; ++b) {
        const uint8_t* blk = row + b * 144;
        const float d = zo_f16_to_f32(rd16(blk)), dmin = zo_f16_to_f32(rd16(blk + 2));
        uint8_t scales[8], mins[8];
        q4k_scales(blk + 4, scales, mins);
        const uint8_t* qs = blk + 16;
        const float* xb = x + 256 * b;
        for (int j = 0; j < 4; ++j) {
            v16f vd0, vm0, vd1, vm1;
            const float d0 = d * (float)scales[2 * j], m0 = dmin * (float)mins[2 * j];
            const float d1 = d * (float)scales[2 * j + 1], m1 = dmin * (float)mins[2 * j + 1];
            for (int k = 0; k < 16; ++k) {
                vd0[k] = d0;
                vm0[k] = m0;
                vd1[k] = d1;
                vm1[k] = m1;
            }
            for (int half = 0; half < 2; ++half) {
                const int off = half * 16;
                v16f q0, q1;
                for (int k = 0; k < 16; ++k) {
                    const uint8_t q = qs[32 * j + off + k];
                    q0[k] = (float)(q & 0x0F);
                    q1[k] = (float)(q >> 4);
                }
                const v16f b0 = ld16f(xb + 64 * j + off), b1 = ld16f(xb + 64 * j + 32 + off);
                total += (q0 * vd0 - vm0) * b0 + (q1 * vd1 - vm1) * b1;
            }
        }
    }
    return red16(total);
}

/* math.zig:556-616 dotQ6_KF32: 210-byte super-blocks {ql[128], qh[64], int8 scales[16],
 * f16 d}; total += ((q1*s1)*b1 + (q2*s2)*b2 + (q3*s3)*b3 + (q4*s4)*b4) * d. */
float zo_dot_q6_k(const uint8_t* row, const float* x, size_t n) {
    v16f total = {0};
    for (size_t b = 0; b < n / 256; ++b) {
        const uint8_t* blk = row + b * 210;
        const uint8_t* ql = blk;
        const uint8_t* qh = blk + 128;
        const int8_t* sc = (const int8_t*)(blk + 192);
        const float d = zo_f16_to_f32(rd16(blk + 208));
        v16f vd;
        for (int k = 0; k < 16; ++k) vd[k] = d;
        const float* xb = x + 256 * b;
        for (int nn = 0; nn < 2; ++nn) {
            for (int chunk = 0; chunk < 2; ++chunk) {
                const int l0 = chunk * 16, is = chunk;
                v16f q1, q2, q3, q4, s1, s2, s3, s4;
                for (int k = 0; k < 16; ++k) {
                    const int l = l0 + k;
                    const uint8_t a = ql[nn * 64 + l], a32 = ql[nn * 64 + l + 32], h = qh[nn * 32 + l];
                    q1[k] = (float)((int)((a & 0x0F) | (((h >> 0) & 3) << 4)) - 32);
                    q2[k] = (float)((int)((a32 & 0x0F) | (((h >> 2) & 3) << 4)) - 32);
                    q3[k] = (float)((int)((a >> 4) | (((h >> 4) & 3) << 4)) - 32);
                    q4[k] = (float)((int)((a32 >> 4) | (((h >> 6) & 3) << 4)) - 32);
                    s1[k] = (float)sc[nn * 8 + is + 0];
                    s2[k] = (float)sc[nn * 8 + is + 2];
                    s3[k] = (float)sc[nn * 8 + is + 4];
                    s4[k] = (float)sc[nn * 8 + is + 6];
                }
                const float* bp = xb + nn * 128 + l0;
                const v16f b1 = ld16f(bp), b2 = ld16f(bp + 32), b3 = ld16f(bp + 64), b4 = ld16f(bp + 96);
                total += (q1 * s1 * b1 + q2 * s2 * b2 + q3 * s3 * b3 + q4 * s4 * b4) * vd;
            }
        }
    }
    return red16(total);
}

/* math.zig:652-708 dotRow for the types the GPU GEMV supports. */
float zo_dot_row(int qtype, const uint8_t* row, const float* x, size_t cols) {
    switch (qtype) {
        case ZO_F32: {
            /* 4-byte aligned rows: the dotF32F32 branch (656-657) */
            if (((uintptr_t)row & 3u) == 0) return zo_dot_f32((const float*)(const void*)row, x, cols);
            float total = 0.0f; /* unaligned branch (659-664) */
            for (size_t i = 0; i < cols; ++i) {
                float f;
                memcpy(&f, row + 4 * i, 4);
                total += f * x[i];
            }
            return total;
        }
        case ZO_F16: return dot_half(row, x, cols, 0);
        case ZO_BF16: return dot_half(row, x, cols, 1);
        case ZO_Q8_0: return zo_dot_q8_0(row, x, cols);
        case ZO_Q4_0: return zo_dot_q4_0(row, x, cols);
        case ZO_Q4_K: return zo_dot_q4_k(row, x, cols);
        case ZO_Q6_K: return zo_dot_q6_k(row, x, cols);
        default: return 0.0f;
    }
}

/* math.zig:714-806 gemv: y[r] = dotRow(row r, x) (the thread pool only splits rows). */
int zo_gemv(int qtype, const uint8_t* w, const float* x, float* y, size_t rows, size_t cols) {
    const size_t rb = zo_row_bytes(qtype, cols);
    if (!rb) return -1;
    for (size_t r = 0; r < rows; ++r) y[r] = zo_dot_row(qtype, w + r * rb, x, cols);
    return 0;
}

/* math.zig:808-846 gemm: batch 1 is gemv; otherwise each row is dequantised once
 * (quant.dequantizeRow) and Y[b*rows + r] = dotF32F32(row, X[b]) (F32 weights: dotRow). */
int zo_gemm(int qtype, const uint8_t* w, const float* x, float* y, size_t batch, size_t rows,
            size_t cols) {
    if (batch == 0 || rows == 0 || cols == 0) return 0;
    if (batch == 1) return zo_gemv(qtype, w, x, y, rows, cols);
    const size_t rb = zo_row_bytes(qtype, cols);
    if (!rb) return -1;
    float* tmp = (float*)malloc(cols * sizeof(float));
    if (!tmp) return -1;
    int rc = 0;
    for (size_t r = 0; r < rows && rc == 0; ++r) {
        const uint8_t* row = w + r * rb;
        if (qtype != ZO_F32 && zo_dequantize_row(qtype, row, tmp, cols) != 0) {
            rc = -1;
            break;
        }
        for (size_t b = 0; b < batch; ++b) {
            y[b * rows + r] = qtype == ZO_F32 ? zo_dot_row(ZO_F32, row, x + b * cols, cols)
                                              : zo_dot_f32(tmp, x + b * cols, cols);
        }
    }
    free(tmp);
    return rc;
}

/* ------------------------------------------------------------------------------------ */
/* Decode attention (model.zig:658-700, math.zig:1088-1106)                                */
/* ------------------------------------------------------------------------------------ */

/* math.zig:1088-1106 softmax: max, exp(v - max) (Zig @exp f32; restated with expf),
 * sequential sum, inv = 1/sum, v *= inv. Parity unpinned at the bit level for exp. */
static void softmax_f32(float* x, size_t n) {
    if (n == 0) return;
    float m = x[0];
    for (size_t i = 1; i < n; ++i)
        if (x[i] > m) m = x[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float e = expf(x[i] - m);
        x[i] = e;
        sum += e;
    }
    const float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) x[i] *= inv;
}

/* One query token, all heads (model.zig:658-700): for head h with kv head h / (nh/nkv),
 * score_t = dotF32F32(q_h, k_t) * scale, soft-capped cap*tanh(s/cap) when cap > 0, over
 * t in [start, pos] (start = pos+1-window when window > 0 and pos+1 > window); softmax;
 * out_h = sum_t w_t v_t accumulated in t order (8-wide vectors, no contraction).
 * K/V rows: key of position t, kv head j at kc[(row0 + t) * row_stride + j*d] (the logical
 * cache layout); kv_dtype 0 f32, 1 bf16 (upconverted exactly). */
int zo_attention_token(const float* q, const void* kc, const void* vc, int kv_dtype, size_t row0,
                       size_t row_stride, size_t pos, size_t window, size_t n_heads,
                       size_t n_kv_heads, size_t d, float scale, float softcap, float* out) {
    const size_t seq = pos + 1;
    const size_t start = (window > 0 && seq > window) ? seq - window : 0;
    const size_t n = seq - start;
    const size_t group = n_kv_heads ? n_heads / n_kv_heads : 1;
    float* scores = (float*)malloc(n * sizeof(float));
    float* kv = (float*)malloc(d * sizeof(float));
    if (!scores || !kv) {
        free(scores);
        free(kv);
        return -1;
    }
    for (size_t h = 0; h < n_heads; ++h) {
        const size_t kh = h / group;
        const float* qh = q + h * d;
        for (size_t t = start; t < seq; ++t) {
            const size_t off = (row0 + t) * row_stride + kh * d;
            if (kv_dtype == 0) memcpy(kv, (const float*)kc + off, d * sizeof(float));
            else for (size_t i = 0; i < d; ++i) kv[i] = bf16f(((const uint16_t*)kc)[off + i]);
            float s = zo_dot_f32(qh, kv, d) * scale;
            if (softcap > 0.0f) s = softcap * zo_tanhf(s / softcap);
            scores[t - start] = s;
        }
        softmax_f32(scores, n);
        float* oh = out + h * d;
        memset(oh, 0, d * sizeof(float));
        for (size_t t = start; t < seq; ++t) {
            const size_t off = (row0 + t) * row_stride + kh * d;
            if (kv_dtype == 0) memcpy(kv, (const float*)vc + off, d * sizeof(float));
            else for (size_t i = 0; i < d; ++i) kv[i] = bf16f(((const uint16_t*)vc)[off + i]);
            const float w = scores[t - start];
            for (size_t i = 0; i < d; ++i) oh[i] = oh[i] + w * kv[i];
        }
    }
    free(scores);
    free(kv);
    return 0;
}

/* sampler.zig:158-170 sampleGreedy: index 0 (the pad token) is never chosen; the first
 * index of the strictly greatest value from index 1 on; n <= 1 gives 0. NaN compares false,
 * so a NaN at index 1 is kept and NaNs elsewhere are skipped. Pinned by the reference's own
 * test (sampler.zig:173-177) and by brute force in the tests. */
uint32_t zo_argmax(const float* logits, size_t n) {
    if (n <= 1) return 0;
    size_t best = 1;
    float m = logits[1];
    for (size_t i = 2; i < n; ++i) {
        if (logits[i] > m) {
            m = logits[i];
            best = i;
        }
    }
    return (uint32_t)best;
}
