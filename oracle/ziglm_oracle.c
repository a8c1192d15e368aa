/*
 * ziglm CPU oracle -- plain-C restatement of ziglm's CPU path for the fused per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels (tests/, __graft_entry__.smoke)
 * and the timed CPU baseline (bench.py cpu_baseline). The product library never links,
 * loads or calls this code.
 *
 * Build: oracle/Makefile. Both builds use -ffp-contract=off and no fast-math, because Zig
 * never contracts a*b+c into an FMA and evaluates float expressions left to right in IEEE
 * single precision; the -O3 -march=x86-64-v3 build (the timed baseline) must agree with
 * the -O2 build bit for bit (tests/test_oracle_cpu.py checks it).
 *
 * Zig's @Vector(8, f32) is restated with GCC vector extensions (lane-wise IEEE ops, the
 * same as Zig's). @reduce(.Add, v) is restated as the ordered lane sum v0+v1+...+v7, which
 * is what LLVM's vector.reduce.fadd means without the reassoc flag.
 *
 * Parity status (what pins each function; see tests/test_oracle_cpu.py):
 *   conversions, dequant, gather, residual add, KV append ......... pinned (closed form,
 *       exhaustive f16/bf16 sweeps against numpy, brute force on tiny tables)
 *   rmsNorm / rmsNormNoScale ........................................ pinned to the
 *       mathematics (f64 closed forms, constant rows, reference test math.zig:1149-1160);
 *       lane order of @reduce is parity unpinned at the bit level (no Zig toolchain)
 *   RoPE ........................................................... pinned to the
 *       mathematics (pos 0 identity, i = 0 angle = pos, pair norm preserved, reference
 *       test math.zig:1171-1177); agreement with Zig's std.math.pow / @cos / @sin bits is
 *       parity unpinned
 *   tanh / expm1 / gelu / soft-cap .................................. pinned to the
 *       mathematics (<= 2.5 ulp of f64 tanh, <= 1 ulp expm1 over dense sweeps, odd symmetry,
 *       saturation); agreement with Zig's std.math.tanh bits is parity unpinned
 */
#include "ziglm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float* p) {
    v8f v;
    memcpy(&v, p, sizeof(v));
    return v;
}

static inline void st8(float* p, v8f v) { memcpy(p, &v, sizeof(v)); }

static inline float reduce_add8(v8f v) {
    float s = v[0];
    for (int j = 1; j < 8; ++j) s += v[j];
    return s;
}

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------------------------ */
/* Conversions                                                                            */
/* ------------------------------------------------------------------------------------ */

/* quant.zig:22-24 (@floatCast f16 -> f32, exact). Pinned: exhaustive sweep vs numpy. */
float zo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f;
    uint32_t m = h & 0x3ff;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in f32 */
        float f = (float)m * 0x1p-24f;
        return sign ? -f : f;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* quant.zig:30-33 */
float zo_bf16_to_f32(uint16_t u) { return u2f((uint32_t)u << 16); }

/* quant.zig:35-40: round-to-nearest-even by bias, NaN not special-cased. */
uint16_t zo_f32_to_bf16(float f) {
    uint32_t bits = f2u(f);
    uint32_t bias = 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + bias) >> 16);
}

void zo_bf16_to_f32_n(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = zo_bf16_to_f32(src[i]);
}

void zo_f32_to_bf16_n(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = zo_f32_to_bf16(src[i]);
}

/* ------------------------------------------------------------------------------------ */
/* Quant rows and the embedding gather                                                    */
/* ------------------------------------------------------------------------------------ */

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* types.zig:113-116 (Q4_0, 18 B), 141-144 (Q8_0, 34 B), 170-175 (Q4_K, 144 B), 187-192 (Q6_K,
 * 210 B), 320-330. */
size_t zo_row_bytes(int qtype, size_t n) {
    switch (qtype) {
        case ZO_F32: return n * 4;
        case ZO_F16:
        case ZO_BF16: return n * 2;
        case ZO_Q8_0: return (n / 32) * 34;
        case ZO_Q4_0: return (n / 32) * 18;
        case ZO_Q4_K: return (n / 256) * 144;
        case ZO_Q6_K: return (n / 256) * 210;
        default: return 0;
    }
}

/* quant.zig:413-607 dequantizeRow for the types the GPU gather supports:
 *   F32 memcpy (414-426); F16 @floatCast (427-443); BF16 bits<<16 (444-450);
 *   Q8_0 f32(qs[i]) * f32(d) (quant.zig:73-79);
 *   Q4_0 f32(i32(nibble)-8) * d, low nibbles -> 0..15, high -> 16..31 (quant.zig:119-130);
 *   Q4_K f32(q) * (d * scale_j) - dmin * min_j (quant.zig:276-309);
 *   Q6_K d * f32(scale) * f32(q) (quant.zig:357-385).
 * Returns -1 for any other type (the reference zero-fills, quant.zig:603-605). */
int zo_dequantize_row(int qtype, const uint8_t* src, float* dst, size_t n) {
    switch (qtype) {
        case ZO_F32:
            memcpy(dst, src, n * 4);
            return 0;
        case ZO_F16:
            for (size_t i = 0; i < n; ++i) dst[i] = zo_f16_to_f32(rd16(src + 2 * i));
            return 0;
        case ZO_BF16:
            for (size_t i = 0; i < n; ++i) dst[i] = zo_bf16_to_f32(rd16(src + 2 * i));
            return 0;
        case ZO_Q8_0:
            for (size_t b = 0; b < n / 32; ++b) {
                const uint8_t* blk = src + b * 34;
                float d = zo_f16_to_f32(rd16(blk));
                for (int i = 0; i < 32; ++i) dst[b * 32 + i] = (float)(int8_t)blk[2 + i] * d;
            }
            return 0;
        case ZO_Q4_0:
            for (size_t b = 0; b < n / 32; ++b) {
                const uint8_t* blk = src + b * 18;
                float d = zo_f16_to_f32(rd16(blk));
                for (int i = 0; i < 16; ++i) {
                    uint8_t qs = blk[2 + i];
                    int v0 = (int)(qs & 0x0F) - 8;
                    int v1 = (int)((qs >> 4) & 0x0F) - 8;
                    dst[b * 32 + i] = (float)v0 * d;
                    dst[b * 32 + i + 16] = (float)v1 * d;
                }
            }
            return 0;
        case ZO_Q4_K:
            for (size_t b = 0; b < n / 256; ++b) {
                const uint8_t* blk = src + b * 144;
                const float d = zo_f16_to_f32(rd16(blk)), dmin = zo_f16_to_f32(rd16(blk + 2));
                const uint8_t* sc = blk + 4;
                uint8_t scales[8], mins[8];
                for (int j = 0; j < 4; ++j) {
                    scales[j] = sc[j] & 63;
                    mins[j] = sc[j + 4] & 63;
                    scales[j + 4] = (uint8_t)((sc[j + 8] & 0x0F) | ((sc[j] >> 6) << 4));
                    mins[j + 4] = (uint8_t)((sc[j + 8] >> 4) | ((sc[j + 4] >> 6) << 4));
                }
                const uint8_t* qs = blk + 16;
                float* y = dst + b * 256;
                for (int j = 0; j < 4; ++j) {
                    const float d0 = d * (float)scales[2 * j], m0 = dmin * (float)mins[2 * j];
                    const float d1 = d * (float)scales[2 * j + 1], m1 = dmin * (float)mins[2 * j + 1];
                    for (int l = 0; l < 32; ++l) {
                        const uint8_t q = qs[32 * j + l];
                        y[64 * j + l] = (float)(q & 0x0F) * d0 - m0;
                        y[64 * j + 32 + l] = (float)((q >> 4) & 0x0F) * d1 - m1;
                    }
                }
            }
            return 0;
        case ZO_Q6_K:
            for (size_t b = 0; b < n / 256; ++b) {
                const uint8_t* ql = src + b * 210;
                const uint8_t* qh = ql + 128;
                const int8_t* sc = (const int8_t*)(ql + 192);
                float d = zo_f16_to_f32(rd16(ql + 208));
                float* y = dst + b * 256;
                for (int half = 0; half < 2; ++half) {
                    for (int l = 0; l < 32; ++l) {
                        int is = l / 16;
                        uint8_t a = ql[half * 64 + l], a32 = ql[half * 64 + l + 32];
                        uint8_t h = qh[half * 32 + l];
                        int q1 = (int)((a & 0x0F) | (((h >> 0) & 3) << 4)) - 32;
                        int q2 = (int)((a32 & 0x0F) | (((h >> 2) & 3) << 4)) - 32;
                        int q3 = (int)((a >> 4) | (((h >> 4) & 3) << 4)) - 32;
                        int q4 = (int)((a32 >> 4) | (((h >> 6) & 3) << 4)) - 32;
                        const int8_t* s = sc + half * 8;
                        y[half * 128 + l + 0] = d * (float)s[is + 0] * (float)q1;
                        y[half * 128 + l + 32] = d * (float)s[is + 2] * (float)q2;
                        y[half * 128 + l + 64] = d * (float)s[is + 4] * (float)q3;
                        y[half * 128 + l + 96] = d * (float)s[is + 6] * (float)q4;
                    }
                }
            }
            return 0;
        default:
            return -1;
    }
}

/* model.zig:494-503: dequantizeRow(type, token_embd.getRow(id), x, dim), then
 * x[i] *= scale (scale = @sqrt(f32(dim)) for the Gemma family). One rounding per element
 * for Q8_0/Q4_0/BF16/F16 because q*d is exact. Returns -1 on an unsupported type. Ids are
 * not range-checked here: the tests only pass ids inside the table. */
int zo_embed_gather(const uint8_t* table, int qtype, const int32_t* ids, size_t n_tokens,
                    size_t dim, float scale, float* out) {
    size_t rb = zo_row_bytes(qtype, dim);
    if (rb == 0) return -1;
    for (size_t t = 0; t < n_tokens; ++t) {
        float* o = out + t * dim;
        if (zo_dequantize_row(qtype, table + (size_t)ids[t] * rb, o, dim) != 0) return -1;
        for (size_t i = 0; i < dim; ++i) o[i] *= scale;
    }
    return 0;
}

/* ------------------------------------------------------------------------------------ */
/* RMSNorm                                                                                */
/* ------------------------------------------------------------------------------------ */

/* math.zig:850-945. Sum of squares: four 8-wide accumulators over floor(n/32)*32
 * elements (871-881), 8-wide remainder into acc0 (883-886), @reduce of
 * (a0+a1)+(a2+a3) (888), scalar tail (890-892). mean = sum/n (894),
 * inv = 1.0/@sqrt(mean+eps) (895, IEEE sqrt then divide). Apply (x*inv)*(1+w) or
 * (x*inv)*w (897-944). x == out is allowed. */
void zo_rms_norm(const float* x, const float* w, float* out, size_t n, float eps, int uo) {
    size_t n_unroll = n / 32, i = 0;
    v8f s0 = {0}, s1 = {0}, s2 = {0}, s3 = {0};
    for (; i < n_unroll * 32; i += 32) {
        v8f a = ld8(x + i), b = ld8(x + i + 8), c = ld8(x + i + 16), d = ld8(x + i + 24);
        s0 += a * a;
        s1 += b * b;
        s2 += c * c;
        s3 += d * d;
    }
    for (; i + 8 <= n; i += 8) {
        v8f a = ld8(x + i);
        s0 += a * a;
    }
    float sum = reduce_add8((s0 + s1) + (s2 + s3));
    for (; i < n; ++i) sum += x[i] * x[i];
    float mean = sum / (float)n;
    float inv = 1.0f / sqrtf(mean + eps);

    const v8f invv = {inv, inv, inv, inv, inv, inv, inv, inv};
    const v8f one = {1, 1, 1, 1, 1, 1, 1, 1};
    i = 0;
    for (; i < n_unroll * 32; i += 32) {
        for (int u = 0; u < 4; ++u) {
            v8f a = ld8(x + i + 8 * u), wv = ld8(w + i + 8 * u);
            st8(out + i + 8 * u, uo ? (a * invv) * (one + wv) : (a * invv) * wv);
        }
    }
    for (; i + 8 <= n; i += 8) {
        v8f a = ld8(x + i), wv = ld8(w + i);
        st8(out + i, uo ? (a * invv) * (one + wv) : (a * invv) * wv);
    }
    for (; i < n; ++i) {
        float nx = x[i] * inv;
        out[i] = uo ? nx * (1.0f + w[i]) : nx * w[i];
    }
}

/* math.zig:947-988: one 8-wide accumulator (963-968), @reduce, scalar tail,
 * inv = 1.0/@sqrt(mean+eps), out = x*inv. */
void zo_rms_norm_no_scale(const float* x, float* out, size_t n, float eps) {
    size_t n_vec = n / 8, i = 0;
    v8f s = {0};
    for (; i < n_vec * 8; i += 8) {
        v8f a = ld8(x + i);
        s += a * a;
    }
    float sum = reduce_add8(s);
    for (; i < n; ++i) sum += x[i] * x[i];
    float mean = sum / (float)n;
    float inv = 1.0f / sqrtf(mean + eps);
    for (i = 0; i < n; ++i) out[i] = x[i] * inv;
}

/* model.zig:714-716 / 753-755: x[d] += xb[d] (scalar f32). */
void zo_add(float* x, const float* r, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] += r[i];
}

/* Residual add then norm of the sum (model.zig:714-723): x += r; out = rmsNorm(x). */
void zo_add_rms_norm(float* x, const float* r, const float* w, float* out, size_t n, float eps,
                     int uo) {
    zo_add(x, r, n);
    zo_rms_norm(x, w, out, n, eps, uo);
}

/* Post-FFN norm then residual add (model.zig:748-755): x += rmsNorm(in). */
void zo_rms_norm_add(float* x, const float* in, const float* w, size_t n, float eps, int uo) {
    float* tmp = (float*)malloc(n * sizeof(float));
    zo_rms_norm(in, w, tmp, n, eps, uo);
    zo_add(x, tmp, n);
    free(tmp);
}

/* Post-attention norm, residual add, pre-FFN norm (model.zig:709-723), row by row:
 * xb = rmsNorm(xb, w1); x += xb; xb = rmsNorm(x, w2). The same sequence is the post-FFN
 * norm + add (748-755) followed by the next layer's input norm (545-546). */
void zo_rms_norm_add_rms_norm(float* x, float* xb, const float* w1, const float* w2, size_t rows,
                              size_t n, float eps, int uo) {
    for (size_t r = 0; r < rows; ++r) {
        float* xr = x + r * n;
        float* br = xb + r * n;
        zo_rms_norm(br, w1, br, n, eps, uo);
        zo_add(xr, br, n);
        zo_rms_norm(xr, w2, br, n, eps, uo);
    }
}

/* ------------------------------------------------------------------------------------ */
/* RoPE                                                                                   */
/* ------------------------------------------------------------------------------------ */

/* math.zig:1058-1059 denominator std.math.pow(f32, base, e), e = f32(2i)/f32(eff).
 * Recipe fixed for this build: the f32 rounding of the double-precision power of the two
 * f32 inputs (glibc pow is accurate to < 1 ulp of double, so this is the correctly rounded
 * f32 power except when pow(base, e) lies within ~1e-16 relative of an f32 midpoint).
 * Zig's std.math.pow(f32) is not necessarily correctly rounded: parity unpinned at the
 * last bit. The HIP bridge fills its kernels' denominator table with this same function. */
float zo_rope_denominator(float base, size_t i, size_t eff) {
    float e = (float)(2 * i) / (float)eff;
    return (float)pow((double)base, (double)e);
}

/* math.zig:1059-1061: theta = pos_f / denom (IEEE f32 divide), c = @cos(theta),
 * s = @sin(theta). Recipe: f32 rounding of the double cos/sin of the f32 theta. */
void zo_rope_cos_sin(float pos_f, float denom, float* c, float* s) {
    float theta = pos_f / denom;
    *c = (float)cos((double)theta);
    *s = (float)sin((double)theta);
}

/* math.zig:1048-1078 applyRoPEHead: .normal rotates pairs (i, i+half), .neox (2i, 2i+1);
 * new0 = v0*c - v1*s, new1 = v0*s + v1*c (no FMA). */
static void rope_head(float* head, float pos_f, size_t eff, size_t half, float base, int neox) {
    for (size_t i = 0; i < half; ++i) {
        float c, s;
        zo_rope_cos_sin(pos_f, zo_rope_denominator(base, i, eff), &c, &s);
        size_t a = neox ? 2 * i : i;
        size_t b = neox ? 2 * i + 1 : i + half;
        float v0 = head[a], v1 = head[b];
        head[a] = v0 * c - v1 * s;
        head[b] = v0 * s + v1 * c;
    }
}

/* math.zig:1019-1046 applyRoPE: pos_f = f32(pos)*freq_scale (1031);
 * eff = (rotary_dim == 0 or > head_size) ? head_size : rotary_dim; half = eff/2
 * (1032-1033); only the first eff dims of each head rotate. q or k may be NULL. */
void zo_apply_rope(float* q, float* k, size_t pos, size_t head_size, size_t rotary_dim,
                   size_t n_heads, size_t n_kv_heads, float base, float freq_scale, int neox) {
    float pos_f = (float)pos * freq_scale;
    size_t eff = (rotary_dim == 0 || rotary_dim > head_size) ? head_size : rotary_dim;
    size_t half = eff / 2;
    if (q)
        for (size_t h = 0; h < n_heads; ++h) rope_head(q + h * head_size, pos_f, eff, half, base, neox);
    if (k)
        for (size_t h = 0; h < n_kv_heads; ++h)
            rope_head(k + h * head_size, pos_f, eff, half, base, neox);
}

/* kv_cache.zig:63-85 (contiguous copy of n_kv*head_dim values into row pos) in the GPU
 * cache layout [layer][max_seq][max_kv_dim] (cuda_bridge.cu:2349). Pinned: memcpy. */
void zo_kv_cache_put(float* k_cache, float* v_cache, const float* k, const float* v,
                     size_t layer, size_t pos, size_t max_seq, size_t n_kv, size_t hd,
                     size_t max_kv_dim) {
    size_t off = (layer * max_seq + pos) * max_kv_dim;
    memcpy(k_cache + off, k, n_kv * hd * sizeof(float));
    memcpy(v_cache + off, v, n_kv * hd * sizeof(float));
}

/* One token of the attention prologue in model.zig order: per-head Q RMSNorm
 * (562-567), per-head K RMSNorm (628-633), Gemma-4 V no-scale norm (635-640), RoPE on Q
 * and K (569-597, 642-653; angles by the math.zig:1019-1078 recipe). NULL weights skip
 * that norm. q, k, v are updated in place. */
void zo_qk_norm_rope_kv_token(float* q, float* k, float* v, const float* wq, const float* wk,
                              int v_norm, size_t pos, size_t nh, size_t nkv, size_t hd,
                              size_t rotary_dim, float base, float freq_scale, float eps, int uo) {
    if (wq)
        for (size_t h = 0; h < nh; ++h) zo_rms_norm(q + h * hd, wq, q + h * hd, hd, eps, uo);
    if (wk)
        for (size_t h = 0; h < nkv; ++h) zo_rms_norm(k + h * hd, wk, k + h * hd, hd, eps, uo);
    if (v_norm)
        for (size_t h = 0; h < nkv; ++h) zo_rms_norm_no_scale(v + h * hd, v + h * hd, hd, eps);
    zo_apply_rope(q, k, pos, hd, rotary_dim, nh, nkv, base, freq_scale, 0);
}

void zo_qk_norm_rope_kv(int dtype, void* q, const void* k, const void* v, const float* wq,
                        const float* wk, int v_norm, void* k_cache, void* v_cache, size_t layer,
                        size_t max_seq, size_t max_kv_dim, const int32_t* pos, int64_t pos_base,
                        const int64_t* slots, size_t n_tokens, size_t nh, size_t nkv, size_t hd,
                        size_t rotary_dim, float base, float freq_scale, float eps, int uo) {
    size_t qn = nh * hd, kn = nkv * hd;
    float* qb = (float*)malloc(qn * sizeof(float));
    float* kb = (float*)malloc(kn * sizeof(float));
    float* vb = (float*)malloc(kn * sizeof(float));
    for (size_t t = 0; t < n_tokens; ++t) {
        int64_t p = pos ? (int64_t)pos[t] : pos_base + (int64_t)t;
        int64_t slot = slots ? slots[t] : (int64_t)(layer * max_seq) + p;
        if (dtype == 0) {
            memcpy(qb, (const float*)q + t * qn, qn * 4);
            memcpy(kb, (const float*)k + t * kn, kn * 4);
            memcpy(vb, (const float*)v + t * kn, kn * 4);
        } else {
            zo_bf16_to_f32_n((const uint16_t*)q + t * qn, qb, qn);
            zo_bf16_to_f32_n((const uint16_t*)k + t * kn, kb, kn);
            zo_bf16_to_f32_n((const uint16_t*)v + t * kn, vb, kn);
        }
        zo_qk_norm_rope_kv_token(qb, kb, vb, wq, wk, v_norm, (size_t)p, nh, nkv, hd, rotary_dim,
                                 base, freq_scale, eps, uo);
        size_t off = (size_t)slot * max_kv_dim;
        if (dtype == 0) {
            memcpy((float*)q + t * qn, qb, qn * 4);
            memcpy((float*)k_cache + off, kb, kn * 4);
            memcpy((float*)v_cache + off, vb, kn * 4);
        } else {
            zo_f32_to_bf16_n(qb, (uint16_t*)q + t * qn, qn);
            zo_f32_to_bf16_n(kb, (uint16_t*)k_cache + off, kn);
            zo_f32_to_bf16_n(vb, (uint16_t*)v_cache + off, kn);
        }
    }
    free(qb);
    free(kb);
    free(vb);
}

/* ------------------------------------------------------------------------------------ */
/* tanh family                                                                            */
/* ------------------------------------------------------------------------------------ */

/* Zig 0.16 std.math.expm1(f32), which ports musl's expm1f (itself FreeBSD's s_expm1f.c,
 * Sun Microsystems' algorithm): argument reduction x = k*ln2 + r with ln2 split in
 * hi/lo parts, a rational approximation of r on [-0.5ln2, 0.5ln2] with the two-term
 * polynomial Q1, Q2, and reconstruction by 2^k. Restated from the published algorithm;
 * the Zig port itself could not be compiled here (parity unpinned at the bit level). */
float zo_expm1f(float x) {
    const float o_threshold = 8.8721679688e+01f;
    const float ln2_hi = 6.9313812256e-01f;
    const float ln2_lo = 9.0580006145e-06f;
    const float invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333212137e-2f;
    const float Q2 = 1.5807170421e-3f;
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1, twopk;
    uint32_t ux = f2u(x);
    uint32_t hx = ux & 0x7fffffffu;
    int k, sign = (int)(ux >> 31);

    if (hx >= 0x4195b844u) { /* |x| >= 27*ln2 */
        if (hx > 0x7f800000u) return x; /* NaN */
        if (sign) return -1.0f;
        if (x > o_threshold) return x * 0x1p127f;
    }
    if (hx > 0x3eb17218u) {     /* |x| > 0.5 ln2 */
        if (hx < 0x3F851592u) { /* and |x| < 1.5 ln2 */
            if (!sign) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = (int)(invln2 * x + (sign ? -0.5f : 0.5f));
            t = (float)k;
            hi = x - t * ln2_hi; /* t*ln2_hi is exact here */
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) { /* |x| < 2^-25 */
        return x;
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = 1.0f + hxs * (Q1 + hxs * Q2);
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    twopk = u2f((uint32_t)(0x7f + k) << 23);
    if (k < 0 || k > 56) {
        y = x - e + 1.0f;
        if (k == 128)
            y = y * 2.0f * 0x1p127f;
        else
            y = y * twopk;
        return y - 1.0f;
    }
    float tk = u2f((uint32_t)(0x7f - k) << 23); /* 2^-k */
    if (k < 23)
        y = (x - e + (1.0f - tk)) * twopk;
    else
        y = (x - (e + tk) + 1.0f) * twopk;
    return y;
}

/* Zig 0.16 std.math.tanh(f32), which ports musl's tanhf: with a = |x|,
 *   a > 10            -> 1
 *   a > log(3)/2      -> 1 - 2/(expm1(2a)+2)
 *   a > log(5/3)/2    -> t/(t+2),  t = expm1(2a)
 *   a >= 2^-126       -> -t/(t+2), t = expm1(-2a)
 *   else              -> a
 * and the sign of x restored. Parity unpinned against the Zig binary; pinned to f64 tanh
 * (<= 2 ulp) and its symmetries by tests/test_oracle_cpu.py. */
float zo_tanhf(float x) {
    uint32_t ux = f2u(x);
    int sign = (int)(ux >> 31);
    uint32_t w = ux & 0x7fffffffu;
    float a = u2f(w), t;
    if (w > 0x7f800000u) return x; /* NaN */
    if (w > 0x3f0c9f54u) {
        if (w > 0x41200000u) {
            t = 1.0f;
        } else {
            t = zo_expm1f(2.0f * a);
            t = 1.0f - 2.0f / (t + 2.0f);
        }
    } else if (w > 0x3e82c578u) {
        t = zo_expm1f(2.0f * a);
        t = t / (t + 2.0f);
    } else if (w >= 0x00800000u) {
        t = zo_expm1f(-2.0f * a);
        t = -t / (t + 2.0f);
    } else {
        t = a;
    }
    return sign ? -t : t;
}

/* math.zig:1119-1123: 0.5*x*(1+tanh(0.7978845608*(x + 0.044715*x*x*x))), evaluated left to
 * right in f32: ((0.044715*x)*x)*x, x + ..., k*(...), tanh, 1 + ..., (0.5*x)*(...). */
float zo_gelu(float x) {
    const float sqrt_2_over_pi = 0.7978845608f;
    const float coef = 0.044715f;
    return 0.5f * x * (1.0f + zo_tanhf(sqrt_2_over_pi * (x + coef * x * x * x)));
}

/* math.zig:1125-1130: out[i] = gelu(gate[i]) * up[i] (out may alias gate). */
void zo_geglu(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = zo_gelu(gate[i]) * up[i];
}

/* model.zig:805-810 (final) and 672-675 (attention scores): x = cap*tanh(x/cap). */
void zo_softcap(float* x, float cap, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = cap * zo_tanhf(x[i] / cap);
}

/* math.zig:1108-1110: silu(x) = x / (1.0 + @exp(-x)). ziglm links libc (build.zig:76, 92),
 * so Zig's @exp on f32 is the C library's expf: glibc's here, the same function ziglm's
 * Linux build calls (its result is correctly rounded except in rare cases; pinned against
 * the f64 exponential in tests/test_oracle_cpu.py). */
float zo_silu(float x) {
    return x / (1.0f + expf(-x));
}

/* math.zig:1112-1117: out[i] = silu(gate[i]) * up[i] (out may alias gate). */
void zo_swiglu(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = zo_silu(gate[i]) * up[i];
}

/* Per-layer embedding (PLE) injection, model.zig:762-768: gate = gelu(W_gate x) in place,
 * then ple_buf[d] = ple_slice[d] * gate[d]. */
void zo_ple_gate_gelu(const float* gate, const float* slice, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = slice[i] * zo_gelu(gate[i]);
}

/* PLE context fuse, model.zig:525-535 with the reference ABI's flag (cuda_bridge.cu:2908-2923):
 * add_token_embd: ctx[d] = (ctx[d] + s[d]) * inv_sqrt_2, inv_sqrt_2 = f32(1/sqrt(2)) (the
 * comptime `1.0 / @sqrt(2.0)` of model.zig:528 coerced to f32); else ctx[d] = s[d]. */
void zo_ple_ctx_fuse(float* ctx, const float* s, size_t n, int add_token_embd) {
    const float inv_sqrt_2 = 0.70710677f; /* 0x3F3504F3 */
    for (size_t i = 0; i < n; ++i) ctx[i] = add_token_embd ? (ctx[i] + s[i]) * inv_sqrt_2 : s[i];
}

/* ------------------------------------------------------------------------------------ */
/* bf16 activation variants: upconvert (quant.zig:30-33), f32 op, round (quant.zig:35-40)  */
/* ------------------------------------------------------------------------------------ */

void zo_add_rms_norm_bf16(uint16_t* x, const uint16_t* r, const float* w, uint16_t* out,
                          size_t rows, size_t n, float eps, int uo) {
    float* xf = (float*)malloc(n * sizeof(float));
    float* rf = (float*)malloc(n * sizeof(float));
    float* of = (float*)malloc(n * sizeof(float));
    for (size_t row = 0; row < rows; ++row) {
        zo_bf16_to_f32_n(x + row * n, xf, n);
        zo_bf16_to_f32_n(r + row * n, rf, n);
        zo_add_rms_norm(xf, rf, w, of, n, eps, uo);
        zo_f32_to_bf16_n(xf, x + row * n, n);
        zo_f32_to_bf16_n(of, out + row * n, n);
    }
    free(xf);
    free(rf);
    free(of);
}

void zo_rms_norm_bf16(const uint16_t* x, const float* w, uint16_t* out, size_t rows, size_t n,
                      float eps, int uo) {
    float* xf = (float*)malloc(n * sizeof(float));
    for (size_t row = 0; row < rows; ++row) {
        zo_bf16_to_f32_n(x + row * n, xf, n);
        zo_rms_norm(xf, w, xf, n, eps, uo);
        zo_f32_to_bf16_n(xf, out + row * n, n);
    }
    free(xf);
}

void zo_rms_norm_add_rms_norm_bf16(uint16_t* x, uint16_t* xb, const float* w1, const float* w2,
                                   size_t rows, size_t n, float eps, int uo) {
    float* xf = (float*)malloc(n * sizeof(float));
    float* bf = (float*)malloc(n * sizeof(float));
    for (size_t row = 0; row < rows; ++row) {
        zo_bf16_to_f32_n(x + row * n, xf, n);
        zo_bf16_to_f32_n(xb + row * n, bf, n);
        zo_rms_norm_add_rms_norm(xf, bf, w1, w2, 1, n, eps, uo);
        zo_f32_to_bf16_n(xf, x + row * n, n);
        zo_f32_to_bf16_n(bf, xb + row * n, n);
    }
    free(xf);
    free(bf);
}

void zo_rms_norm_add_bf16(uint16_t* x, const uint16_t* in, const float* w, size_t rows, size_t n,
                          float eps, int uo) {
    float* xf = (float*)malloc(n * sizeof(float));
    float* bf = (float*)malloc(n * sizeof(float));
    for (size_t row = 0; row < rows; ++row) {
        zo_bf16_to_f32_n(x + row * n, xf, n);
        zo_bf16_to_f32_n(in + row * n, bf, n);
        zo_rms_norm_add(xf, bf, w, n, eps, uo);
        zo_f32_to_bf16_n(xf, x + row * n, n);
    }
    free(xf);
    free(bf);
}

void zo_geglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = zo_f32_to_bf16(zo_gelu(zo_bf16_to_f32(gate[i])) * zo_bf16_to_f32(up[i]));
}

/* SwiGLU on bf16 activations: upconvert, math.zig:1112-1117 in f32, round once. */
void zo_swiglu_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = zo_f32_to_bf16(zo_silu(zo_bf16_to_f32(gate[i])) * zo_bf16_to_f32(up[i]));
}
