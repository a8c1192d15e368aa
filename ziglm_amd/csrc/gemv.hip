// Quantised / float matrix-vector and small-batch matrix-matrix products for decode
// (replaces cuda_bridge.cu:255-605 and 1021-1445: cuda_gemv_*, cuda_gemv_geglu_q4_0,
// cuda_gemv_qkv_q4_0, cuda_gemm_*).
//
// Numerics follow ziglm's CPU path (math.zig:25-330, 652-846), not the CUDA kernels: the
// activations stay f32 (the CUDA kernels quantise them to Q8_1 first), every weight is
// dequantised exactly ((q - 8) * d, q * d, f16/bf16 -> f32) and the products are summed in
// f32. The summation order differs from the CPU's (lanes, then waves), so results agree
// with the CPU within the f32 rounding of a dot product, not bit for bit.
//
// Layout. y[b][r] = sum_c W[r][c] * x[b][c], W rows of row_bytes(qtype, cols) bytes. One
// 256-thread workgroup owns RPW consecutive rows and a tile of NB tokens; its 256 threads
// split the row into 8-column groups (thread i takes groups i, i + 256, ...), so each
// element of x is read once per workgroup and applied to all RPW rows from registers: f32 x
// is ~7x the bytes of a Q4_0 row, and this reuse keeps its L1/L2 traffic below the weight
// stream. Per group a lane loads, for Q8_0 / Q4_0, the block's f16 scale and 8 / 4 bytes of
// quants with 16-bit loads (blocks are 34 / 18 B, 2-byte aligned; the lanes of a wave read
// one contiguous span of the row), for BF16 / F16 one 16-byte chunk, for F32 two. Partial
// sums are reduced within the wave (DPP / permlane) and across the 4 waves through LDS.
// Fused forms: GeGLU pairs each gate row with its up row and writes gelu(g) * u (the
// elementwise kernels' gelu_fast); QKV treats the three matrices as one row space.
// Batch-1 Q4_0 products with 512-column multiples take k_gemv_q4b instead (one 18-byte
// block per lane from two dword-aligned loads, every weight load of a wave issued at once,
// x staged in LDS; with or without the input prologue), Q4_K and Q6_K products the same
// scheme over 64-column pieces of their super-blocks (k_gemv_q4kb, k_gemv_q6kb); the loops
// above serve every other type, shape and batch. Measured at the Gemma-4B decode shapes (us, weights cold): QKV
// 4096 x 2560 5.4 -> 4.5, O 2560 x 2048 3.5 -> 3.4, gate.up 2 x 10240 x 2560 11.8 -> 10.0,
// down 2560 x 10240 8.4 -> 7.3, LM head 262144 x 2560 110 -> 94; the same-size read-only
// streams take 2.3, 1.9, 6.0, 3.7 and 58 us. Without the dequantisation arithmetic the block
// kernel takes 3.6, 2.9, 7.8, 5.5 and 62 us: at Q4_0's 2.5 VALU instructions per weight
// the larger products are issue-bound as much as memory-bound.
#include <algorithm>
#include <type_traits>

#include "zl_common.h"
#include "zl_host.h"

namespace zl {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

enum GemvMode { GV_PLAIN = 0, GV_GEGLU = 1 };

// Input prologue (HipGemvPrologue, batch 1): every workgroup builds the product's input
// vector in LDS from x before the weight stream starts, so a norm / residual step needs no
// launch of its own. NORM: x1 = (x + [RMSNorm](r)) * scale, input = [RMSNorm](x1), with
// workgroup 0 writing x1 (x_out) and the input (xb_out) when asked; GEGLU: input =
// gelu(x) * r. The statistics are recomputed per workgroup (a few KB read from L2).
enum GemvProMode { GP_NONE = 0, GP_NORM = 1, GP_GEGLU = 2 };
constexpr int kGemvProMaxCols = 16384;  // input vector in LDS: <= 64 KB
#ifndef ZL_GEMV_PRO_GRID
#define ZL_GEMV_PRO_GRID 1024
#endif
constexpr unsigned kGemvProGrid = ZL_GEMV_PRO_GRID;
constexpr int kGemvWaveRowsMin = 65536;  // rows from which batch-1 products use k_gemv_w
constexpr int kGemvWaveColsMax = 16384;  // its x in LDS: at most 64 KB
// Tuning builds: a non-zero ZL_GEMV_FORCE sends every batch-1 product without prologue to
// k_gemv with that many rows per workgroup (> 0) or, for block types, to k_gemv_w with -F
// rows per wave (< 0); GeGLU products take half. 0 (the library) uses the rules below.
#ifndef ZL_GEMV_FORCE
#define ZL_GEMV_FORCE 0
#endif

struct GemvPro {
    int mode;
    const float* r;
    const float* r_w;
    int r_uo;
    float scale;
    float* x_out;
    const float* w;
    int uo;
    float eps;
    float* xb_out;
};

struct GemvSeg {
    const unsigned char* w;
    float* y;
    int rows;
};

struct GemvArgs {
    GemvSeg seg[3];             // one matrix, or Q/K/V sharing cols
    int nseg;
    int total_rows;
    const unsigned char* w_up;  // GeGLU: up rows, paired with seg[0]'s gate rows
    const float* x;             // [batch][cols]
    int cols;
    int64_t row_bytes;
    int batch;
    GemvPro pro;                // used by the PRO kernels only
};

// v & m, opaque to the optimiser: it would otherwise split the byte-wise mask into one
// shift-and-mask per element, where the byte conversions below take v_cvt_f32_ubyte0..3
// straight from the masked word (1 instead of 2 instructions per element).
__device__ __forceinline__ uint32_t mask_bytes(uint32_t v, uint32_t m) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(m), "v"(v));
    return r;
}

__device__ __forceinline__ uint32_t ldw16(const unsigned char* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}
// 32-bit load from a 2-byte aligned address (block quants sit at offset 2 of 18 / 34-byte
// blocks): one global_load_dword, which gfx950 serves unaligned, addressed as the row's base
// plus the lane's 32-bit offset.
typedef uint32_t u32_align2 __attribute__((aligned(2)));
__device__ __forceinline__ uint32_t ldw32_a2(const unsigned char* p) {
    return *reinterpret_cast<const u32_align2*>(p);
}
// (v & m) | c in one instruction, opaque to the optimiser like mask_bytes.
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(m), "v"(c));
    return r;
}
// v, opaque to the optimiser: a lane offset it would otherwise split into separately
// zero-extended terms (64-bit address adds per row) stays one 32-bit offset register.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ float h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Raw weight bytes behind one 8-column group of one row.
template <int QT>
struct WGroup {
    uint32_t v[QT == HIP_BRIDGE_F32 ? 8 : 4];
    // The lane's byte offsets inside a row for group g: computed once per group and shared
    // by all rows. Unsigned 32-bit, so each load is the row's (uniform) base plus a 32-bit
    // vector offset (no per-row 64-bit address arithmetic).
    struct Off {
        uint32_t a, b;
    };
    __device__ __forceinline__ static Off off(uint32_t g) {
        if constexpr (QT == HIP_BRIDGE_Q4_0) {
            const uint32_t blk = opaque((g >> 2) * 18u);
            return {blk, opaque(blk + 2u + (g & 3u) * 4u)};  // d; 4 low + 4 high nibbles
        } else if constexpr (QT == HIP_BRIDGE_Q8_0) {
            const uint32_t blk = opaque((g >> 2) * 34u);
            return {blk, opaque(blk + 2u + (g & 3u) * 8u)};
        } else if constexpr (QT == HIP_BRIDGE_F32) {
            return {32u * g, 32u * g + 16u};
        } else {  // F16, BF16
            return {16u * g, 0u};
        }
    }
    __device__ __forceinline__ void load(const unsigned char* row, const Off& o) {
        if constexpr (QT == HIP_BRIDGE_Q4_0) {
            v[0] = ldw16(row + o.a);
            v[1] = ldw32_a2(row + o.b);
        } else if constexpr (QT == HIP_BRIDGE_Q8_0) {
            v[0] = ldw16(row + o.a);
            v[1] = ldw32_a2(row + o.b);
            v[2] = ldw32_a2(row + (o.b + 4u));
        } else if constexpr (QT == HIP_BRIDGE_F32) {
            const u32x4 a = ld16(row + o.a), b = ld16(row + o.b);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const u32x4 a = ld16(row + o.a);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        }
    }
    // row: the row's base (uniform across the workgroup); g: the lane's group.
    __device__ __forceinline__ void load(const unsigned char* row, uint32_t g) { load(row, off(g)); }
    // sum_j w_j * x_j over the group's 8 columns; xa / xb are the x values of columns
    // [8g, 8g+4) and [8g+4, 8g+8), or for Q4_0 of [32b+o, +4) and [32b+16+o, +4); sx is
    // their sum. Block types take the CPU's form (math.zig:304-305): with u_j the stored
    // unsigned byte / nibble, q_j = u_j - k (k = 8 for Q4_0 nibbles; Q8_0 bytes are read
    // as u = q ^ 0x80, k = 128), d * (sum u_j x_j - k * sum x_j) -- each u_j converted by
    // one v_cvt_f32_ubyteN, sum x_j shared by every row of the workgroup.
    __device__ __forceinline__ float dot(const f32x4& xa, const f32x4& xb, float sx) const {
        const float a[4] = {xa.x, xa.y, xa.z, xa.w};
        const float b[4] = {xb.x, xb.y, xb.z, xb.w};
        if constexpr (QT == HIP_BRIDGE_Q4_0 || QT == HIP_BRIDGE_Q8_0) {
            uint32_t ua, ub;
            float k;
            if constexpr (QT == HIP_BRIDGE_Q4_0) {
                ua = mask_bytes(v[1], 0x0f0f0f0fu);       // low nibbles: columns [32b+o, +4)
                ub = mask_bytes(v[1] >> 4, 0x0f0f0f0fu);  // high nibbles: [32b+16+o, +4)
                k = 8.0f;
            } else {
                ua = v[1] ^ 0x80808080u;
                ub = v[2] ^ 0x80808080u;
                k = 128.0f;
            }
            // The first term is a product, not an fma onto 0 (the same rounding; no zeroed
            // register per row).
            float t = (float)(ua & 0xff) * a[0];
            t = fmaf((float)(ub & 0xff), b[0], t);
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                t = fmaf((float)((ua >> (8 * j)) & 0xff), a[j], t);
                t = fmaf((float)((ub >> (8 * j)) & 0xff), b[j], t);
            }
            return h2f(v[0]) * fmaf(-k, sx, t);
        } else if constexpr (QT == HIP_BRIDGE_F32) {
            float s = __uint_as_float(v[0]) * a[0];
            s = fmaf(__uint_as_float(v[4]), b[0], s);
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                s = fmaf(__uint_as_float(v[j]), a[j], s);
                s = fmaf(__uint_as_float(v[4 + j]), b[j], s);
            }
            return s;
        } else {
            float s = -0.0f;  // x + -0 == x for every x: the first fma is a product
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float w0, w1, w2, w3;
                if constexpr (QT == HIP_BRIDGE_BF16) {
                    w0 = bf16_lo(v[j]); w1 = bf16_hi(v[j]);
                    w2 = bf16_lo(v[2 + j]); w3 = bf16_hi(v[2 + j]);
                } else {
                    w0 = h2f(v[j] & 0xffff); w1 = h2f(v[j] >> 16);
                    w2 = h2f(v[2 + j] & 0xffff); w3 = h2f(v[2 + j] >> 16);
                }
                s = fmaf(w0, a[2 * j], s);
                s = fmaf(w1, a[2 * j + 1], s);
                s = fmaf(w2, b[2 * j], s);
                s = fmaf(w3, b[2 * j + 1], s);
            }
            return s;
        }
    }
};

__device__ __forceinline__ uint32_t ldw32(const unsigned char* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}

__device__ __forceinline__ float dot4u(uint32_t u, const f32x4& x) {
    // sum_k byte_k(u) * x_k, each byte through v_cvt_f32_ubyteN
    float t = (float)(u & 0xff) * x.x;
    t = fmaf((float)((u >> 8) & 0xff), x.y, t);
    t = fmaf((float)((u >> 16) & 0xff), x.z, t);
    return fmaf((float)(u >> 24), x.w, t);
}

__device__ __forceinline__ float sum4(const f32x4& x) { return (x.x + x.y) + (x.z + x.w); }

// Q4_K: 144-byte super-blocks {f16 d, f16 dmin, scales[12] (packed 6-bit scales and mins),
// qs[128]} (types.zig:170-175), rows 4-byte aligned. Group g: super-block g/32; r = g%32,
// jj = r/8 picks the 32-byte qs span shared by sub-blocks 2jj (low nibbles) and 2jj+1 (high
// nibbles), o = 4*(r%8) the lane's 4 bytes, i.e. columns [64jj+o, +4) and [64jj+32+o, +4)
// of the super-block (the same low/high split as Q4_0 blocks). Value of a nibble q of
// sub-block j: q * (d * sc_j) - dmin * m_j (math.zig:440-496), summed here as
// (d*sc_j) * sum(q x) - (dmin*m_j) * sum(x).
template <>
struct WGroup<HIP_BRIDGE_Q4_K> {
    uint32_t dm, s0, s1, s2, q, jj;
    struct Off {
        uint32_t g;
    };
    __device__ __forceinline__ static Off off(uint32_t g) { return {g}; }
    __device__ __forceinline__ void load(const unsigned char* row, const Off& o) { load(row, o.g); }
    __device__ __forceinline__ void load(const unsigned char* row, uint32_t g) {
        const uint32_t base = (g >> 5) * 144u, r = g & 31u;
        jj = r >> 3;
        dm = ldw32(row + base);
        s0 = ldw32(row + (base + 4u));
        s1 = ldw32(row + (base + 8u));
        s2 = ldw32(row + (base + 12u));
        q = ldw32(row + (base + 16u + 32u * jj + 4u * (r & 7u)));
    }
    __device__ __forceinline__ float dot(const f32x4& xa, const f32x4& xb, float) const {
        // scale / min bytes of sub-blocks 2jj and 2jj+1 (quant.zig:285-290): bytes t, t+1
        // (t = 2 (jj & 1)) of the three scale words
        const uint32_t sh = (jj & 1u) * 16u;
        const uint32_t A = s0 >> sh, Bw = s1 >> sh, C = s2 >> sh;
        uint32_t sc0, sc1, m0, m1;
        if (jj < 2) {
            sc0 = A & 63u;
            sc1 = (A >> 8) & 63u;
            m0 = Bw & 63u;
            m1 = (Bw >> 8) & 63u;
        } else {
            sc0 = (C & 15u) | (((A >> 6) & 3u) << 4);
            sc1 = ((C >> 8) & 15u) | (((A >> 14) & 3u) << 4);
            m0 = ((C >> 4) & 15u) | (((Bw >> 6) & 3u) << 4);
            m1 = ((C >> 12) & 15u) | (((Bw >> 14) & 3u) << 4);
        }
        const float d = h2f(dm & 0xffffu), dmin = h2f(dm >> 16);
        const float d0 = d * (float)sc0, d1 = d * (float)sc1;
        const float n0 = dmin * (float)m0, n1 = dmin * (float)m1;
        const float ta = dot4u(mask_bytes(q, 0x0f0f0f0fu), xa);
        const float tb = dot4u(mask_bytes(q >> 4, 0x0f0f0f0fu), xb);
        return fmaf(d0, ta, -(n0 * sum4(xa))) + fmaf(d1, tb, -(n1 * sum4(xb)));
    }
};

// Q6_K: 210-byte super-blocks {ql[128], qh[64], int8 scales[16], f16 d} (types.zig:187-192),
// 2-byte aligned. Group g: super-block g/32; r = g%32: half n = r/16, rr = r%16, l0 =
// 4*(rr/2), p = rr%2; columns [128n + 32p + l0, +4) (6-bit values from the low nibbles of
// ql[64n + 32p + l0 ..] and qh bits 2p) and that + 64 (high nibbles, qh bits 4 + 2p), scales
// 8n + l0/16 + 2p and + 4 (math.zig:556-616: d * sum over quadrants of scale * (u - 32) * x).
template <>
struct WGroup<HIP_BRIDGE_Q6_K> {
    // The loaded words are kept as loaded and combined in dot(), so that nothing waits for
    // a load before the next group's loads are issued.
    uint32_t ql, qh, wa, wb, dd, p, sh;
    struct Off {
        uint32_t oq, oh, os, od, p, sh;
    };
    __device__ __forceinline__ static Off off(uint32_t g) {
        const uint32_t base = (g >> 5) * 210u, r = g & 31u, n = r >> 4, rr = r & 15u;
        const uint32_t l0 = 4u * (rr >> 1), p = rr & 1u;
        // scale bytes ia = base + 192 + 8n + l0/16 + 2p and ia + 4: the 16-bit words at
        // ia & ~1 and ia & ~1 + 4, byte l0/16 of each
        return {opaque(base + 64u * n + 32u * p + l0), opaque(base + 128u + 32u * n + l0),
                opaque(base + 192u + 8u * n + 2u * p), opaque(base + 208u), p, (l0 >> 1) & 8u};
    }
    __device__ __forceinline__ void load(const unsigned char* row, const Off& o) {
        ql = ldw32_a2(row + o.oq);
        qh = ldw32_a2(row + o.oh);
        wa = ldw16(row + o.os);
        wb = ldw16(row + (o.os + 4u));
        dd = ldw16(row + o.od);
        p = o.p;
        sh = o.sh;
    }
    __device__ __forceinline__ void load(const unsigned char* row, uint32_t g) { load(row, off(g)); }
    __device__ __forceinline__ float dot(const f32x4& xa, const f32x4& xb, float) const {
        const uint32_t ha = (qh >> (2u * p)) & 0x03030303u, hb = (qh >> (4u + 2u * p)) & 0x03030303u;
        const uint32_t ua = mask_bytes(ql, 0x0f0f0f0fu) | (ha << 4);
        const uint32_t ub = mask_bytes(ql >> 4, 0x0f0f0f0fu) | (hb << 4);
        const float sa = (float)(int8_t)(uint8_t)(wa >> sh), sb = (float)(int8_t)(uint8_t)(wb >> sh);
        const float ta = fmaf(-32.0f, sum4(xa), dot4u(ua, xa));
        const float tb = fmaf(-32.0f, sum4(xb), dot4u(ub, xb));
        return h2f(dd) * fmaf(sa, ta, sb * tb);
    }
};

// Column offsets of the two 4-float x vectors a group multiplies.
template <int QT>
__device__ __forceinline__ void group_cols(int g, int& ca, int& cb) {
    if constexpr (QT == HIP_BRIDGE_Q4_0) {
        ca = (g >> 2) * 32 + (g & 3) * 4;  // low nibbles: elements o..o+3 of the block
        cb = ca + 16;                      // high nibbles: elements 16+o..16+o+3
    } else if constexpr (QT == HIP_BRIDGE_Q4_K) {
        const int r = g & 31;
        ca = (g >> 5) * 256 + (r >> 3) * 64 + (r & 7) * 4;
        cb = ca + 32;
    } else if constexpr (QT == HIP_BRIDGE_Q6_K) {
        const int r = g & 31, rr = r & 15;
        ca = (g >> 5) * 256 + (r >> 4) * 128 + (rr & 1) * 32 + (rr >> 1) * 4;
        cb = ca + 64;
    } else {
        ca = 8 * g;
        cb = ca + 4;
    }
}

// Sum over the workgroup (wave sums, then the 4 wave values in order); s_red[4] in LDS.
__device__ __forceinline__ float gemv_block_sum(float v, float* s_red) {
    v = group_sum<kWave>(v);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    __syncthreads();  // s_red is reused by the next reduction
    return t;
}

// Builds the input vector of a PRO product in s_x[0, cols) (cols % 4 == 0, 16-byte aligned
// operands): see GemvProMode. The RMSNorm arithmetic is the norm kernels' (rms_inv, then
// (v * inv) * (1 + w) or * w). Up to kProRegChunks 16-byte chunks per thread (cols <= 4096)
// every operand is loaded at once through range-checked loads and kept in registers (one
// memory round trip before the first reduction); wider inputs loop over the operands.
constexpr int kProRegChunks = 4;
__device__ __forceinline__ f32x4 norm_w4(const f32x4& v, float inv, const f32x4& w, int uo) {
    f32x4 o;
    o.x = uo ? (v.x * inv) * (1.0f + w.x) : (v.x * inv) * w.x;
    o.y = uo ? (v.y * inv) * (1.0f + w.y) : (v.y * inv) * w.y;
    o.z = uo ? (v.z * inv) * (1.0f + w.z) : (v.z * inv) * w.z;
    o.w = uo ? (v.w * inv) * (1.0f + w.w) : (v.w * inv) * w.w;
    return o;
}
__device__ __forceinline__ float sumsq4(const f32x4& v, float ss) {
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    return fmaf(v.w, v.w, ss);
}
// x1 = (x + [norm(r)]) * scale (the NORM prologue's first vector), from registers.
__device__ __forceinline__ f32x4 pro_x1(const GemvPro& p, const f32x4& xv, const f32x4& rv, const f32x4& rwv,
                                        float inv1) {
    float v[4] = {xv.x, xv.y, xv.z, xv.w};
    if (p.r) {
        float y[4] = {rv.x, rv.y, rv.z, rv.w};
        if (p.r_w) {
            const float w[4] = {rwv.x, rwv.y, rwv.z, rwv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float t = y[j] * inv1;
                y[j] = p.r_uo ? t * (1.0f + w[j]) : t * w[j];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = v[j] + y[j];
    }
    if (p.scale != 1.0f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = v[j] * p.scale;
    }
    return f32x4{v[0], v[1], v[2], v[3]};
}
__device__ void gemv_prologue(const GemvArgs& a, float* s_x, float* s_red) {
    const GemvPro& p = a.pro;
    const int n4 = a.cols / 4;
    const int tid = threadIdx.x;
    f32x4* sx4 = reinterpret_cast<f32x4*>(s_x);
    const bool wr = p.x_out && blockIdx.x == 0;
    if (n4 <= kProRegChunks * kGemvThreads) {
        constexpr int K = kProRegChunks;
        const uint32_t nb = (uint32_t)n4 * 16u;
        const auto rs_x = buf_rsrc(a.x, nb);
        const auto rs_r = buf_rsrc(p.r, p.r ? nb : 0u);
        f32x4 xv[K], rv[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const uint32_t o = (uint32_t)(tid + k * kGemvThreads) * 16u;
            xv[k] = bldf4(rs_x, o);
            rv[k] = bldf4(rs_r, o);
        }
        if (p.mode == GP_GEGLU) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int c = tid + k * kGemvThreads;
                if (c < n4) {
                    f32x4 o;
                    o.x = gelu_fast(xv[k].x) * rv[k].x;
                    o.y = gelu_fast(xv[k].y) * rv[k].y;
                    o.z = gelu_fast(xv[k].z) * rv[k].z;
                    o.w = gelu_fast(xv[k].w) * rv[k].w;
                    sx4[c] = o;
                }
            }
        } else {
            const auto rs_rw = buf_rsrc(p.r_w, p.r && p.r_w ? nb : 0u);
            const auto rs_w = buf_rsrc(p.w, p.w ? nb : 0u);
            f32x4 rwv[K], wv[K];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const uint32_t o = (uint32_t)(tid + k * kGemvThreads) * 16u;
                rwv[k] = bldf4(rs_rw, o);
                wv[k] = bldf4(rs_w, o);
            }
            float inv1 = 0.0f;
            if (p.r && p.r_w) {
                float ss = 0.0f;
#pragma unroll
                for (int k = 0; k < K; ++k)
                    if (tid + k * kGemvThreads < n4) ss = sumsq4(rv[k], ss);
                inv1 = rms_inv(gemv_block_sum(ss, s_red), a.cols, p.eps);
            }
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int c = tid + k * kGemvThreads;
                if (c < n4) {
                    xv[k] = pro_x1(p, xv[k], rv[k], rwv[k], inv1);
                    if (wr) *reinterpret_cast<f32x4*>(p.x_out + 4 * c) = xv[k];
                    ss = sumsq4(xv[k], ss);
                }
            }
            if (p.w) {
                const float inv2 = rms_inv(gemv_block_sum(ss, s_red), a.cols, p.eps);
#pragma unroll
                for (int k = 0; k < K; ++k) xv[k] = norm_w4(xv[k], inv2, wv[k], p.uo);
            }
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int c = tid + k * kGemvThreads;
                if (c < n4) sx4[c] = xv[k];
            }
        }
    } else if (p.mode == GP_GEGLU) {
        for (int c = tid; c < n4; c += kGemvThreads) {
            const f32x4 g = ldf4(a.x + 4 * c), u = ldf4(p.r + 4 * c);
            f32x4 o;
            o.x = gelu_fast(g.x) * u.x;
            o.y = gelu_fast(g.y) * u.y;
            o.z = gelu_fast(g.z) * u.z;
            o.w = gelu_fast(g.w) * u.w;
            sx4[c] = o;
        }
    } else {
        float inv1 = 0.0f;
        if (p.r && p.r_w) {
            float ss = 0.0f;
            for (int c = tid; c < n4; c += kGemvThreads) ss = sumsq4(ldf4(p.r + 4 * c), ss);
            inv1 = rms_inv(gemv_block_sum(ss, s_red), a.cols, p.eps);
        }
        float ss = 0.0f;
        const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int c = tid; c < n4; c += kGemvThreads) {
            const f32x4 o = pro_x1(p, ldf4(a.x + 4 * c), p.r ? ldf4(p.r + 4 * c) : zero,
                                   p.r && p.r_w ? ldf4(p.r_w + 4 * c) : zero, inv1);
            if (wr) *reinterpret_cast<f32x4*>(p.x_out + 4 * c) = o;
            sx4[c] = o;
            ss = sumsq4(o, ss);
        }
        if (p.w) {
            const float inv2 = rms_inv(gemv_block_sum(ss, s_red), a.cols, p.eps);
            for (int c = tid; c < n4; c += kGemvThreads)  // the elements this thread wrote
                sx4[c] = norm_w4(sx4[c], inv2, ldf4(p.w + 4 * c), p.uo);
        }
    }
    if (p.xb_out && blockIdx.x == 0)
        for (int c = tid; c < n4; c += kGemvThreads) *reinterpret_cast<f32x4*>(p.xb_out + 4 * c) = sx4[c];
    __syncthreads();
}

template <int QT, int RPW, int NB, int MODE, bool PRO = false>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(GemvArgs a) {
    constexpr int NM = MODE == GV_GEGLU ? 2 : 1;  // matrices per row (gate, up)
    constexpr int NACC = RPW * NB * NM;
    __shared__ float s_part[kGemvWaves][NACC];
    extern __shared__ float s_x[];  // PRO: the input vector, cols floats
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int G = a.cols / 8;
    // Row pointers of the block at row0. Rows past the end read the block's first row (in
    // range: row0 < total_rows) and are never written.
    auto rows_of = [&](int row0, const unsigned char* (&wrow)[RPW][NM], float* (&yrow)[RPW], int (&ystride)[RPW]) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const bool ok = row0 + r < a.total_rows;
            int R = ok ? row0 + r : row0;
            int s = 0;
            if (a.nseg > 1 && R >= a.seg[0].rows) {
                R -= a.seg[0].rows;
                s = 1;
                if (a.nseg > 2 && R >= a.seg[1].rows) {
                    R -= a.seg[1].rows;
                    s = 2;
                }
            }
            wrow[r][0] = a.seg[s].w + (int64_t)R * a.row_bytes;
            if constexpr (NM == 2) wrow[r][1] = a.w_up + (int64_t)R * a.row_bytes;
            yrow[r] = ok ? a.seg[s].y + R : nullptr;
            ystride[r] = a.seg[s].rows;
        }
    };
    // PRO: the first row block's first column group of weights (group tid, clamped into the
    // row) is loaded before the prologue, so its HBM latency overlaps the prologue's.
    WGroup<QT> wpre[RPW][NM];
    if constexpr (PRO) {
        const unsigned char* w0[RPW][NM];
        float* y0[RPW];
        int s0[RPW];
        rows_of(blockIdx.x * RPW, w0, y0, s0);
        const typename WGroup<QT>::Off o = WGroup<QT>::off((uint32_t)min(tid, G - 1));
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) wpre[r][m].load(w0[r][m], o);
        gemv_prologue(a, s_x, &s_part[0][0]);
    }

    // Row blocks: one per workgroup, except PRO kernels, whose grid is capped (the prologue
    // is paid once per workgroup) and which take every gridDim.x-th block.
    for (int row0 = blockIdx.x * RPW;;) {
    const bool first = PRO && row0 == (int)blockIdx.x * RPW;  // wpre holds its group tid
    const unsigned char* wrow[RPW][NM];
    float* yrow[RPW];
    int ystride[RPW];
    rows_of(row0, wrow, yrow, ystride);

    for (int b0 = 0; b0 < a.batch; b0 += NB) {
        float acc[RPW][NM][NB];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int b = 0; b < NB; ++b) acc[r][m][b] = 0.0f;

        // Q8_0 / dense: double-buffered, the next group's weights and x are in flight while
        // the current group is multiplied. Q4_0 (4.5 bytes per group and row) measured faster
        // single-buffered with more rows per workgroup (LM head 262144 x 2560: 141 against
        // 180 us; Q8_0: 187 against 209 us double- against single-buffered).
        if constexpr (QT != HIP_BRIDGE_Q4_0) {
        const float* xt[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
            xt[b] = PRO ? s_x : a.x + (int64_t)(b0 + b < a.batch ? b0 + b : a.batch - 1) * a.cols;
        WGroup<QT> cur[RPW][NM], nxt[RPW][NM];
        f32x4 cxa[NB], cxb[NB], nxa[NB], nxb[NB];
        auto fetch = [&](int g, WGroup<QT> (&w)[RPW][NM], f32x4 (&xa)[NB], f32x4 (&xb)[NB]) {
            const typename WGroup<QT>::Off o = WGroup<QT>::off((uint32_t)g);
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int m = 0; m < NM; ++m) w[r][m].load(wrow[r][m], o);
            int ca, cb;
            group_cols<QT>(g, ca, cb);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                xa[b] = ldf4(xt[b] + ca);
                xb[b] = ldf4(xt[b] + cb);
            }
        };
        int g = tid;
        if (g < G) {
            if (first) {  // weights prefetched before the prologue; x from LDS
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int m = 0; m < NM; ++m) cur[r][m] = wpre[r][m];
                int ca, cb;
                group_cols<QT>(g, ca, cb);
                cxa[0] = ldf4(s_x + ca);
                cxb[0] = ldf4(s_x + cb);
            } else {
                fetch(g, cur, cxa, cxb);
            }
        }
        for (; g < G; g += kGemvThreads) {
            const int gn = g + kGemvThreads;
            if (gn < G) fetch(gn, nxt, nxa, nxb);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const f32x4 xa = cxa[b], xb = cxb[b];
                const float sx = ((xa.x + xa.y) + (xa.z + xa.w)) + ((xb.x + xb.y) + (xb.z + xb.w));
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int m = 0; m < NM; ++m) acc[r][m][b] += cur[r][m].dot(xa, xb, sx);
            }
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int m = 0; m < NM; ++m) cur[r][m] = nxt[r][m];
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                cxa[b] = nxa[b];
                cxb[b] = nxb[b];
            }
        }

        } else {
        for (int g = tid; g < G; g += kGemvThreads) {
            WGroup<QT> wg[RPW][NM];
            if (first && g == tid) {  // the group prefetched before the prologue
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int m = 0; m < NM; ++m) wg[r][m] = wpre[r][m];
            } else {
                const typename WGroup<QT>::Off o = WGroup<QT>::off((uint32_t)g);
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int m = 0; m < NM; ++m) wg[r][m].load(wrow[r][m], o);
            }
            int ca, cb;
            group_cols<QT>(g, ca, cb);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int bt = b0 + b < a.batch ? b0 + b : a.batch - 1;
                const float* xr = PRO ? s_x : a.x + (int64_t)bt * a.cols;
                const f32x4 xa = ldf4(xr + ca), xb = ldf4(xr + cb);
                const float sx = ((xa.x + xa.y) + (xa.z + xa.w)) + ((xb.x + xb.y) + (xb.z + xb.w));
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int m = 0; m < NM; ++m) acc[r][m][b] += wg[r][m].dot(xa, xb, sx);
            }
        }
        }

        // wave sums, then the 4 wave partials in order through LDS
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const float v = group_sum<kWave>(acc[r][m][b]);
                    if (lane == 0) s_part[wave][(r * NM + m) * NB + b] = v;
                }
        __syncthreads();
        if (tid < RPW * NB) {
            const int r = tid / NB, b = tid % NB;
            float tot[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const int i = (r * NM + m) * NB + b;
                tot[m] = (s_part[0][i] + s_part[1][i]) + (s_part[2][i] + s_part[3][i]);
            }
            float* yr = nullptr;
            int ys = 0;
#pragma unroll
            for (int rr = 0; rr < RPW; ++rr)
                if (rr == r) {  // select without indexing the register arrays at run time
                    yr = yrow[rr];
                    ys = ystride[rr];
                }
            if (yr && b0 + b < a.batch) {
                float out = tot[0];
                if constexpr (MODE == GV_GEGLU) out = gelu_fast(tot[0]) * tot[1];
                yr[(int64_t)(b0 + b) * ys] = out;
            }
        }
        __syncthreads();  // s_part is rewritten by the next token tile
    }
    if constexpr (!PRO) break;
    row0 += gridDim.x * RPW;
    if (row0 >= a.total_rows) break;
    }
}

// Batch-1 products, wave-owned rows: each wave of the workgroup owns RW consecutive rows and
// walks all G column groups of them with its 64 lanes (lane l takes groups l, l + 64, ...),
// so a row's work is balanced over the lanes for any G that is a multiple of 64 (the
// workgroup-wide split above leaves waves idle when G is not a multiple of 256: 2560 columns
// are 320 groups), the row sums reduce within the wave (no LDS, no barrier), and the next
// group's weights and x are loaded while the current group is multiplied.
template <int QT, int RW, int MODE>
__global__ __launch_bounds__(kGemvThreads) __attribute__((amdgpu_waves_per_eu(QT == HIP_BRIDGE_Q4_0 && MODE == GV_PLAIN ? 8 : 1))) void k_gemv_w(GemvArgs a) {
    constexpr int NM = MODE == GV_GEGLU ? 2 : 1;
    const int lane = threadIdx.x & 63;
    // The wave index is uniform across the wave: read from the first lane, it makes the row
    // pointers scalar (each load is a scalar base plus the lane's 32-bit offset).
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * kGemvWaves + wv) * RW;
    const int G = a.cols / 8;
    if (G <= 0) return;  // the whole grid
    // Waves past the last row take part in staging x (below) and then leave.
    const bool live = row0 < a.total_rows;
    const unsigned char* wrow[RW][NM];
    float* yrow[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const bool ok = row0 + r < a.total_rows;
        int R = ok ? row0 + r : row0;
        int sg = 0;
        if (a.nseg > 1 && R >= a.seg[0].rows) {
            R -= a.seg[0].rows;
            sg = 1;
            if (a.nseg > 2 && R >= a.seg[1].rows) {
                R -= a.seg[1].rows;
                sg = 2;
            }
        }
        wrow[r][0] = a.seg[sg].w + (int64_t)R * a.row_bytes;
        if constexpr (NM == 2) wrow[r][1] = a.w_up + (int64_t)R * a.row_bytes;
        yrow[r] = ok ? a.seg[sg].y + R : nullptr;
    }
    float acc[RW][NM];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[r][m] = 0.0f;
    // Step k takes group lane + 64k. The step count is the same for every lane, so all
    // branches below are uniform: a lane past the last group loads the last group again
    // (in bounds) and drops its products. (A load under a per-lane branch would make the
    // compiler wait for it where the branch ends, i.e. before the step that needs it.)
    const int n = (G + kWave - 1) / kWave;
    // x is staged once per workgroup in LDS and read there at each step (it is not held in
    // registers across a step, which keeps the kernel's VGPRs at 8 waves per SIMD for Q4_0;
    // the cols * 4 bytes of LDS per 4-wave workgroup allow 8 waves per SIMD up to 5120
    // columns of the CU's 160 KB, 4 up to 10240).
    extern __shared__ __attribute__((aligned(16))) float s_xw[];
    auto fetch = [&](int k, WGroup<QT> (&w)[RW][NM]) {
        const int g = min(lane + kWave * k, G - 1);
        const typename WGroup<QT>::Off o = WGroup<QT>::off((uint32_t)g);
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) w[r][m].load(wrow[r][m], o);
    };
    auto fold = [&](const WGroup<QT> (&w)[RW][NM], int k, bool last) {
        int ca, cb;
        group_cols<QT>(min(lane + kWave * k, G - 1), ca, cb);
        const f32x4 xa = *reinterpret_cast<const f32x4*>(s_xw + ca);
        const f32x4 xb = *reinterpret_cast<const f32x4*>(s_xw + cb);
        const float sx = ((xa.x + xa.y) + (xa.z + xa.w)) + ((xb.x + xb.y) + (xb.z + xb.w));
        const bool ok = !last || lane + kWave * k < G;
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const float d = w[r][m].dot(xa, xb, sx);
                if (last) acc[r][m] = ok ? acc[r][m] + d : acc[r][m];
                else acc[r][m] += d;
            }
    };
    // Two register sets in turn (no copy of the prefetched set per step). The scheduling
    // barriers keep each step's loads ahead of the previous step's arithmetic: otherwise
    // the scheduler hoists that arithmetic, and with it the wait for its operands, above
    // the new loads, and every step waits a full memory round trip.
    WGroup<QT> wa[RW][NM], wb[RW][NM];
    if (live) fetch(0, wa);  // the first weights are in flight while x is staged
    for (int i = threadIdx.x; i < a.cols / 4; i += kGemvThreads)
        *reinterpret_cast<f32x4*>(s_xw + 4 * i) = ldf4(a.x + 4 * i);
    __syncthreads();
    if (!live) return;
    for (int k = 0;; k += 2) {
        if (k + 1 >= n) {
            fold(wa, k, true);
            break;
        }
        fetch(k + 1, wb);
        __builtin_amdgcn_sched_barrier(0);
        fold(wa, k, false);
        if (k + 2 >= n) {
            fold(wb, k + 1, true);
            break;
        }
        fetch(k + 2, wa);
        __builtin_amdgcn_sched_barrier(0);
        fold(wb, k + 1, false);
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        float t[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) t[m] = group_sum<kWave>(acc[r][m]);
        if (lane == 0 && yrow[r]) {
            float out = t[0];
            if constexpr (MODE == GV_GEGLU) out = gelu_fast(t[0]) * t[1];
            *yrow[r] = out;
        }
    }
}

// Batch-1 Q4_0 / Q8_0 products, one 32-column block per lane and step: the loops above issue
// two or three loads per 8-column group (the 16-bit scale and 4 or 8 quant bytes, every other
// one 2-byte aligned), and at decode sizes that instruction stream, not HBM, sets the rate
// (measured with the arithmetic removed: Q4_0 262144 x 2560 in 97 us against 82 us with every
// quant load 4-byte aligned). Here a lane takes the whole block with dword-aligned loads
// (BlkWin: 20 bytes for Q4_0, 36 for Q8_0) and picks the scale and the quant bytes out of the
// window with byte permutes (Q8_0 262144 x 2560: 164 -> 128 us).
//
// Layout: LPR lanes per row (8, 16, 32 or 64) and 64 / LPR row sets of RW rows per wave; lane i
// of a set takes blocks i, i + LPR, ... (bpl <= kQ4bMaxB of them) of each of its rows, every
// weight load of the wave issued before any arithmetic (one memory round trip per wave).
// x is staged once per workgroup in LDS, 36 floats per 32-column block: the block's 32 values
// and, at slot 32, their sum (the padding keeps the 16 lanes of a set, which read consecutive
// blocks, on distinct banks); each lane reads its blocks' x there once and applies them to
// all its rows. The sum is formed at staging, once per workgroup and block, not by each lane
// for each of its blocks (31 additions per block, a quarter of a plain product's VALU work).
// Row sums: LPR-lane butterfly.
constexpr int kQ4bMaxB = 6;
constexpr int kQ4bXStride = 36;
constexpr int kQ4bMaxCols = 12288;    // x staged through registers: 12 float4 per thread at 256
constexpr int kQ4bProMaxCols = 4096;  // PRO operands: 4 float4 each per thread at 256
#ifndef ZL_GEMV_Q4B_PRO_WAVES
#define ZL_GEMV_Q4B_PRO_WAVES 4
#endif
#ifndef ZL_GEMV_Q4B
#define ZL_GEMV_Q4B 1
#endif
#ifndef ZL_GEMV_Q4B_WAVES
#define ZL_GEMV_Q4B_WAVES 1024
#endif
// GeGLU pairs over two row sets (k_gemv_q4b SPL); 0 keeps both rows of a pair in every lane
// (tuning builds).
#ifndef ZL_Q4B_GEGLU_SPLIT
#define ZL_Q4B_GEGLU_SPLIT 1
#endif
#ifndef ZL_GEMV_Q4B_NW
#define ZL_GEMV_Q4B_NW 4
#endif
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef uint32_t u32_a4 __attribute__((aligned(4)));

// The dword-aligned window holding block b of a Q4_0 (18-byte) or Q8_0 (34-byte) row: it
// starts at BB*b rounded down to 4 bytes, so the scale sits at window byte 0 (even b) or 2
// (odd b) and the quants follow it; an even block count per row keeps both ends of every
// window inside the row. Quant dword i is the window's bytes 2 + 4i .. 5 + 4i (even) or
// 4 + 4i .. 7 + 4i (odd), one v_perm_b32 of two window dwords either way.
template <int QT>
struct BlkWin;
template <>
struct BlkWin<HIP_BRIDGE_Q4_0> {
    static constexpr uint32_t BB = 18;
    u32x4 a;     // window bytes 0..15
    uint32_t e;  // window bytes 16..19
    __device__ __forceinline__ void load(const unsigned char* p) {
        a = *reinterpret_cast<const u32x4_a4*>(p);
        e = *reinterpret_cast<const u32_a4*>(p + 16);
    }
    // d * (sum_j u_j x_j - 8 * sum x) over the block (math.zig:304-305): u_j the stored nibble,
    // low nibbles columns 0..15, high nibbles 16..31; xl / xh: the block's x, columns 0..15
    // and 16..31; sx their sum.
    __device__ __forceinline__ float dot(bool odd, const f32x4 (&xl)[4], const f32x4 (&xh)[4], float sx) const {
        const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
        const uint32_t q[4] = {__builtin_amdgcn_perm(a.y, a.x, sel), __builtin_amdgcn_perm(a.z, a.y, sel),
                               __builtin_amdgcn_perm(a.w, a.z, sel), __builtin_amdgcn_perm(e, a.w, sel)};
        const uint32_t d16 = __builtin_amdgcn_perm(0u, a.x, odd ? 0x0c0c0302u : 0x0c0c0100u);
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = mask_bytes(q[i], 0x0f0f0f0fu);       // columns 4i .. 4i+3
            const uint32_t hi = mask_bytes(q[i] >> 4, 0x0f0f0f0fu);  // columns 16+4i .. 16+4i+3
            t = i == 0 ? (float)(lo & 0xff) * xl[0].x : fmaf((float)(lo & 0xff), xl[i].x, t);
            t = fmaf((float)((lo >> 8) & 0xff), xl[i].y, t);
            t = fmaf((float)((lo >> 16) & 0xff), xl[i].z, t);
            t = fmaf((float)(lo >> 24), xl[i].w, t);
            t = fmaf((float)(hi & 0xff), xh[i].x, t);
            t = fmaf((float)((hi >> 8) & 0xff), xh[i].y, t);
            t = fmaf((float)((hi >> 16) & 0xff), xh[i].z, t);
            t = fmaf((float)(hi >> 24), xh[i].w, t);
        }
        return h2f(d16) * fmaf(-8.0f, sx, t);
    }
};
template <>
struct BlkWin<HIP_BRIDGE_Q8_0> {
    static constexpr uint32_t BB = 34;
    u32x4 a, b;  // window bytes 0..31
    uint32_t e;  // window bytes 32..35
    __device__ __forceinline__ void load(const unsigned char* p) {
        a = *reinterpret_cast<const u32x4_a4*>(p);
        b = *reinterpret_cast<const u32x4_a4*>(p + 16);
        e = *reinterpret_cast<const u32_a4*>(p + 32);
    }
    // d * (sum_j u_j x_j - 128 * sum x): the int8 quants read as u = q ^ 0x80 (columns 4i ..
    // 4i+3 in quant dword i), as the group kernels do.
    __device__ __forceinline__ float dot(bool odd, const f32x4 (&xl)[4], const f32x4 (&xh)[4], float sx) const {
        const uint32_t sel = odd ? 0x07060504u : 0x05040302u;
        const uint32_t D[9] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, e};
        const uint32_t d16 = __builtin_amdgcn_perm(0u, a.x, odd ? 0x0c0c0302u : 0x0c0c0100u);
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t u = __builtin_amdgcn_perm(D[i + 1], D[i], sel) ^ 0x80808080u;
            const f32x4 xv = i < 4 ? xl[i] : xh[i - 4];
            t = i == 0 ? (float)(u & 0xff) * xv.x : fmaf((float)(u & 0xff), xv.x, t);
            t = fmaf((float)((u >> 8) & 0xff), xv.y, t);
            t = fmaf((float)((u >> 16) & 0xff), xv.z, t);
            t = fmaf((float)(u >> 24), xv.w, t);
        }
        return h2f(d16) * fmaf(-128.0f, sx, t);
    }
};

// PRO prologue of the block kernel, in two phases around the weight loads: q4b_pro_load
// issues the operand loads (x, r, r's weights, the norm weights: K float4 each per thread,
// range-checked), q4b_pro_finish forms the input vector in registers with the arithmetic of
// gemv_prologue (workgroup 0 writes x1 and the input when asked).
template <int K, int T>
__device__ __forceinline__ void q4b_pro_load(const GemvArgs& a, f32x4 (&xv)[K], f32x4 (&rv)[K], f32x4 (&rwv)[K],
                                             f32x4 (&wv)[K]) {
    const GemvPro& p = a.pro;
    const uint32_t nb = (uint32_t)a.cols * 4u;
    const auto rs_x = buf_rsrc(a.x, nb);
    const auto rs_r = buf_rsrc(p.r, p.r ? nb : 0u);
    const auto rs_rw = buf_rsrc(p.r_w, p.mode == GP_NORM && p.r && p.r_w ? nb : 0u);
    const auto rs_w = buf_rsrc(p.w, p.mode == GP_NORM && p.w ? nb : 0u);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const uint32_t o = (uint32_t)(threadIdx.x + k * T) * 16u;
        xv[k] = bldf4(rs_x, o);
        rv[k] = bldf4(rs_r, o);
        rwv[k] = bldf4(rs_rw, o);
        wv[k] = bldf4(rs_w, o);
    }
}
// Sum over a workgroup of T threads (wave sums, then the wave values in wave order); s_red
// holds T / 64 floats.
template <int T>
__device__ __forceinline__ float q4b_block_sum(float v, float* s_red) {
    v = group_sum<kWave>(v);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = s_red[0];
#pragma unroll
    for (int w = 1; w < T / kWave; ++w) t += s_red[w];
    __syncthreads();  // s_red is reused by the next reduction
    return t;
}
template <int K, int T>
__device__ __forceinline__ void q4b_pro_finish(const GemvArgs& a, f32x4 (&xv)[K], const f32x4 (&rv)[K],
                                               const f32x4 (&rwv)[K], const f32x4 (&wv)[K], float* s_red) {
    const GemvPro& p = a.pro;
    const int n4 = a.cols / 4;
    const int tid = threadIdx.x;
    if (p.mode == GP_GEGLU) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            xv[k].x = gelu_fast(xv[k].x) * rv[k].x;
            xv[k].y = gelu_fast(xv[k].y) * rv[k].y;
            xv[k].z = gelu_fast(xv[k].z) * rv[k].z;
            xv[k].w = gelu_fast(xv[k].w) * rv[k].w;
        }
    } else {
        const bool wr = p.x_out && blockIdx.x == 0;
        float inv1 = 0.0f;
        if (p.r && p.r_w) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k)
                if (tid + k * T < n4) ss = sumsq4(rv[k], ss);
            inv1 = rms_inv(q4b_block_sum<T>(ss, s_red), a.cols, p.eps);
        }
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int c = tid + k * T;
            if (c < n4) {
                xv[k] = pro_x1(p, xv[k], rv[k], rwv[k], inv1);
                if (wr) *reinterpret_cast<f32x4*>(p.x_out + 4 * c) = xv[k];
                ss = sumsq4(xv[k], ss);
            }
        }
        if (p.w) {
            const float inv2 = rms_inv(q4b_block_sum<T>(ss, s_red), a.cols, p.eps);
#pragma unroll
            for (int k = 0; k < K; ++k) xv[k] = norm_w4(xv[k], inv2, wv[k], p.uo);
        }
    }
    if (p.xb_out && blockIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int c = tid + k * T;
            if (c < n4) *reinterpret_cast<f32x4*>(p.xb_out + 4 * c) = xv[k];
        }
    }
}

template <int QT, int MODE, int LPR, int RW, int BPL, bool PRO, int NW, bool SPLIT = false>
__global__ __launch_bounds__(NW * kWave) void k_gemv_q4b(GemvArgs a) {
    constexpr int T = NW * kWave;
    constexpr int SETS = kWave / LPR;
    // SPL (GeGLU): the gate and up rows of a pair in two neighbouring sets, combined across
    // the wave at the end, instead of both in every lane (twice the waves, half the blocks each)
    constexpr bool SPL = SPLIT && MODE == GV_GEGLU && SETS >= 2;
    constexpr int NM = MODE == GV_GEGLU && !SPL ? 2 : 1;
    constexpr int XK = (PRO ? kQ4bProMaxCols : kQ4bMaxCols) / 4 / T;  // x float4 per thread
    extern __shared__ __attribute__((aligned(16))) float s_xq[];
    __shared__ float s_red[NW];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int li = lane % LPR, set = lane / LPR;
    const int gset = (blockIdx.x * NW + wv) * SETS + set;
    const int mat = SPL ? (gset & 1) : 0;  // SPL: 0 gate, 1 up
    const int row0 = (SPL ? gset >> 1 : gset) * RW;
    // x (PRO: the prologue's operands) first: its loads complete before the weights' do, so
    // staging it waits on it alone
    const int n4 = a.cols / 4;
    f32x4 xv[XK], rv[PRO ? XK : 1], rwv[PRO ? XK : 1], wnv[PRO ? XK : 1];
    if constexpr (PRO) {
        q4b_pro_load<XK, T>(a, xv, rv, rwv, wnv);
    } else {
#pragma unroll
        for (int k = 0; k < XK; ++k) {
            const int i = (int)threadIdx.x + k * T;
            if (i < n4) xv[k] = ldf4(a.x + 4 * i);
        }
    }
    // Row pointers: the segment of each row by selects over the (uniform) segment fields, so
    // no per-lane indexed read of the arguments.
    const unsigned char* wrow[RW][NM];
    float* yrow[RW];
    const int r0 = a.seg[0].rows, r1 = a.nseg > 1 ? a.seg[1].rows : 0;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const bool ok = row0 + r < a.total_rows;
        const int R = ok ? row0 + r : a.total_rows - 1;  // past the end: the last row, not written
        const bool s0 = R < r0, s1 = !s0 && R - r0 < r1;
        const int Rs = s0 ? R : s1 ? R - r0 : R - r0 - r1;
        const unsigned char* wb = s0 ? a.seg[0].w : s1 ? a.seg[1].w : a.seg[2].w;
        float* yb = s0 ? a.seg[0].y : s1 ? a.seg[1].y : a.seg[2].y;
        wrow[r][0] = (SPL && mat ? a.w_up : wb) + (int64_t)Rs * a.row_bytes;
        if constexpr (NM == 2) wrow[r][1] = a.w_up + (int64_t)Rs * a.row_bytes;
        yrow[r] = ok ? yb + Rs : nullptr;
    }
    BlkWin<QT> w[BPL][RW][NM];
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const uint32_t off = ((uint32_t)(li + LPR * j) * BlkWin<QT>::BB) & ~3u;
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) w[j][r][m].load(wrow[r][m] + off);
    }
    // the input into LDS: float4 i of block i / 8 at slot offset 4 * (i % 8), the block's sum
    // at slot 32. Lanes 8j .. 8j+7 hold one block's float4s (T and 8 divide k * T), all in
    // range or all out (n4 is a multiple of 64). The sum is ((v0 + v1) + v2) + v3, v_i the sum
    // of float4s i and i + 4 (columns 4i.. and 16+4i..), each ((x + y) + (z + w)): DPP row
    // shifts within the 8 lanes (v_i lands in lane 4 + i, the running sum moves up one lane a
    // step and ends in lane 7; every lane read lies in the same 8-lane group).
    if constexpr (PRO) q4b_pro_finish<XK, T>(a, xv, rv, rwv, wnv, s_red);
    // Staged block sums where a lane has few blocks of x to stage: at 64 lanes per row (more
    // than 6144 columns) each thread stages 6+ float4s and the staging, which every wave waits
    // for at the barrier, outlasts the additions it saves (2560 x 10240: 7.25 -> 7.55 us).
    constexpr bool ssum = LPR < 64;
#pragma unroll
    for (int k = 0; k < XK; ++k) {
        const int i = (int)threadIdx.x + k * T;
        if (k * T >= n4) break;  // uniform
        float bs = 0.0f;
        if constexpr (ssum) {
            const float s4 = i < n4 ? (xv[k].x + xv[k].y) + (xv[k].z + xv[k].w) : 0.0f;
            const float v = s4 + dpp<0x114>(s4);  // row_shr:4
            bs = v + dpp<0x111>(v);               // row_shr:1
            bs = v + dpp<0x111>(bs);
            bs = v + dpp<0x111>(bs);
        }
        if (i < n4) {
            float* xs = s_xq + (i >> 3) * kQ4bXStride;
            *reinterpret_cast<f32x4*>(xs + 4 * (i & 7)) = xv[k];
            if (ssum && (i & 7) == 7) xs[32] = bs;
        }
    }
    __syncthreads();
    // nothing below moves above the barrier: the scheduler would otherwise start the first
    // block's byte permutes there, and each wave would wait for its first weights before it
    // arrives (and reads x) instead of after
    __builtin_amdgcn_sched_barrier(0);
    float acc[RW][NM];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const int b = li + LPR * j;
        const float* xs = s_xq + b * kQ4bXStride;
        f32x4 xl[4], xh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xl[i] = *reinterpret_cast<const f32x4*>(xs + 4 * i);
            xh[i] = *reinterpret_cast<const f32x4*>(xs + 16 + 4 * i);
        }
        float sx = 0.0f;
        if constexpr (ssum) {
            sx = xs[32];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                sx += ((xl[i].x + xl[i].y) + (xl[i].z + xl[i].w)) + ((xh[i].x + xh[i].y) + (xh[i].z + xh[i].w));
        }
        const bool odd = b & 1;
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) acc[r][m] += w[j][r][m].dot(odd, xl, xh, sx);
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[r][m] = group_sum<LPR>(acc[r][m]);
    if constexpr (SPL) {
        // the up set's sums to the gate set's lanes (LPR lanes further)
        float up[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) up[r] = __shfl_down(acc[r][0], LPR);
        if (li == 0 && mat == 0) {
#pragma unroll
            for (int r = 0; r < RW; ++r)
                if (yrow[r]) *yrow[r] = gelu_fast(acc[r][0]) * up[r];
        }
    } else if (li == 0) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            if (!yrow[r]) continue;
            float out = acc[r][0];
            if constexpr (MODE == GV_GEGLU) out = gelu_fast(acc[r][0]) * acc[r][1];
            *yrow[r] = out;
        }
    }
}

// Launches k_gemv_q4b when the product suits it (batch 1, Q4_0, blocks per row a multiple of
// 8 with at most kQ4bMaxB per lane at 8 to 64 lanes per row, x within 64 KB of LDS); returns
// false otherwise. LPR: the fewest lanes per row that take every block in kQ4bMaxB steps,
// more while the grid has fewer than ZL_GEMV_Q4B_WAVES waves; RW = 2 rows per set from
// 4 * ZL_GEMV_Q4B_WAVES waves.
template <int QT, int MODE, bool PRO>
static bool launch_q4b(const GemvArgs& a, hipStream_t s) {
    if constexpr (QT != HIP_BRIDGE_Q4_0 && QT != HIP_BRIDGE_Q8_0) {
        return false;
    } else {
    if (!ZL_GEMV_Q4B || a.batch != 1) return false;
    // the windows are dword loads from the row base: every matrix 4-byte aligned (rows are a
    // whole number of block pairs, 36 / 68 bytes, so each row is too)
    auto a4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; };
    for (int i = 0; i < a.nseg; ++i)
        if (a.seg[i].rows > 0 && !a4(a.seg[i].w)) return false;
    if (MODE == GV_GEGLU && !a4(a.w_up)) return false;
    const int nblk = a.cols / 32;
    if (a.cols % 256 != 0) return false;
    const size_t lds = (size_t)nblk * kQ4bXStride * sizeof(float);
    if (a.cols > (PRO ? kQ4bProMaxCols : kQ4bMaxCols) || lds > 65536) return false;
    // waves per workgroup: a prologue is paid once per workgroup, so its kernels take more
    constexpr int NW = PRO ? ZL_GEMV_Q4B_PRO_WAVES : ZL_GEMV_Q4B_NW;
    // 8 lanes per row only for block counts that 16 does not divide (8, 24, 40: e.g. the
    // per-layer-embedding projection's 256 columns)
    int lpr = nblk % 16 != 0 && nblk / 8 <= kQ4bMaxB ? 8 : 0;
    for (int l : {16, 32, 64})
        if (!lpr && nblk % l == 0 && nblk / l <= kQ4bMaxB) {
            lpr = l;
            break;
        }
    if (!lpr) return false;
    // GeGLU pairs split over two sets (SPL in the kernel) where lanes per row leave at least
    // two sets per wave: the row space counts each pair twice
    const bool spl = ZL_Q4B_GEGLU_SPLIT && MODE == GV_GEGLU && !PRO;
    int64_t vrows = spl ? 2 * (int64_t)a.total_rows : a.total_rows;
    auto waves = [&](int l, int rw) { return cdiv(vrows, (int64_t)(kWave / l) * rw); };
    while (lpr < 64 && waves(lpr, 1) < ZL_GEMV_Q4B_WAVES && nblk % (2 * lpr) == 0) lpr *= 2;
    if (spl && lpr == 64) vrows = a.total_rows;  // one set per wave: the pairs stay whole
    const int rw = waves(lpr, 2) >= 4 * ZL_GEMV_Q4B_WAVES ? 2 : 1;
    const int bpl = nblk / lpr;
    const unsigned grid = (unsigned)cdiv(waves(lpr, rw), (int64_t)NW);
    auto go = [&](auto lpr_c, auto rw_c) {
        constexpr int L = decltype(lpr_c)::value, RW = decltype(rw_c)::value;
        constexpr bool SP = ZL_Q4B_GEGLU_SPLIT && MODE == GV_GEGLU && !PRO && L < 64;
        switch (bpl) {
            case 1: k_gemv_q4b<QT, MODE, L, RW, 1, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a); break;
            case 2: k_gemv_q4b<QT, MODE, L, RW, 2, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a); break;
            case 3: k_gemv_q4b<QT, MODE, L, RW, 3, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a); break;
            case 4: k_gemv_q4b<QT, MODE, L, RW, 4, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a); break;
            case 5: k_gemv_q4b<QT, MODE, L, RW, 5, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a); break;
            default: k_gemv_q4b<QT, MODE, L, RW, 6, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a); break;
        }
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    if (lpr == 8) {  // odd block counts per lane only
        auto go8 = [&](auto rw_c) {
            constexpr int RW = decltype(rw_c)::value;
            constexpr bool SP = ZL_Q4B_GEGLU_SPLIT && MODE == GV_GEGLU && !PRO;
            if (bpl == 1) k_gemv_q4b<QT, MODE, 8, RW, 1, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a);
            else if (bpl == 3) k_gemv_q4b<QT, MODE, 8, RW, 3, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a);
            else k_gemv_q4b<QT, MODE, 8, RW, 5, PRO, NW, SP><<<grid, NW * kWave, lds, s>>>(a);
        };
        rw == 2 ? go8(I2{}) : go8(I1{});
    } else if (lpr == 16) rw == 2 ? go(std::integral_constant<int, 16>{}, I2{}) : go(std::integral_constant<int, 16>{}, I1{});
    else if (lpr == 32) rw == 2 ? go(std::integral_constant<int, 32>{}, I2{}) : go(std::integral_constant<int, 32>{}, I1{});
    else rw == 2 ? go(std::integral_constant<int, 64>{}, I2{}) : go(std::integral_constant<int, 64>{}, I1{});
    return true;
    }
}

// Batch-1 Q4_K products, the block kernel's scheme over 64-column chunks. A Q4_K super-block
// (144 bytes, 256 columns: f16 d, f16 dmin, 12 bytes of packed 6-bit scales and mins, 128 quant
// bytes; types.zig:170-175) holds four chunks; chunk jj is sub-blocks 2jj (the low nibbles of
// quant bytes 32jj .. 32jj+31, columns 64jj ..) and 2jj+1 (their high nibbles, columns
// 64jj+32 ..). A lane takes whole chunks with three 16-byte loads (the super-block's 16-byte
// header and the chunk's 32 quant bytes; rows are 144n bytes, so 16-byte aligned with the
// matrix): the group-wise loops issue five 32-bit loads per 8 columns. x is staged per
// workgroup at 72 floats per chunk, its two sub-block sums at slots 64 and 65 (the padding puts
// the 8 lanes of a set, which read consecutive chunks, on distinct banks). Arithmetic as the
// group kernels: (d sc_j) sum(q x) - (dmin m_j) sum(x) per sub-block (math.zig:440-496).
constexpr int kQ4kbXStride = 72;
struct KChunk {
    u32x4 h;       // d | dmin << 16, scale bytes 0..3, 4..7, 8..11
    u32x4 q0, q1;  // the chunk's quant bytes 0..15, 16..31
    __device__ __forceinline__ void load(const unsigned char* sb, uint32_t jj) {
        h = *reinterpret_cast<const u32x4*>(sb);
        q0 = *reinterpret_cast<const u32x4*>(sb + 16u + 32u * jj);
        q1 = *reinterpret_cast<const u32x4*>(sb + 32u + 32u * jj);
    }
    // xs: the chunk's x in LDS (columns 0..31 / 32..63, sub-blocks 2jj / 2jj+1, at slots 0 / 32,
    // their sums at 64 / 65), read one sub-block at a time.
    __device__ __forceinline__ float dot(uint32_t jj, const float* xs) const {
        // 6-bit scale / min of sub-blocks 2jj and 2jj+1 (quant.zig:285-290): bytes t, t+1
        // (t = 2 (jj & 1)) of the three scale words
        // (selects rather than a branch: jj differs between lanes)
        const uint32_t sft = (jj & 1u) * 16u;
        const uint32_t A = h.y >> sft, Bw = h.z >> sft, C = h.w >> sft;
        const bool lo = jj < 2;
        const uint32_t sc0 = lo ? A & 63u : (C & 15u) | (((A >> 6) & 3u) << 4);
        const uint32_t sc1 = lo ? (A >> 8) & 63u : ((C >> 8) & 15u) | (((A >> 14) & 3u) << 4);
        const uint32_t m0 = lo ? Bw & 63u : ((C >> 4) & 15u) | (((Bw >> 6) & 3u) << 4);
        const uint32_t m1 = lo ? (Bw >> 8) & 63u : ((C >> 12) & 15u) | (((Bw >> 14) & 3u) << 4);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        float t[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {  // low nibbles: columns 4i.., high: 32+4i..
            f32x4 xv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = *reinterpret_cast<const f32x4*>(xs + 32 * hf + 4 * i);
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t u = mask_bytes(hf ? q[i] >> 4 : q[i], 0x0f0f0f0fu);
                acc = i == 0 ? (float)(u & 0xff) * xv[0].x : fmaf((float)(u & 0xff), xv[i].x, acc);
                acc = fmaf((float)((u >> 8) & 0xff), xv[i].y, acc);
                acc = fmaf((float)((u >> 16) & 0xff), xv[i].z, acc);
                acc = fmaf((float)(u >> 24), xv[i].w, acc);
            }
            t[hf] = acc;
        }
        const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
        const float d0 = d * (float)sc0, d1 = d * (float)sc1;
        const float n0 = dmin * (float)m0, n1 = dmin * (float)m1;
        return fmaf(d0, t[0], -(n0 * xs[64])) + fmaf(d1, t[1], -(n1 * xs[65]));
    }
};

// (3 waves per SIMD: up to 168 registers, which five chunks of weights, a chunk of x and the
// prologue's operands take without spilling)
template <int MODE, int LPR, int RW, int BPL, bool PRO, int NW>
__global__ __launch_bounds__(NW * kWave, 12 / NW) void k_gemv_q4kb(GemvArgs a) {
    constexpr int T = NW * kWave;
    constexpr int NM = MODE == GV_GEGLU ? 2 : 1;
    constexpr int SETS = kWave / LPR;
    constexpr int XK = (PRO ? kQ4bProMaxCols : kQ4bMaxCols) / 4 / T;  // x float4 per thread
    extern __shared__ __attribute__((aligned(16))) float s_xq[];
    __shared__ float s_red[NW];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int li = lane % LPR, set = lane / LPR;
    const int row0 = ((blockIdx.x * NW + wv) * SETS + set) * RW;
    const int n4 = a.cols / 4;
    f32x4 xv[XK], rv[PRO ? XK : 1], rwv[PRO ? XK : 1], wnv[PRO ? XK : 1];
    if constexpr (PRO) {
        q4b_pro_load<XK, T>(a, xv, rv, rwv, wnv);
    } else {
#pragma unroll
        for (int k = 0; k < XK; ++k) {
            const int i = (int)threadIdx.x + k * T;
            if (i < n4) xv[k] = ldf4(a.x + 4 * i);
        }
    }
    const unsigned char* wrow[RW][NM];
    float* yrow[RW];
    const int r0 = a.seg[0].rows, r1 = a.nseg > 1 ? a.seg[1].rows : 0;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const bool ok = row0 + r < a.total_rows;
        const int R = ok ? row0 + r : a.total_rows - 1;  // past the end: the last row, not written
        const bool s0 = R < r0, s1 = !s0 && R - r0 < r1;
        const int Rs = s0 ? R : s1 ? R - r0 : R - r0 - r1;
        const unsigned char* wb = s0 ? a.seg[0].w : s1 ? a.seg[1].w : a.seg[2].w;
        float* yb = s0 ? a.seg[0].y : s1 ? a.seg[1].y : a.seg[2].y;
        wrow[r][0] = wb + (int64_t)Rs * a.row_bytes;
        if constexpr (NM == 2) wrow[r][1] = a.w_up + (int64_t)Rs * a.row_bytes;
        yrow[r] = ok ? yb + Rs : nullptr;
    }
    KChunk w[BPL][RW][NM];
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const uint32_t c = (uint32_t)(li + LPR * j);
        const uint32_t off = (c >> 2) * 144u;
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) w[j][r][m].load(wrow[r][m] + off, c & 3u);
    }
    if constexpr (PRO) q4b_pro_finish<XK, T>(a, xv, rv, rwv, wnv, s_red);
    // x into LDS: float4 i at chunk i / 16, slot 4 (i % 16); the sum of each sub-block's 8
    // float4s (lanes 8j .. 8j+7) at slot 64 + (i / 8) % 2, formed by DPP row shifts as in the
    // Q4_0 kernel: ((v0 + v1) + v2) + v3, v_i the sum of float4s i and i + 4 of the sub-block.
#pragma unroll
    for (int k = 0; k < XK; ++k) {
        const int i = (int)threadIdx.x + k * T;
        if (k * T >= n4) break;  // uniform
        const float s4 = i < n4 ? (xv[k].x + xv[k].y) + (xv[k].z + xv[k].w) : 0.0f;
        const float v = s4 + dpp<0x114>(s4);  // row_shr:4
        float bs = v + dpp<0x111>(v);         // row_shr:1
        bs = v + dpp<0x111>(bs);
        bs = v + dpp<0x111>(bs);
        if (i < n4) {
            float* xs = s_xq + (i >> 4) * kQ4kbXStride;
            *reinterpret_cast<f32x4*>(xs + 4 * (i & 15)) = xv[k];
            if ((i & 7) == 7) xs[64 + ((i >> 3) & 1)] = bs;
        }
    }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    float acc[RW][NM];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const uint32_t c = (uint32_t)(li + LPR * j);
        const float* xs = s_xq + c * kQ4kbXStride;
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int m = 0; m < NM; ++m) acc[r][m] += w[j][r][m].dot(c & 3u, xs);
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[r][m] = group_sum<LPR>(acc[r][m]);
    if (li == 0) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            if (!yrow[r]) continue;
            float out = acc[r][0];
            if constexpr (MODE == GV_GEGLU) out = gelu_fast(acc[r][0]) * acc[r][1];
            *yrow[r] = out;
        }
    }
}

#ifndef ZL_GEMV_Q4KB
#define ZL_GEMV_Q4KB 1
#endif
// Launches k_gemv_q4kb for batch-1 Q4_K products with a whole number of 8-chunk groups per row
// (cols % 512 == 0), at most kQ4bMaxB chunks per lane at 8 to 64 lanes per row, 16-byte
// aligned matrices and x within the LDS; returns false otherwise. Lanes per row as the Q4_0
// kernel's (the fewest that take every chunk in kQ4bMaxB steps, more while the grid has under
// ZL_GEMV_Q4B_WAVES waves); one row per set.
template <int QT, int MODE, bool PRO>
static bool launch_q4kb(const GemvArgs& a, hipStream_t s) {
    // (not the GeGLU pair: holding both matrices' chunks, the compiler converts every quant of
    // a chunk to f32 ahead of the arithmetic and runs out of registers)
    if constexpr (QT != HIP_BRIDGE_Q4_K || MODE == GV_GEGLU) {
        return false;
    } else {
    if (!ZL_GEMV_Q4KB || a.batch != 1 || a.cols % 512 != 0) return false;
    for (int i = 0; i < a.nseg; ++i)
        if (a.seg[i].rows > 0 && !aligned16(a.seg[i].w)) return false;
    if (MODE == GV_GEGLU && !aligned16(a.w_up)) return false;
    const int nch = a.cols / 64;
    const size_t lds = (size_t)nch * kQ4kbXStride * sizeof(float);
    if (a.cols > (PRO ? kQ4bProMaxCols : kQ4bMaxCols) || lds > 65536) return false;
    constexpr int NW = PRO ? ZL_GEMV_Q4B_PRO_WAVES : ZL_GEMV_Q4B_NW;
    int lpr = 0;
    for (int l : {8, 16, 32, 64})
        if (!lpr && nch % l == 0 && nch / l <= kQ4bMaxB) lpr = l;
    if (!lpr) return false;
    auto waves = [&](int l) { return cdiv(a.total_rows, (int64_t)(kWave / l)); };
    while (lpr < 64 && waves(lpr) < ZL_GEMV_Q4B_WAVES && nch % (2 * lpr) == 0) lpr *= 2;
    const int bpl = nch / lpr;
    const unsigned grid = (unsigned)cdiv(waves(lpr), (int64_t)NW);
    auto go = [&](auto lpr_c) {
        constexpr int L = decltype(lpr_c)::value;
        switch (bpl) {
            case 1: k_gemv_q4kb<MODE, L, 1, 1, PRO, NW><<<grid, NW * kWave, lds, s>>>(a); break;
            case 2: k_gemv_q4kb<MODE, L, 1, 2, PRO, NW><<<grid, NW * kWave, lds, s>>>(a); break;
            case 3: k_gemv_q4kb<MODE, L, 1, 3, PRO, NW><<<grid, NW * kWave, lds, s>>>(a); break;
            case 4: k_gemv_q4kb<MODE, L, 1, 4, PRO, NW><<<grid, NW * kWave, lds, s>>>(a); break;
            case 5: k_gemv_q4kb<MODE, L, 1, 5, PRO, NW><<<grid, NW * kWave, lds, s>>>(a); break;
            default: k_gemv_q4kb<MODE, L, 1, 6, PRO, NW><<<grid, NW * kWave, lds, s>>>(a); break;
        }
    };
    if (lpr == 8) go(std::integral_constant<int, 8>{});
    else if (lpr == 16) go(std::integral_constant<int, 16>{});
    else if (lpr == 32) go(std::integral_constant<int, 32>{});
    else go(std::integral_constant<int, 64>{});
    return true;
    }
}

// Batch-1 Q6_K products, the same scheme over 64-column quarter chunks. A Q6_K super-block
// (210 bytes, 256 columns: ql[128] low nibbles, qh[64] two high bits each, int8 scales[16],
// f16 d; types.zig:187-192) holds four quarters (n, p), n the 128-column half, p the 16-column
// half of each of its four 32-column quadrants qd: quarter (n, p) is columns 128n + 32qd + 16p
// + i (i < 16), whose 6-bit values take their low nibbles from ql bytes 64n + 16p + i (qd 0
// low, qd 2 high) and 64n + 32 + 16p + i (qd 1 low, qd 3 high) and their high bits from qh
// byte 32n + 16p + i (bits 2qd, 2qd + 1), with scale 8n + 2qd + p (quant.zig:357-385,
// math.zig:556-616). A lane takes a whole quarter with three 16-byte loads and an 8-byte one
// (super-blocks are 210 bytes, so every other one starts 2 bytes past a dword: these are
// unaligned vector loads, which gfx950 serves from 2-byte aligned addresses) and the f16 d.
// x is staged per workgroup at 68 floats per quarter in the quarter's column order, its four
// 16-column sums at slots 64-67 (68 = 4 mod 32 puts the 8 lanes of a set, which read
// consecutive quarters, on distinct banks). Arithmetic as the group kernels:
// d * sum_qd sc_qd * (sum u x - 32 sum x) over each 16-column group.
constexpr int kQ6kbXStride = 68;
typedef u32x4 u32x4_a2 __attribute__((aligned(2)));
typedef u32x2 u32x2_a2 __attribute__((aligned(2)));
struct Q6Chunk {
    u32x4 a, b, h;  // ql bytes 64n+16p .. +16, 64n+32+16p .. +16; qh bytes 32n+16p .. +16
    u32x2 s;        // scale bytes 8n .. 8n+7
    uint32_t d;     // f16 d
    __device__ __forceinline__ void load(const unsigned char* sb, uint32_t n, uint32_t p) {
        a = *reinterpret_cast<const u32x4_a2*>(sb + 64u * n + 16u * p);
        b = *reinterpret_cast<const u32x4_a2*>(sb + 64u * n + 32u + 16u * p);
        h = *reinterpret_cast<const u32x4_a2*>(sb + 128u + 32u * n + 16u * p);
        s = *reinterpret_cast<const u32x2_a2*>(sb + 192u + 8u * n);
        d = *reinterpret_cast<const uint16_t*>(sb + 208u);
    }
    // xs: the quarter's x in LDS (quadrant qd at slots 16 qd .., its sum at 64 + qd).
    __device__ __forceinline__ float dot(uint32_t p, const float* xs) const {
        const uint32_t A[4] = {a.x, a.y, a.z, a.w}, Bq[4] = {b.x, b.y, b.z, b.w}, H[4] = {h.x, h.y, h.z, h.w};
        float r = 0.0f;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            f32x4 xv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[i] = *reinterpret_cast<const f32x4*>(xs + 16 * qd + 4 * i);
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // 6-bit values of columns 4i .. 4i+3 of quadrant qd (the high bits masked, then
                // one and-or with the low nibbles)
                const uint32_t lo = qd == 0 ? A[i] : qd == 1 ? Bq[i] : qd == 2 ? A[i] >> 4 : Bq[i] >> 4;
                const uint32_t hi = qd == 0 ? H[i] << 4 : qd == 1 ? H[i] << 2 : qd == 2 ? H[i] : H[i] >> 2;
                const uint32_t u = and_or(lo, 0x0f0f0f0fu, mask_bytes(hi, 0x30303030u));
                t = i == 0 ? (float)(u & 0xff) * xv[0].x : fmaf((float)(u & 0xff), xv[i].x, t);
                t = fmaf((float)((u >> 8) & 0xff), xv[i].y, t);
                t = fmaf((float)((u >> 16) & 0xff), xv[i].z, t);
                t = fmaf((float)(u >> 24), xv[i].w, t);
            }
            // scale byte 2 qd + p of the half's eight
            const uint32_t w = qd < 2 ? s.x : s.y;
            const float sc = (float)(int32_t)__builtin_amdgcn_sbfe((int32_t)w, 16u * (qd & 1) + 8u * p, 8u);
            const float g = fmaf(-32.0f, xs[64 + qd], t);
            r = qd == 0 ? sc * g : fmaf(sc, g, r);
        }
        return h2f(d & 0xffffu) * r;
    }
};

// (4 waves per SIMD, up to 128 registers, where x takes at most 4 float4 per thread and no
// prologue: six quarters of weights and a quadrant of x fit without spilling; otherwise 3)
template <int MODE, int LPR, int BPL, bool PRO, int NW, int MAXC>
__global__ __launch_bounds__(NW * kWave, (PRO || MAXC > kQ4bProMaxCols ? 3 : 4) * 4 / NW) void k_gemv_q6kb(GemvArgs a) {
    constexpr int T = NW * kWave;
    constexpr int SETS = kWave / LPR;
    constexpr int XK = MAXC / 4 / T;  // x float4 per thread (MAXC: the most columns taken)
    extern __shared__ __attribute__((aligned(16))) float s_xq[];
    __shared__ float s_red[NW];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int li = lane % LPR, set = lane / LPR;
    const int row0 = (blockIdx.x * NW + wv) * SETS + set;
    const int n4 = a.cols / 4;
    f32x4 xv[XK], rv[PRO ? XK : 1], rwv[PRO ? XK : 1], wnv[PRO ? XK : 1];
    if constexpr (PRO) {
        q4b_pro_load<XK, T>(a, xv, rv, rwv, wnv);
    } else {
#pragma unroll
        for (int k = 0; k < XK; ++k) {
            const int i = (int)threadIdx.x + k * T;
            if (i < n4) xv[k] = ldf4(a.x + 4 * i);
        }
    }
    const int r0 = a.seg[0].rows, r1 = a.nseg > 1 ? a.seg[1].rows : 0;
    const bool ok = row0 < a.total_rows;
    const int R = ok ? row0 : a.total_rows - 1;  // past the end: the last row, not written
    const bool s0 = R < r0, s1 = !s0 && R - r0 < r1;
    const int Rs = s0 ? R : s1 ? R - r0 : R - r0 - r1;
    const unsigned char* wrow = (s0 ? a.seg[0].w : s1 ? a.seg[1].w : a.seg[2].w) + (int64_t)Rs * a.row_bytes;
    float* yrow = ok ? (s0 ? a.seg[0].y : s1 ? a.seg[1].y : a.seg[2].y) + Rs : nullptr;
    Q6Chunk w[BPL];
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const uint32_t c = (uint32_t)(li + LPR * j);
        w[j].load(wrow + (c >> 2) * 210u, (c >> 1) & 1u, c & 1u);
    }
    if constexpr (PRO) q4b_pro_finish<XK, T>(a, xv, rv, rwv, wnv, s_red);
    // x into LDS: float4 i (columns 4i ..) of super-block i / 64 goes to quarter
    // (n, p) = (bit 5, bit 2 of i), quadrant qd = bits 3-4, slot 16 qd + 4 (i & 3); the sum of
    // each 16-column group (4 consecutive float4s, lanes 4k .. 4k+3) by two DPP row shifts.
#pragma unroll
    for (int k = 0; k < XK; ++k) {
        const int i = (int)threadIdx.x + k * T;
        if (k * T >= n4) break;  // uniform
        const float s4 = i < n4 ? (xv[k].x + xv[k].y) + (xv[k].z + xv[k].w) : 0.0f;
        const float v = s4 + dpp<0x111>(s4);  // row_shr:1
        const float gs = v + dpp<0x112>(v);   // row_shr:2
        if (i < n4) {
            const int c = ((i >> 6) << 2) | (((i >> 5) & 1) << 1) | ((i >> 2) & 1);
            const int qd = (i >> 3) & 3;
            float* xs = s_xq + c * kQ6kbXStride;
            *reinterpret_cast<f32x4*>(xs + 16 * qd + 4 * (i & 3)) = xv[k];
            if ((i & 3) == 3) xs[64 + qd] = gs;
        }
    }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const uint32_t c = (uint32_t)(li + LPR * j);
        acc += w[j].dot(c & 1u, s_xq + c * kQ6kbXStride);
    }
    acc = group_sum<LPR>(acc);
    if (li == 0 && yrow) *yrow = acc;
}

#ifndef ZL_GEMV_Q6KB
#define ZL_GEMV_Q6KB 1
#endif
// Launches k_gemv_q6kb for batch-1 Q6_K products with a whole number of 8-quarter groups per
// row (cols % 512 == 0), at most kQ4bMaxB quarters per lane at 8 to 64 lanes per row and x
// within the LDS; returns false otherwise. Lanes per row as the Q4_K kernel's; one row per
// set. (Not the GeGLU pair: two matrices' quarters do not fit the registers.)
template <int QT, int MODE, bool PRO>
static bool launch_q6kb(const GemvArgs& a, hipStream_t s) {
    if constexpr (QT != HIP_BRIDGE_Q6_K || MODE == GV_GEGLU) {
        return false;
    } else {
    if (!ZL_GEMV_Q6KB || a.batch != 1 || a.cols % 512 != 0) return false;
    const int nch = a.cols / 64;
    const size_t lds = (size_t)nch * kQ6kbXStride * sizeof(float);
    if (a.cols > (PRO ? kQ4bProMaxCols : kQ4bMaxCols) || lds > 65536) return false;
    constexpr int NW = PRO ? ZL_GEMV_Q4B_PRO_WAVES : ZL_GEMV_Q4B_NW;
    // (with the prologue at most 5 quarters per lane: 6 spill)
    const int maxb = PRO ? 5 : kQ4bMaxB;
    int lpr = 0;
    for (int l : {8, 16, 32, 64})
        if (!lpr && nch % l == 0 && nch / l <= maxb) lpr = l;
    if (!lpr) return false;
    auto waves = [&](int l) { return cdiv(a.total_rows, (int64_t)(kWave / l)); };
    while (lpr < 64 && waves(lpr) < ZL_GEMV_Q4B_WAVES && nch % (2 * lpr) == 0) lpr *= 2;
    const int bpl = nch / lpr;
    const unsigned grid = (unsigned)cdiv(waves(lpr), (int64_t)NW);
    // x staged through registers: kQ4bProMaxCols columns' worth per thread for products up
    // to that width (fewer registers held beside the weights), kQ4bMaxCols' above
    const bool narrow = PRO || a.cols <= kQ4bProMaxCols;
    auto go = [&](auto lpr_c) {
        constexpr int L = decltype(lpr_c)::value;
        auto go2 = [&](auto c_c) {
            constexpr int MC = decltype(c_c)::value;
            switch (bpl) {
                case 1: k_gemv_q6kb<MODE, L, 1, PRO, NW, MC><<<grid, NW * kWave, lds, s>>>(a); break;
                case 2: k_gemv_q6kb<MODE, L, 2, PRO, NW, MC><<<grid, NW * kWave, lds, s>>>(a); break;
                case 3: k_gemv_q6kb<MODE, L, 3, PRO, NW, MC><<<grid, NW * kWave, lds, s>>>(a); break;
                case 4: k_gemv_q6kb<MODE, L, 4, PRO, NW, MC><<<grid, NW * kWave, lds, s>>>(a); break;
                case 5: k_gemv_q6kb<MODE, L, 5, PRO, NW, MC><<<grid, NW * kWave, lds, s>>>(a); break;
                default: k_gemv_q6kb<MODE, L, PRO ? 5 : 6, PRO, NW, MC><<<grid, NW * kWave, lds, s>>>(a); break;
            }
        };
        if (narrow) go2(std::integral_constant<int, kQ4bProMaxCols>{});
        else if constexpr (!PRO) go2(std::integral_constant<int, kQ4bMaxCols>{});
    };
    if (lpr == 8) go(std::integral_constant<int, 8>{});
    else if (lpr == 16) go(std::integral_constant<int, 16>{});
    else if (lpr == 32) go(std::integral_constant<int, 32>{});
    else go(std::integral_constant<int, 64>{});
    return true;
    }
}

// Any alignment / column count: one workgroup per row, scalar dequantisation per element.
template <int QT>
__device__ __forceinline__ float w_elem(const unsigned char* row, int c) {
    if constexpr (QT == HIP_BRIDGE_Q4_0) {
        const unsigned char* blk = row + (c >> 5) * 18;
        const int o = c & 31;
        const int byte = blk[2 + (o & 15)];
        const int q = (o < 16 ? (byte & 0xf) : (byte >> 4)) - 8;
        return (float)q * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    } else if constexpr (QT == HIP_BRIDGE_Q8_0) {
        const unsigned char* blk = row + (c >> 5) * 34;
        return (float)(int8_t)blk[2 + (c & 31)] * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    } else if constexpr (QT == HIP_BRIDGE_Q4_K) {
        const unsigned char* sb = row + (c >> 8) * 144;
        const int w = c & 255, jj = w >> 6, hi = (w >> 5) & 1, j = 2 * jj + hi;
        const unsigned char* sc = sb + 4;
        const int s6 = j < 4 ? (sc[j] & 63) : ((sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4));
        const int m6 = j < 4 ? (sc[j + 4] & 63) : ((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
        const float d = h2f((uint32_t)sb[0] | ((uint32_t)sb[1] << 8));
        const float dmin = h2f((uint32_t)sb[2] | ((uint32_t)sb[3] << 8));
        const int byte = sb[16 + 32 * jj + (w & 31)];
        return (float)(hi ? byte >> 4 : byte & 0x0F) * (d * (float)s6) - dmin * (float)m6;
    } else if constexpr (QT == HIP_BRIDGE_Q6_K) {
        const unsigned char* sb = row + (c >> 8) * 210;
        const int w = c & 255, half = w >> 7, grp = (w & 127) >> 5, l = w & 31;
        const int lo = (sb[half * 64 + l + ((grp & 1) ? 32 : 0)] >> ((grp & 2) ? 4 : 0)) & 0xf;
        const int hi = (sb[128 + half * 32 + l] >> (2 * grp)) & 3;
        const int8_t sc = (int8_t)sb[192 + half * 8 + (l >> 4) + 2 * grp];
        const float d = h2f((uint32_t)sb[208] | ((uint32_t)sb[209] << 8));
        return d * (float)sc * (float)((lo | (hi << 4)) - 32);
    } else if constexpr (QT == HIP_BRIDGE_F32) {
        const unsigned char* p = row + 4 * (size_t)c;
        return __uint_as_float((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                               ((uint32_t)p[3] << 24));
    } else {
        const unsigned char* p = row + 2 * (size_t)c;
        const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
        return QT == HIP_BRIDGE_BF16 ? bf16_lo(h) : h2f(h);
    }
}

template <int QT, int MODE>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_scalar(GemvArgs a) {
    __shared__ float s_red[2][kGemvWaves];
    int R = blockIdx.x;
    int s = 0;
    if (a.nseg > 1 && R >= a.seg[0].rows) {
        R -= a.seg[0].rows;
        s = 1;
        if (a.nseg > 2 && R >= a.seg[1].rows) {
            R -= a.seg[1].rows;
            s = 2;
        }
    }
    const unsigned char* wr = a.seg[s].w + (int64_t)R * a.row_bytes;
    const unsigned char* ur = MODE == GV_GEGLU ? a.w_up + (int64_t)R * a.row_bytes : nullptr;
    for (int b = 0; b < a.batch; ++b) {
        const float* xr = a.x + (int64_t)b * a.cols;
        float sg = 0.0f, su = 0.0f;
        for (int c = threadIdx.x; c < a.cols; c += kGemvThreads) {
            sg = fmaf(w_elem<QT>(wr, c), xr[c], sg);
            if constexpr (MODE == GV_GEGLU) su = fmaf(w_elem<QT>(ur, c), xr[c], su);
        }
        sg = group_sum<kWave>(sg);
        su = group_sum<kWave>(su);
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) {
            s_red[0][wave] = sg;
            s_red[1][wave] = su;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const float g = (s_red[0][0] + s_red[0][1]) + (s_red[0][2] + s_red[0][3]);
            float out = g;
            if constexpr (MODE == GV_GEGLU) {
                const float u = (s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]);
                out = gelu_fast(g) * u;
            }
            a.seg[s].y[(int64_t)b * a.seg[s].rows + R] = out;
        }
        __syncthreads();
    }
}

static int64_t gemv_row_bytes(int qtype, int cols) {
    switch (qtype) {
        case HIP_BRIDGE_F32: return (int64_t)cols * 4;
        case HIP_BRIDGE_F16:
        case HIP_BRIDGE_BF16: return (int64_t)cols * 2;
        case HIP_BRIDGE_Q8_0: return cols % 32 ? -1 : (int64_t)(cols / 32) * 34;
        case HIP_BRIDGE_Q4_0: return cols % 32 ? -1 : (int64_t)(cols / 32) * 18;
        case HIP_BRIDGE_Q4_K: return cols % 256 ? -1 : (int64_t)(cols / 256) * 144;
        case HIP_BRIDGE_Q6_K: return cols % 256 ? -1 : (int64_t)(cols / 256) * 210;
        default: return -1;
    }
}

// Rows per workgroup (x is reused across them from registers) against workgroup count:
// measured on Gemma-4B decode shapes, small matrices (1024-4096 rows) want 2 rows and more
// workgroups, large ones 4, Q4_0 (the most x per weight byte) 8 from 16384 rows. GeGLU
// reads two matrices per row and takes half as many rows; Q4_0 GeGLU products take 4 row
// pairs from 4096 pairs (gate-up 2 x 6144 x 1536: 7.6 -> 6.4 us; 2 x 10240 x 2560: 12.6 ->
// 11.8 us).
template <int QT, int MODE, bool PRO>
static void launch_vec(const GemvArgs& a, hipStream_t s) {
    constexpr int H = MODE == GV_GEGLU ? 2 : 1;
    const unsigned g8 = (unsigned)cdiv(a.total_rows, 8 / H), g4 = (unsigned)cdiv(a.total_rows, 4 / H),
                   g2 = (unsigned)cdiv(a.total_rows, 2 / H);
    if (PRO && (launch_q4b<QT, MODE, true>(a, s) || launch_q4kb<QT, MODE, true>(a, s) ||
                launch_q6kb<QT, MODE, true>(a, s))) {
        // launched: batch-1 Q4_0 / Q8_0 / Q4_K / Q6_K block kernel with the prologue
    } else if (PRO) {  // batch 1; the input vector in dynamic LDS; at most kGemvProGrid workgroups
        const size_t lds = (size_t)a.cols * sizeof(float);
        const unsigned cap = kGemvProGrid;
        if (QT == HIP_BRIDGE_Q4_0 && a.total_rows >= 16384)
            k_gemv<QT, 8 / H, 1, MODE, true><<<std::min(g8, cap), kGemvThreads, lds, s>>>(a);
        else if (a.total_rows >= 8192)
            k_gemv<QT, 4 / H, 1, MODE, true><<<std::min(g4, cap), kGemvThreads, lds, s>>>(a);
        else
            k_gemv<QT, 2 / H, 1, MODE, true><<<std::min(g2, cap), kGemvThreads, lds, s>>>(a);
    } else if (ZL_GEMV_FORCE != 0 && a.batch == 1) {  // tuning builds only (see the macro)
        constexpr int F = ZL_GEMV_FORCE;
        constexpr bool blockq = QT != HIP_BRIDGE_F16 && QT != HIP_BRIDGE_BF16 && QT != HIP_BRIDGE_F32;
        if constexpr (F < 0 && blockq) {
            constexpr int RW = std::max(1, -F / H);
            if (a.cols <= kGemvWaveColsMax)  // x in LDS: at most 64 KB
                k_gemv_w<QT, RW, MODE><<<(unsigned)cdiv(a.total_rows, (int64_t)RW * kGemvWaves), kGemvThreads, (size_t)a.cols * 4, s>>>(a);
            else
                k_gemv<QT, 2 / H, 1, MODE><<<g2, kGemvThreads, 0, s>>>(a);
        } else {
            constexpr int RP = F > 0 ? std::max(1, F / H) : 2 / H;
            k_gemv<QT, RP, 1, MODE><<<(unsigned)cdiv(a.total_rows, RP), kGemvThreads, 0, s>>>(a);
        }
    } else if (launch_q4b<QT, MODE, false>(a, s) || launch_q4kb<QT, MODE, false>(a, s) ||
               launch_q6kb<QT, MODE, false>(a, s)) {
        // launched: batch-1 Q4_0 / Q8_0 with 256-column multiples, Q4_K / Q6_K with 512
    } else if (MODE == GV_PLAIN && a.batch == 1 && a.total_rows >= kGemvWaveRowsMin && a.cols <= kGemvWaveColsMax &&
               QT != HIP_BRIDGE_F16 && QT != HIP_BRIDGE_BF16 && QT != HIP_BRIDGE_F32) {
        // (k_gemv_w is instantiated for these cases only)
        if constexpr (MODE == GV_PLAIN && QT != HIP_BRIDGE_F16 && QT != HIP_BRIDGE_BF16 && QT != HIP_BRIDGE_F32) {
        // LM-head-sized block-quantised products: wave-owned rows (measured, 262144 x 2560,
        // us: Q4_K 226 -> 157 with 2 rows per wave, Q6_K 310 -> 177 with 4, Q8_0 185 -> 173
        // and Q4_0 137 -> 113 with 8; smaller matrices, whose rows are long against their
        // count, and dense types are faster above: 2560 x 10240 Q4_0 8.0 us above, 14.6 here)
        constexpr int RW = QT == HIP_BRIDGE_Q4_K ? 2 : QT == HIP_BRIDGE_Q6_K ? 4 : 8;
        k_gemv_w<QT, RW, MODE><<<(unsigned)cdiv(a.total_rows, (int64_t)RW * kGemvWaves), kGemvThreads, (size_t)a.cols * 4, s>>>(a);
        }
    } else if (a.batch == 1) {
        if (QT == HIP_BRIDGE_Q4_0 && (a.total_rows >= 16384 || (MODE == GV_GEGLU && a.total_rows >= 4096)))
            k_gemv<QT, 8 / H, 1, MODE><<<g8, kGemvThreads, 0, s>>>(a);
        else if (a.total_rows >= 8192)
            k_gemv<QT, 4 / H, 1, MODE><<<g4, kGemvThreads, 0, s>>>(a);
        else
            k_gemv<QT, 2 / H, 1, MODE><<<g2, kGemvThreads, 0, s>>>(a);
    } else if (a.batch == 2) {
        k_gemv<QT, 4 / H, 2, MODE><<<g4, kGemvThreads, 0, s>>>(a);
    } else {
        k_gemv<QT, 2 / H, 4, MODE><<<g2, kGemvThreads, 0, s>>>(a);
    }
}

template <int MODE>
static void launch_gemv(int qtype, GemvArgs& a, hipStream_t s) {
    if (a.total_rows <= 0 || a.cols <= 0 || a.batch <= 0) return;
    a.row_bytes = gemv_row_bytes(qtype, a.cols);
    if (a.row_bytes < 0) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    if (!a.x || (MODE == GV_GEGLU && !a.w_up)) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    // Vector path: x 16-byte aligned, cols % 8 == 0; Q4_0 / Q8_0 rows 2-byte aligned (16-bit
    // loads), dense rows 16-byte aligned (cols % 8 == 0 makes every row so).
    // weight alignment the vector loads need: 2 bytes for Q4_0 / Q8_0 / Q6_K blocks (16-bit
    // loads), 4 for Q4_K (32-bit loads; 144-byte blocks), 16 for dense rows
    const uintptr_t walign = qtype == HIP_BRIDGE_Q4_0 || qtype == HIP_BRIDGE_Q8_0 || qtype == HIP_BRIDGE_Q6_K ? 1u
                             : qtype == HIP_BRIDGE_Q4_K                                                   ? 3u
                                                                                                          : 15u;
    auto w_ok = [&](const void* w) { return (reinterpret_cast<uintptr_t>(w) & walign) == 0; };
    bool ok = a.cols % 8 == 0 && aligned16(a.x);
    for (int i = 0; i < a.nseg; ++i) {
        if (a.seg[i].rows <= 0) continue;
        if (!a.seg[i].w || !a.seg[i].y) {
            set_error(HIP_BRIDGE_EINVAL);
            return;
        }
        ok = ok && w_ok(a.seg[i].w);
    }
    if (MODE == GV_GEGLU) ok = ok && w_ok(a.w_up);
    const GemvPro& p = a.pro;
    if (p.mode != GP_NONE) {
        // prologue: batch 1, vector path, input vector within LDS, 16-byte aligned operands
        const bool args = (p.mode == GP_NORM || p.mode == GP_GEGLU) && (p.mode != GP_GEGLU || p.r) &&
                          (p.r || !p.r_w);
        if (!args) {
            set_error(HIP_BRIDGE_EINVAL);
            return;
        }
        const bool pro_ok = ok && a.batch == 1 && a.cols <= kGemvProMaxCols && aligned16(p.r) &&
                            aligned16(p.r_w) && aligned16(p.w) && aligned16(p.x_out) && aligned16(p.xb_out);
        if (!pro_ok) {
            set_error(HIP_BRIDGE_EUNSUPPORTED);
            return;
        }
        switch (qtype) {
            case HIP_BRIDGE_Q4_0: launch_vec<HIP_BRIDGE_Q4_0, MODE, true>(a, s); break;
            case HIP_BRIDGE_Q8_0: launch_vec<HIP_BRIDGE_Q8_0, MODE, true>(a, s); break;
            case HIP_BRIDGE_Q4_K: launch_vec<HIP_BRIDGE_Q4_K, MODE, true>(a, s); break;
            case HIP_BRIDGE_Q6_K: launch_vec<HIP_BRIDGE_Q6_K, MODE, true>(a, s); break;
            case HIP_BRIDGE_F16: launch_vec<HIP_BRIDGE_F16, MODE, true>(a, s); break;
            case HIP_BRIDGE_BF16: launch_vec<HIP_BRIDGE_BF16, MODE, true>(a, s); break;
            default: launch_vec<HIP_BRIDGE_F32, MODE, true>(a, s); break;
        }
    } else if (ok) {
        switch (qtype) {
            case HIP_BRIDGE_Q4_0: launch_vec<HIP_BRIDGE_Q4_0, MODE, false>(a, s); break;
            case HIP_BRIDGE_Q8_0: launch_vec<HIP_BRIDGE_Q8_0, MODE, false>(a, s); break;
            case HIP_BRIDGE_Q4_K: launch_vec<HIP_BRIDGE_Q4_K, MODE, false>(a, s); break;
            case HIP_BRIDGE_Q6_K: launch_vec<HIP_BRIDGE_Q6_K, MODE, false>(a, s); break;
            case HIP_BRIDGE_F16: launch_vec<HIP_BRIDGE_F16, MODE, false>(a, s); break;
            case HIP_BRIDGE_BF16: launch_vec<HIP_BRIDGE_BF16, MODE, false>(a, s); break;
            default: launch_vec<HIP_BRIDGE_F32, MODE, false>(a, s); break;
        }
    } else {
        const unsigned grid = (unsigned)a.total_rows;
        switch (qtype) {
            case HIP_BRIDGE_Q4_0: k_gemv_scalar<HIP_BRIDGE_Q4_0, MODE><<<grid, kGemvThreads, 0, s>>>(a); break;
            case HIP_BRIDGE_Q8_0: k_gemv_scalar<HIP_BRIDGE_Q8_0, MODE><<<grid, kGemvThreads, 0, s>>>(a); break;
            case HIP_BRIDGE_Q4_K: k_gemv_scalar<HIP_BRIDGE_Q4_K, MODE><<<grid, kGemvThreads, 0, s>>>(a); break;
            case HIP_BRIDGE_Q6_K: k_gemv_scalar<HIP_BRIDGE_Q6_K, MODE><<<grid, kGemvThreads, 0, s>>>(a); break;
            case HIP_BRIDGE_F16: k_gemv_scalar<HIP_BRIDGE_F16, MODE><<<grid, kGemvThreads, 0, s>>>(a); break;
            case HIP_BRIDGE_BF16: k_gemv_scalar<HIP_BRIDGE_BF16, MODE><<<grid, kGemvThreads, 0, s>>>(a); break;
            default: k_gemv_scalar<HIP_BRIDGE_F32, MODE><<<grid, kGemvThreads, 0, s>>>(a); break;
        }
    }
    check_launch();
}

// ---- small batches on the matrix cores ------------------------------------------------------
// Products of 2 to gemm_mfma_min_batch - 1 tokens (hip_gemm below the prefill GEMM) with Q4_0,
// Q8_0, Q4_K, Q6_K or BF16 weights: v_mfma_f32_16x16x32_bf16 over tiles of 16 tokens x 16 rows x one
// 32-column block, tokens on the A side (each x as three bf16 terms h + m + l, as the prefill
// GEMM: exact to the f32 value's 24 bits), rows on the B side. Block quants enter as their
// unsigned codes u (Q4_0 nibbles 0..15, Q8_0 q ^ 0x80: exact in bf16) and a block's sum is
// d * (sum u x - c * sum x), c = 8 / 128, the batch-1 kernels' arithmetic; sum x per token and
// block comes from three more MFMAs against a ones operand. A wave takes NT 16-row tiles over
// a 1/KS share of the blocks and converts each block's x once for its NT tiles; the KS waves
// of a workgroup cover the whole width and are added in wave order through LDS. Layouts
// (16x16x32): lane l supplies A row (token) l % 16 and B column (weight row) l % 16, each over
// the block's columns 8 (l / 16) .. + 8, and holds D[4 (l / 16) + r][l % 16], r < 4.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kMbTok = 16;  // tokens per tile

// x0, x1 -> three packed bf16 pairs (h, m, l) with x = h + m + l (each term RNE of the rest).
__device__ __forceinline__ void mb_split3(float x0, float x1, uint32_t& h, uint32_t& m, uint32_t& l) {
    h = pack_bf16x2(x0, x1);
    x0 -= bf16_lo(h);
    x1 -= bf16_hi(h);
    m = pack_bf16x2(x0, x1);
    x0 -= bf16_lo(m);
    x1 -= bf16_hi(m);
    l = pack_bf16x2(x0, x1);
}
// Four byte codes (0..255) -> two packed bf16 pairs (small integers: the f32's high half).
__device__ __forceinline__ void mb_codes(uint32_t u, uint32_t& p0, uint32_t& p1) {
    const float f0 = (float)(u & 0xffu), f1 = (float)((u >> 8) & 0xffu);
    const float f2 = (float)((u >> 16) & 0xffu), f3 = (float)(u >> 24);
    p0 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    p1 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}

template <int QT, int NT, int KS>
__global__ __launch_bounds__(KS * kWave) void k_gemv_mb(GemvArgs a) {
    constexpr bool SC = QT != HIP_BRIDGE_BF16;
    // Q4_K: a 32-column block is sub-block j = kb % 8 of super-block kb / 8 (144 bytes:
    // {f16 d, f16 dmin, scales[12], qs[128]}); its codes are the low (j even) or high nibbles
    // of qs[32 (j / 2) ..], and its sum is (d sc_j) sum u x - (dmin m_j) sum x
    constexpr bool KQ = QT == HIP_BRIDGE_Q4_K;
    // Q6_K: a 32-column block is quadrant t of half n (kb % 8 = 4 n + t) of super-block kb / 8
    // (210 bytes: {ql[128], qh[64], int8 scales[16], f16 d}); lane group g's 8 values take the
    // low (t < 2) or high nibbles of ql[64 n + 32 (t & 1) + 8 g ..], bits 2t, 2t + 1 of
    // qh[32 n + 8 g ..] and scale sc[8 n + g / 2 + 2 t]; sc * (u - 32) (at most 13 bits) enters
    // as two exact bf16 terms, and the super-block's d scales the block's sum
    constexpr bool Q6 = QT == HIP_BRIDGE_Q6_K;
    constexpr uint32_t BB = QT == HIP_BRIDGE_Q4_0 ? 18u : QT == HIP_BRIDGE_Q8_0 ? 34u : KQ ? 144u : Q6 ? 210u : 64u;  // bytes / block
    constexpr float C = QT == HIP_BRIDGE_Q4_0 ? 8.0f : 128.0f;
    __shared__ f32x4 s_red[KS][NT][kWave];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int mn = lane & 15, g = lane >> 4;
    const int t0 = blockIdx.y * kMbTok;
    const int r0 = blockIdx.x * 16 * NT;
    const int nblk = a.cols / 32;
    // the workgroup's blocks: all, or with gridDim.z = 2 one half (added into zeroed y)
    const int kbs = (int)((int64_t)nblk * blockIdx.z / gridDim.z), kbn = (int)((int64_t)nblk * (blockIdx.z + 1) / gridDim.z) - kbs;
    const int kb0 = kbs + (int)((int64_t)kbn * wv / KS), kb1 = kbs + (int)((int64_t)kbn * (wv + 1) / KS);
    // the x row of token t0 + mn (past the batch: token 0's, zeroed), columns 8g .. of a block
    const bool tok_ok = t0 + mn < a.batch;
    const float* xr = a.x + (int64_t)(tok_ok ? t0 + mn : 0) * a.cols + 8 * g;
    // the weight row of tile j (past the last row: the last row, not stored)
    const unsigned char* wrow[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int row = min(r0 + 16 * j + mn, a.total_rows - 1);
        wrow[j] = a.seg[0].w + (int64_t)row * a.row_bytes;
    }
    // the lane's quant bytes in a block: Q4_0 columns 8g .. are the low (g < 2) / high nibbles
    // of bytes 8 (g & 1) ..; Q8_0 bytes 8g ..; BF16 elements 8g ..
    const uint32_t qoff = QT == HIP_BRIDGE_Q4_0 ? 2u + 8u * (g & 1) : QT == HIP_BRIDGE_Q8_0 ? 2u + 8u * g : KQ ? 16u + 8u * g : 16u * g;
    const uint32_t nsh = QT == HIP_BRIDGE_Q4_0 ? 4u * (g >> 1) : 0u;
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (__bf16)1.0f;
    f32x4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // One block at a time (measured: issuing 2-6 blocks' loads before their arithmetic was
    // slower at every shape, 20.0 -> 22.5-25.3 us for 10240 x 2560 at 8 tokens).
    for (int kb = kb0; kb < kb1; ++kb) {
        const f32x4 xa = ldf4(xr + 32 * kb), xb = ldf4(xr + 32 * kb + 4);
        u32x4 wq[NT];
        uint32_t dd[NT];
        uint32_t ks3[KQ ? NT : 1][3];  // Q4_K: scales[12] of the super-block
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const unsigned char* blk = wrow[j] + BB * (uint32_t)kb;
            if constexpr (Q6) {
                const unsigned char* sb = wrow[j] + BB * (uint32_t)(kb >> 3);
                const uint32_t n6 = ((uint32_t)kb >> 2) & 1u, t6 = (uint32_t)kb & 3u;
                const u32x2 ql = *reinterpret_cast<const u32x2_a2*>(sb + 64u * n6 + 32u * (t6 & 1u) + 8u * g);
                const u32x2 qh = *reinterpret_cast<const u32x2_a2*>(sb + 128u + 32u * n6 + 8u * g);
                wq[j] = u32x4{ql.x, ql.y, qh.x, qh.y};
                const uint32_t scw = ldw16(sb + 192u + 8u * n6 + 2u * t6);  // scales 8n+2t, 8n+2t+1
                dd[j] = ldw16(sb + 208u) | (((scw >> (8u * ((uint32_t)g >> 1))) & 0xffu) << 16);
            } else if constexpr (KQ) {
                const unsigned char* sb = wrow[j] + BB * (uint32_t)(kb >> 3);
                const u32x2 v = *reinterpret_cast<const u32x2_a2*>(sb + qoff + 32u * ((uint32_t)(kb & 7) >> 1));
                wq[j] = u32x4{v.x, v.y, 0u, 0u};
                dd[j] = ldw32_a2(sb);
#pragma unroll
                for (int i = 0; i < 3; ++i) ks3[j][i] = ldw32_a2(sb + 4u + 4u * i);
            } else if constexpr (QT == HIP_BRIDGE_BF16) {
                wq[j] = *reinterpret_cast<const u32x4*>(blk + qoff);
                dd[j] = 0;
            } else {
                const u32x2 v = *reinterpret_cast<const u32x2_a2*>(blk + qoff);
                wq[j] = u32x4{v.x, v.y, 0u, 0u};
                dd[j] = ldw16(blk);
            }
        }
        {
            const float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            u32x4 th, tm, tl;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t h, m, l;
                mb_split3(tok_ok ? xs[2 * e] : 0.0f, tok_ok ? xs[2 * e + 1] : 0.0f, h, m, l);
                th[e] = h;
                tm[e] = m;
                tl[e] = l;
            }
            const bf16x8 Ah = __builtin_bit_cast(bf16x8, th), Am = __builtin_bit_cast(bf16x8, tm),
                         Al = __builtin_bit_cast(bf16x8, tl);
            f32x4 sx{};
            if constexpr (SC && !Q6) {
                sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, ones, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Am, ones, sx, 0, 0, 0);
                sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, ones, sx, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                if constexpr (Q6) {
                    const uint32_t t6 = (uint32_t)kb & 3u, nsh6 = t6 < 2 ? 0u : 4u, hsh = 2u * t6;
                    const float sc = (float)(int8_t)(uint8_t)(dd[j] >> 16);
                    const uint32_t qlw[2] = {wq[j].x, wq[j].y}, qhw[2] = {wq[j].z, wq[j].w};
                    u32x4 hw, lw;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float v[2];
#pragma unroll
                        for (int k = 0; k < 2; ++k) {
                            const uint32_t b = 8u * (uint32_t)((2 * e + k) & 3), w = (uint32_t)(2 * e + k) >> 2;
                            const uint32_t u = ((qlw[w] >> (b + nsh6)) & 15u) | (((qhw[w] >> (b + hsh)) & 3u) << 4);
                            v[k] = sc * (float)((int)u - 32);  // an integer of at most 13 bits: exact
                        }
                        const uint32_t hi = pack_bf16x2(v[0], v[1]);
                        hw[e] = hi;
                        lw[e] = pack_bf16x2(v[0] - bf16_lo(hi), v[1] - bf16_hi(hi));
                    }
                    const bf16x8 Wh = __builtin_bit_cast(bf16x8, hw), Wl = __builtin_bit_cast(bf16x8, lw);
                    f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Wh, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Am, Wh, p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Wl, p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Wh, p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Am, Wl, p, 0, 0, 0);
                    const float d = h2f(dd[j] & 0xffffu);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[j][r] = fmaf(d, p[r], acc[j][r]);
                    continue;
                }
                u32x4 bw;
                if constexpr (QT == HIP_BRIDGE_BF16) {
                    bw = wq[j];
                } else {
                    uint32_t u0 = wq[j].x, u1 = wq[j].y;
                    if constexpr (KQ) {
                        const uint32_t ksh = 4u * ((uint32_t)kb & 1u);
                        u0 = mask_bytes(u0 >> ksh, 0x0f0f0f0fu);
                        u1 = mask_bytes(u1 >> ksh, 0x0f0f0f0fu);
                    } else if constexpr (QT == HIP_BRIDGE_Q4_0) {
                        u0 = mask_bytes(u0 >> nsh, 0x0f0f0f0fu);
                        u1 = mask_bytes(u1 >> nsh, 0x0f0f0f0fu);
                    } else {
                        u0 ^= 0x80808080u;
                        u1 ^= 0x80808080u;
                    }
                    uint32_t p0, p1, p2, p3;
                    mb_codes(u0, p0, p1);
                    mb_codes(u1, p2, p3);
                    bw = u32x4{p0, p1, p2, p3};
                }
                const bf16x8 Bw = __builtin_bit_cast(bf16x8, bw);
                if constexpr (SC) {
                    f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bw, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Am, Bw, p, 0, 0, 0);
                    p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Bw, p, 0, 0, 0);
                    if constexpr (KQ) {
                        // 6-bit scale and min of sub-block sj (quant.zig:285-290), as the prefill GEMM
                        const uint32_t sj = (uint32_t)kb & 7u, b = 8u * (sj & 3u);
                        const uint32_t s0 = (ks3[j][0] >> b) & 0xffu, s1 = (ks3[j][1] >> b) & 0xffu,
                                       s2 = (ks3[j][2] >> b) & 0xffu;
                        const uint32_t sc = sj < 4 ? (s0 & 63u) : ((s2 & 15u) | ((s0 >> 6) << 4));
                        const uint32_t mq = sj < 4 ? (s1 & 63u) : ((s2 >> 4) | ((s1 >> 6) << 4));
                        const float A = h2f(dd[j] & 0xffffu) * (float)sc, Bm = h2f(dd[j] >> 16) * (float)mq;
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[j][r] = fmaf(A, p[r], fmaf(-Bm, sx[r], acc[j][r]));
                    } else {
                        const float d = h2f(dd[j]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[j][r] = fmaf(d, fmaf(-C, sx[r], p[r]), acc[j][r]);
                    }
                } else {
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, Bw, acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Am, Bw, acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, Bw, acc[j], 0, 0, 0);
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) s_red[wv][j][lane] = acc[j];
    __syncthreads();
    if (wv == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            f32x4 t = s_red[0][j][lane];
#pragma unroll
            for (int w = 1; w < KS; ++w) t += s_red[w][j][lane];
            const int row = r0 + 16 * j + mn;
            if (row >= a.total_rows) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = t0 + 4 * g + r;
                if (tok >= a.batch) continue;
                float* const yp = a.seg[0].y + (int64_t)tok * a.total_rows + row;
                if (gridDim.z > 1) unsafeAtomicAdd(yp, t[r]);  // two halves: 0 + a + b in either order
                else *yp = t[r];
            }
        }
    }
}

#ifndef ZL_GEMV_MB
#define ZL_GEMV_MB 1
#endif
#ifndef ZL_GEMV_MB_SPLIT
#define ZL_GEMV_MB_SPLIT 1
#endif
#ifndef ZL_GEMV_MB_SPLIT_NT
#define ZL_GEMV_MB_SPLIT_NT 2
#endif
#ifndef ZL_GEMV_MB_WAVES
#define ZL_GEMV_MB_WAVES 1024
#endif
// Launches k_gemv_mb for a batch of 2 (Q6_K 8) to gemm_mfma_min_batch - 1 tokens (Q4_0 / Q8_0 /
// Q4_K / Q6_K with 2-byte aligned rows, BF16 with 16-byte aligned ones; cols % 32 == 0, K-quants
// % 256; at most
// 160 blocks, or 320 from 12 tokens; x 16-byte aligned); returns false otherwise (the vector
// kernels take the product).
template <int QT>
static bool launch_mb_t(const GemvArgs& a, hipStream_t s) {
    const int nblk = a.cols / 32;
    const int64_t tiles = cdiv(a.total_rows, 16), ttiles = cdiv(a.batch, kMbTok);
    // the fewest waves per workgroup that leave each at most 10 blocks (a wave's blocks are a
    // serial chain of memory round trips: longer rows keep the vector kernels, 2560 x 10240
    // at 8 tokens 22.7 us there against 35.5), then the widest row tiles that still give the
    // grid ZL_GEMV_MB_WAVES waves
    int ks = 0;
    for (int k : {4, 8, 16})
        if (!ks && cdiv(nblk, k) <= 10) ks = k;
    // Rows too long for 16 waves of 10 blocks: from 12 tokens (Q4_K 8), two halves of the blocks
    // per row tile added into zeroed y, at most 2 row tiles per wave (Q4_0 2560 x 10240 at 16 /
    // 32 / 48 / 63 tokens: 36 / 67 / 68 / 99 us against the vector kernel's 39 / 73 / 105 / ~137;
    // at 8 tokens 33 against 23, so fewer tokens keep the vector kernel; Q4_K's is slower: 46
    // us at 8 tokens).
    unsigned kz = 1;
    if (!ks && ZL_GEMV_MB_SPLIT && a.batch >= (QT == HIP_BRIDGE_Q4_K ? 8 : 12) && cdiv(nblk, 2 * 16) <= 10) {
        ks = 16;
        kz = 2;
    }
    if (!ks) return false;
    int nt = 1;
    for (int n : {4, 2})
        if (nt == 1 && cdiv(tiles, n) * ttiles * ks * kz >= ZL_GEMV_MB_WAVES && (kz == 1 || n <= ZL_GEMV_MB_SPLIT_NT)) nt = n;
    const dim3 grid((unsigned)cdiv(tiles, nt), (unsigned)ttiles, kz);
    if (kz > 1) launch_zero_f32(a.seg[0].y, (int64_t)a.batch * a.total_rows, s);
    auto go = [&](auto n_c) {
        constexpr int N = decltype(n_c)::value;
        if (ks == 4) k_gemv_mb<QT, N, 4><<<grid, 4 * kWave, 0, s>>>(a);
        else if (ks == 8) k_gemv_mb<QT, N, 8><<<grid, 8 * kWave, 0, s>>>(a);
        else k_gemv_mb<QT, N, 16><<<grid, 16 * kWave, 0, s>>>(a);
    };
    if (nt == 4) go(std::integral_constant<int, 4>{});
    else if (nt == 2) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 1>{});
    return true;
}
static bool launch_gemv_mb(int qtype, GemvArgs& a, hipStream_t s) {
    if (!ZL_GEMV_MB || a.batch < 2 || a.batch >= gemm_mfma_min_batch(qtype, a.total_rows, a.cols) ||
        a.cols % 32 != 0 || a.nseg != 1 ||
        !a.seg[0].w || !a.seg[0].y || !a.x || !aligned16(a.x))
        return false;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(a.seg[0].w);
    a.row_bytes = gemv_row_bytes(qtype, a.cols);
    switch (qtype) {
        case HIP_BRIDGE_Q4_0:
            return wa % 2 == 0 && launch_mb_t<HIP_BRIDGE_Q4_0>(a, s);
        case HIP_BRIDGE_Q8_0:
            return wa % 2 == 0 && launch_mb_t<HIP_BRIDGE_Q8_0>(a, s);
        case HIP_BRIDGE_Q4_K:
            return a.cols % 256 == 0 && wa % 2 == 0 && launch_mb_t<HIP_BRIDGE_Q4_K>(a, s);
        case HIP_BRIDGE_Q6_K:  // (below 8 tokens the vector kernel: 10240 x 2560 at 4, 24 against 38 us)
            return a.batch >= 8 && a.cols % 256 == 0 && wa % 2 == 0 && launch_mb_t<HIP_BRIDGE_Q6_K>(a, s);
        case HIP_BRIDGE_BF16:
            return wa % 16 == 0 && a.row_bytes % 16 == 0 && launch_mb_t<HIP_BRIDGE_BF16>(a, s);
        default:
            return false;
    }
}

static GemvArgs one_matrix(const void* w, const float* x, float* y, int rows, int cols, int batch) {
    GemvArgs a{};
    a.seg[0] = GemvSeg{(const unsigned char*)w, y, rows};
    a.nseg = 1;
    a.total_rows = rows;
    a.x = x;
    a.cols = cols;
    a.batch = batch;
    return a;
}

}  // namespace zl

using namespace zl;

extern "C" {

void hip_gemm(int qtype, const void* weights, const float* x, float* y, int batch_size, int rows,
              int cols, HipStream_t stream) {
    if (batch_size <= 0 || rows <= 0 || cols <= 0) return;
    if (batch_size >= gemm_mfma_min_batch(qtype, rows, cols) && weights && x) {
        const int64_t rb = gemv_row_bytes(qtype, cols);
        if (rb > 0 && launch_gemm_mfma(qtype, weights, rb, x, y, rows, cols, batch_size, stream_of(stream))) return;
    }
    GemvArgs a = one_matrix(weights, x, y, rows, cols, batch_size);
    if (launch_gemv_mb(qtype, a, stream_of(stream))) {
        check_launch();
        return;
    }
    launch_gemv<GV_PLAIN>(qtype, a, stream_of(stream));
}

void hip_gemv(int qtype, const void* weights, const float* x, float* y, int rows, int cols,
              HipStream_t stream) {
    hip_gemm(qtype, weights, x, y, 1, rows, cols, stream);
}

void hip_gemm_ex(int qtype, const void* weights, const void* up_weights, int x_dtype, const void* x,
                 int y_dtype, void* y, int batch_size, int rows, int cols, HipStream_t stream) {
    if (batch_size <= 0 || rows <= 0 || cols <= 0) return;
    if (!weights || !x || !y) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    if (!up_weights && x_dtype == HIP_BRIDGE_F32 && y_dtype == HIP_BRIDGE_F32) {
        hip_gemm(qtype, weights, (const float*)x, (float*)y, batch_size, rows, cols, stream);
        return;
    }
    const int64_t rb = gemv_row_bytes(qtype, cols);
    const int rc = rb > 0 ? launch_gemm_mfma_ex(qtype, weights, up_weights, rb, x_dtype, x, y_dtype, y, rows, cols,
                                                batch_size, stream_of(stream))
                          : HIP_BRIDGE_EUNSUPPORTED;
    if (rc != 0) set_error(rc);
}

void hip_gemv_q4_0(const void* weights, const float* x, float* y, int rows, int cols, HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_Q4_0, weights, x, y, 1, rows, cols, stream);
}
void hip_gemv_q8_0(const void* weights, const float* x, float* y, int rows, int cols, HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_Q8_0, weights, x, y, 1, rows, cols, stream);
}
void hip_gemv_q4_k(const void* weights, const float* x, float* y, int rows, int cols, HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_Q4_K, weights, x, y, 1, rows, cols, stream);
}
void hip_gemv_q6_k(const void* weights, const float* x, float* y, int rows, int cols, HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_Q6_K, weights, x, y, 1, rows, cols, stream);
}
void hip_gemv_f16(const void* weights, const float* x, float* y, int rows, int cols, HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_F16, weights, x, y, 1, rows, cols, stream);
}
void hip_gemv_bf16(const void* weights, const float* x, float* y, int rows, int cols, HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_BF16, weights, x, y, 1, rows, cols, stream);
}
void hip_gemv_f32(const float* weights, const float* x, float* y, int rows, int cols, HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_F32, weights, x, y, 1, rows, cols, stream);
}

void hip_gemm_q4_0(const void* weights, const float* x, float* y, int batch_size, int rows, int cols,
                   HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_Q4_0, weights, x, y, batch_size, rows, cols, stream);
}
void hip_gemm_q8_0(const void* weights, const float* x, float* y, int batch_size, int rows, int cols,
                   HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_Q8_0, weights, x, y, batch_size, rows, cols, stream);
}
void hip_gemm_f16(const void* weights, const float* x, float* y, int batch_size, int rows, int cols,
                  HipStream_t stream) {
    hip_gemm(HIP_BRIDGE_F16, weights, x, y, batch_size, rows, cols, stream);
}

void hip_gemv_geglu_q4_0(const void* gate_w, const void* up_w, const float* x, float* act_out, int rows,
                         int cols, HipStream_t stream) {
    if (rows <= 0 || cols <= 0) return;
    GemvArgs a = one_matrix(gate_w, x, act_out, rows, cols, 1);
    a.w_up = (const unsigned char*)up_w;
    launch_gemv<GV_GEGLU>(HIP_BRIDGE_Q4_0, a, stream_of(stream));
}

static bool qkv_args(GemvArgs& a, const void* q_w, const void* k_w, const void* v_w, const float* x,
                     float* q_out, float* k_out, float* v_out, int q_rows, int k_rows, int v_rows, int cols) {
    if (q_rows < 0 || k_rows < 0 || v_rows < 0) {
        set_error(HIP_BRIDGE_EINVAL);
        return false;
    }
    const int total = q_rows + k_rows + v_rows;
    if (total <= 0 || cols <= 0) return false;
    a = GemvArgs{};
    a.seg[0] = GemvSeg{(const unsigned char*)q_w, q_out, q_rows};
    a.seg[1] = GemvSeg{(const unsigned char*)k_w, k_out, k_rows};
    a.seg[2] = GemvSeg{(const unsigned char*)v_w, v_out, v_rows};
    a.nseg = 3;
    a.total_rows = total;
    a.x = x;
    a.cols = cols;
    a.batch = 1;
    return true;
}

static void set_pro(GemvArgs& a, const HipGemvPrologue* pro) {
    if (!pro) return;
    a.pro.mode = pro->mode;
    a.pro.r = pro->r;
    a.pro.r_w = pro->r_weight;
    a.pro.r_uo = pro->r_unit_offset;
    a.pro.scale = pro->scale;
    a.pro.x_out = pro->x_out;
    a.pro.w = pro->weight;
    a.pro.uo = pro->unit_offset;
    a.pro.eps = pro->eps;
    a.pro.xb_out = pro->xb_out;
}

void hip_gemv_qkv_q4_0(const void* q_w, const void* k_w, const void* v_w, const float* x, float* q_out,
                       float* k_out, float* v_out, int q_rows, int k_rows, int v_rows, int cols,
                       HipStream_t stream) {
    GemvArgs a;
    if (qkv_args(a, q_w, k_w, v_w, x, q_out, k_out, v_out, q_rows, k_rows, v_rows, cols))
        launch_gemv<GV_PLAIN>(HIP_BRIDGE_Q4_0, a, stream_of(stream));
}

void hip_gemv_pro(int qtype, const void* weights, const void* up_weights, const float* x, float* y, int rows,
                  int cols, const HipGemvPrologue* pro, HipStream_t stream) {
    if (rows <= 0 || cols <= 0) return;
    GemvArgs a = one_matrix(weights, x, y, rows, cols, 1);
    set_pro(a, pro);
    if (up_weights) {
        a.w_up = (const unsigned char*)up_weights;
        launch_gemv<GV_GEGLU>(qtype, a, stream_of(stream));
    } else {
        launch_gemv<GV_PLAIN>(qtype, a, stream_of(stream));
    }
}

void hip_gemv_qkv_pro(int qtype, const void* q_w, const void* k_w, const void* v_w, const float* x, float* q_out,
                      float* k_out, float* v_out, int q_rows, int k_rows, int v_rows, int cols,
                      const HipGemvPrologue* pro, HipStream_t stream) {
    GemvArgs a;
    if (!qkv_args(a, q_w, k_w, v_w, x, q_out, k_out, v_out, q_rows, k_rows, v_rows, cols)) return;
    set_pro(a, pro);
    launch_gemv<GV_PLAIN>(qtype, a, stream_of(stream));
}

}  // extern "C"
