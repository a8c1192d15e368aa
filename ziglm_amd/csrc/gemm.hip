// Prefill-sized GEMM on the matrix cores (gfx950 MFMA): Y[b][r] = sum_c W[r][c] * X[b][c] for
// Q4_0, Q8_0, F16, BF16 and F32 weights and f32 or bf16 activations (replaces
// cuda_bridge.cu:1179-1445, k_gemm_q4_0 / k_gemm_q8_0 / k_gemm_f16, used by ziglm's batched
// prefill at cuda_model.zig:1264-1383), with ziglm's CPU arithmetic (math.zig:440-616): weights
// dequantised exactly, activations kept in full, f32 sums. Outputs are f32 or bf16, and the
// gate.up pair of a GeGLU FFN runs as one launch that writes gelu(gate) * up (the reference's
// two prefill GEMMs and k_geglu, cuda_model.zig:1372-1387, cuda_bridge.cu:2247-2269): the
// workgroup's W tile holds its output rows of both matrices, the up half's accumulators pass
// to the gate half's waves through LDS, and the gate and up outputs never reach HBM.
//
// Exact operands on a bf16 matrix core. The MFMA multiplies bf16 operands exactly into f32
// accumulators, so every operand is written as a short sum of bf16 terms that is exact or
// nearly so:
//   x (f32) = h + m + l, h = bf16(x), m = bf16(x - h), l = bf16(x - h - m): the three terms
//     carry x's 24 significant bits (the remainder is below 2^-24 |x|); bf16 activations are
//     one exact term (a third of the MFMAs and no split);
//   Q4_0 / Q8_0 quants (integers -8..7 / -127..127) are exact in bf16; the block's f16 scale d
//     multiplies the block's f32 partial sum, sum_k q_k x_k, afterwards (the CPU's
//     (q * d) * x products are all exact-integer-times-f16 values, so applying d after the sum
//     changes only the f32 rounding);
//   BF16 weights are exact; F16 weights (11 significant bits) are hi + lo, both exact in bf16;
//   F32 weights are split like x;
//   Q4_K (math.zig:440-496): a 32-column block is one sub-block j of a 256-column
//     super-block, value q * (d * sc_j) - dmin * m_j with q in 0..15 (exact in bf16): the
//     block's partial sum_k q_k x_k is scaled by A_j = d * sc_j and the min term
//     B_j * sum_k x_k subtracted, with the per-token sums of x formed while staging x (the
//     decode GEMV's decomposition);
//   Q6_K (math.zig:556-616): value d * sc * (u - 32) with an int8 scale per 16 columns;
//     u - 32 is exact in bf16 and d * sc (exact in f32) scales each K = 16 half's partial
//     sum.
// The products of the terms are accumulated down to relative weight 2^-16 (h*w_hi, m*w_hi,
// l*w_hi, and for F16 / F32 the cross terms of the same size); the dropped ones are below
// 2^-24 of a product, so a dot product lies within the f32 rounding of the sum, like the
// decode GEMV's.
//
// Tiling. A 256-thread workgroup owns 32*WT*2 tokens x 32*WR*2 rows; its 4 waves form a 2 x 2
// grid, each computing WT x WR tiles of 32 tokens x 32 rows with v_mfma_f32_32x32x16_bf16
// (tokens on the A side, so a lane's accumulators are one weight row: the block scale is one
// value per lane and tile, and stores of 32 lanes are 128 contiguous bytes of a token's output
// row). The K loop takes one 32-column block per step, software-pipelined: the LDS holds block
// k as bf16 terms (rows padded to 80 bytes against bank conflicts; a block scale sits in its
// row's padding) while registers hold block k + 1's raw X and W, and block k's MFMAs run while
// the same waves convert block k + 1 into the LDS and issue block k + 2's global loads, so the
// matrix cores work during the conversion rather than after it. Where two operand buffers fit
// two workgroups per CU (f32 or bf16 activations with one weight term: 80 KB) block k + 1 goes
// to the other buffer and a step takes one barrier; otherwise every wave first reads all of
// block k's operands into registers and a barrier frees the buffer. Activations load through a
// range-checked resource (tokens past the batch read zeros) and weights from clamped rows with
// zeros selected afterwards, so the loop body has no branches and the compiler interleaves the
// MFMAs with the conversion.
#include "zl_common.h"
#include "zl_host.h"

namespace zl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmThreads = 256;
constexpr int kKB = 32;       // columns per K step (one Q4_0 / Q8_0 block)
constexpr int kLdsRow = 40;   // bf16 per LDS row: 32 + 8 padding (80 bytes)

// Weight terms (bf16 planes) per type: Q4_0 / Q8_0 quants are exact in bf16 and their block
// scale multiplies each 32-column partial sum; BF16 weights are exact; F16 weights are two
// exact terms, F32 three. (Q4_0 products (u - 8) * d are also exact in two bf16 terms, which
// saves the per-block scale products at twice the MFMAs: measured slower, with f32
// activations 333 -> 438 us and with bf16 ones 191 -> 213 us for 10240 x 2560 x 2048.)
// Q6_K: its scale per 16-column half multiplies each K = 16 MFMA half's partial sum, the
// quants u - 32 one exact term. (sc * (u - 32) as two exact terms with one scale d per step
// instead: 5 term products, 10240 x 2560 x 2048 with f32 activations 555 against 453 us.)
template <int QT>
constexpr bool w_halves() {
    return QT == HIP_BRIDGE_Q6_K;
}
template <int QT>
constexpr int w_terms() {
    return QT == HIP_BRIDGE_F16 ? 2 : QT == HIP_BRIDGE_F32 ? 3 : 1;
}
template <int QT>
constexpr bool w_scaled() {
    return QT == HIP_BRIDGE_Q4_0 || QT == HIP_BRIDGE_Q8_0 || QT == HIP_BRIDGE_Q4_K || QT == HIP_BRIDGE_Q6_K;
}
// K-quant super-blocks: 8 K steps of 32 columns each
template <int QT>
constexpr bool k_quant() {
    return QT == HIP_BRIDGE_Q4_K || QT == HIP_BRIDGE_Q6_K;
}

// bf16 (RNE) of two floats and the f32 values of the result.
__device__ __forceinline__ uint32_t bf16_pair(float a, float b, float& ra, float& rb) {
    const uint32_t p = pack_bf16x2(a, b);
    ra = bf16_lo(p);
    rb = bf16_hi(p);
    return p;
}

// x0, x1 -> three packed bf16 pairs (h, m, l).
__device__ __forceinline__ void split3(float x0, float x1, uint32_t* t) {
    float a, b;
    t[0] = bf16_pair(x0, x1, a, b);
    x0 -= a;
    x1 -= b;
    t[1] = bf16_pair(x0, x1, a, b);
    t[2] = pack_bf16x2(x0 - a, x1 - b);
}
// x0, x1 -> two packed bf16 pairs (hi, lo).
__device__ __forceinline__ void split2(float x0, float x1, uint32_t* t) {
    float a, b;
    t[0] = bf16_pair(x0, x1, a, b);
    t[1] = pack_bf16x2(x0 - a, x1 - b);
}

struct GemmArgs {
    const unsigned char* w;
    const unsigned char* wu;  // GeGLU: the up matrix (same type and shape as w)
    const void* x;            // f32 or bf16 [batch][cols]
    void* y;                  // f32 or bf16 [batch][rows]
    int64_t row_bytes;
    int rows, cols, batch;
};

// Raw weight bytes of one 32-column block for half a row (the thread's half: h = 0 or 1).
template <int QT>
struct WRaw;
template <>
struct WRaw<HIP_BRIDGE_Q4_0> {  // d + bytes [8h, 8h + 8): elements 8h.. and 16 + 8h..
    uint32_t d, q0, q1;
};
template <>
struct WRaw<HIP_BRIDGE_Q8_0> {  // d + int8 [16h, 16h + 16)
    uint32_t d, q[4];
};
template <>
struct WRaw<HIP_BRIDGE_BF16> {
    u32x4 v[2];  // elements [16h, 16h + 16)
};
template <>
struct WRaw<HIP_BRIDGE_F16> {
    u32x4 v[2];
};
template <>
struct WRaw<HIP_BRIDGE_F32> {
    u32x4 v[4];
};
template <>
struct WRaw<HIP_BRIDGE_Q4_K> {  // {d, dmin}, scales[12], qs bytes [16h, 16h + 16) of sub-block j's span
    uint32_t dm, s[3], q[4], j;
};
template <>
struct WRaw<HIP_BRIDGE_Q6_K> {  // ql / qh bytes of the half's 16 columns, its int8 scale, d
    uint32_t ql[4], qh[4], sc, d, t;
};

// 32-bit load from a 2-byte aligned address (block quants sit at offset 2 of 18 / 34-byte
// blocks): one global_load_dword, which gfx950 serves unaligned.
typedef uint32_t u32_a2 __attribute__((aligned(2)));
__device__ __forceinline__ uint32_t ld_u32_unaligned(const unsigned char* p) {
    return *reinterpret_cast<const u32_a2*>(p);
}

// `blk` is always a valid block address (the caller clamps it); `ok` false gives zeros, selected
// after the loads so that no load sits under a branch. K-quants: `blk` is the super-block and
// `sub` the K step within it (0..7).
__device__ __forceinline__ u32x4 sel4(bool ok, u32x4 v) { return ok ? v : u32x4{0, 0, 0, 0}; }
template <int QT>
__device__ __forceinline__ void load_w(const unsigned char* blk, int sub, int h, bool ok, WRaw<QT>& r) {
    if constexpr (QT == HIP_BRIDGE_Q4_K) {
        // 144-byte super-block {f16 d, f16 dmin, scales[12], qs[128]} (types.zig:170-175);
        // sub-block j's 32 values are the low (j even) or high (j odd) nibbles of
        // qs[32 (j / 2) .. + 32)
        uint32_t v[8];
        v[0] = ld_u32_unaligned(blk);
#pragma unroll
        for (int i = 0; i < 3; ++i) v[1 + i] = ld_u32_unaligned(blk + 4 + 4 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 + i] = ld_u32_unaligned(blk + 16 + 32 * (sub >> 1) + 16 * h + 4 * i);
        r.dm = ok ? v[0] : 0u;
#pragma unroll
        for (int i = 0; i < 3; ++i) r.s[i] = ok ? v[1 + i] : 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = ok ? v[4 + i] : 0u;
        r.j = (uint32_t)sub;
    } else if constexpr (QT == HIP_BRIDGE_Q6_K) {
        // 210-byte super-block {ql[128], qh[64], int8 scales[16], f16 d} (types.zig:187-192).
        // K step sub = 4 n + t covers values [128 n + 32 t, + 32): value l of it takes the
        // low (t < 2) or high nibble of ql[64 n + 32 (t & 1) + l], bits 2t, 2t + 1 of
        // qh[32 n + l] and scale sc[8 n + l / 16 + 2 t] (quant.zig:357-385); the half h is
        // l in [16 h, 16 h + 16), one scale
        const int n = sub >> 2, t = sub & 3;
        uint32_t ql[4], qh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ql[i] = ld_u32_unaligned(blk + 64 * n + 32 * (t & 1) + 16 * h + 4 * i);
            qh[i] = ld_u32_unaligned(blk + 128 + 32 * n + 16 * h + 4 * i);
        }
        const uint32_t scw = *(const uint16_t*)(blk + 192 + 8 * n + 2 * t);  // scales 8n+2t, +1
        const uint32_t d = *(const uint16_t*)(blk + 208);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.ql[i] = ok ? ql[i] : 0u;
            r.qh[i] = ok ? qh[i] : 0u;
        }
        r.sc = ok ? (scw >> (8 * h)) & 0xffu : 0u;
        r.d = ok ? d : 0u;
        r.t = (uint32_t)t;
    } else if constexpr (QT == HIP_BRIDGE_Q4_0) {
        const uint32_t d = *(const uint16_t*)blk, q0 = ld_u32_unaligned(blk + 2 + 8 * h),
                       q1 = ld_u32_unaligned(blk + 6 + 8 * h);
        r.d = ok ? d : 0u;
        r.q0 = ok ? q0 : 0u;
        r.q1 = ok ? q1 : 0u;
    } else if constexpr (QT == HIP_BRIDGE_Q8_0) {
        const uint32_t d = *(const uint16_t*)blk;
        r.d = ok ? d : 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = ld_u32_unaligned(blk + 2 + 16 * h + 4 * i);
            r.q[i] = ok ? q : 0u;
        }
    } else if constexpr (QT == HIP_BRIDGE_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r.v[i] = sel4(ok, ld16(blk + 64 * h + 16 * i));
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) r.v[i] = sel4(ok, ld16(blk + 32 * h + 16 * i));
    }
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Convert the thread's half row into bf16 terms: sw[t][row][...]; a block scale goes into the
// padding of the row's first plane (bf16 slots 32, 33: kScaleSlot).
constexpr int kScaleSlot = 32;
constexpr int kMinSlot = 34;  // Q4_K: the block's min factor B_j = dmin * m_j (bf16 slots 34, 35)
template <int QT>
__device__ __forceinline__ void store_w(const WRaw<QT>& r, int h, uint16_t* sw, int plane, int row) {
    uint16_t* dst = sw + row * kLdsRow;
    if constexpr (QT == HIP_BRIDGE_Q4_K) {
        // 6-bit scale and min of sub-block j (quant.zig:285-290): j < 4: scales[j] & 63 and
        // scales[j + 4] & 63; else the low / high nibble of scales[j + 4] with the top two
        // bits of scales[j - 4] / scales[j] above them
        const uint32_t j = r.j, b = 8u * (j & 3u);
        const uint32_t s0 = (r.s[0] >> b) & 0xffu, s1 = (r.s[1] >> b) & 0xffu, s2 = (r.s[2] >> b) & 0xffu;
        const uint32_t sc = j < 4 ? (s0 & 63u) : ((s2 & 15u) | ((s0 >> 6) << 4));
        const uint32_t m = j < 4 ? (s1 & 63u) : ((s2 >> 4) | ((s1 >> 6) << 4));
        *reinterpret_cast<float*>(dst + kScaleSlot) = f16_bits_to_f32(r.dm & 0xffffu) * (float)sc;
        *reinterpret_cast<float*>(dst + kMinSlot) = f16_bits_to_f32(r.dm >> 16) * (float)m;
        const int sh = (int)(j & 1u) * 4;
        uint32_t p[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t v = (r.q[i] >> sh) & 0x0f0f0f0fu;
            p[2 * i] = pack_bf16x2((float)(v & 0xffu), (float)((v >> 8) & 0xffu));
            p[2 * i + 1] = pack_bf16x2((float)((v >> 16) & 0xffu), (float)(v >> 24));
        }
        *reinterpret_cast<u32x4*>(dst + 16 * h) = u32x4{p[0], p[1], p[2], p[3]};
        *reinterpret_cast<u32x4*>(dst + 16 * h + 8) = u32x4{p[4], p[5], p[6], p[7]};
    } else if constexpr (QT == HIP_BRIDGE_Q6_K) {
        // the half's scale d * sc (exact) in slot 32 + 2h; quants u - 32, exact in bf16
        *reinterpret_cast<float*>(dst + kScaleSlot + 2 * h) = f16_bits_to_f32(r.d) * (float)(int8_t)(uint8_t)r.sc;
        const int nsh = r.t < 2 ? 0 : 4, hsh = 2 * (int)r.t;
        uint32_t p[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t u = ((r.ql[i] >> (8 * e + nsh)) & 15u) | (((r.qh[i] >> (8 * e + hsh)) & 3u) << 4);
                v[e] = (float)((int)u - 32);
            }
            p[2 * i] = pack_bf16x2(v[0], v[1]);
            p[2 * i + 1] = pack_bf16x2(v[2], v[3]);
        }
        *reinterpret_cast<u32x4*>(dst + 16 * h) = u32x4{p[0], p[1], p[2], p[3]};
        *reinterpret_cast<u32x4*>(dst + 16 * h + 8) = u32x4{p[4], p[5], p[6], p[7]};
    } else if constexpr (QT == HIP_BRIDGE_Q4_0) {
        *reinterpret_cast<float*>(dst + kScaleSlot) = f16_bits_to_f32(r.d);  // both halves store it
        // byte j: low nibble = element j, high nibble = element j + 16 (value u - 8, exact)
        uint32_t lo[4], hi[4];
        const uint32_t q[2] = {r.q0, r.q1};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t lo4 = q[w] & 0x0f0f0f0fu, hi4 = (q[w] >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int b = 0; b < 4; b += 2) {
                lo[w * 2 + b / 2] = pack_bf16x2((float)((lo4 >> (8 * b)) & 0xffu) - 8.0f, (float)((lo4 >> (8 * b + 8)) & 0xffu) - 8.0f);
                hi[w * 2 + b / 2] = pack_bf16x2((float)((hi4 >> (8 * b)) & 0xffu) - 8.0f, (float)((hi4 >> (8 * b + 8)) & 0xffu) - 8.0f);
            }
        }
        *reinterpret_cast<u32x4*>(dst + 8 * h) = u32x4{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<u32x4*>(dst + 16 + 8 * h) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    } else if constexpr (QT == HIP_BRIDGE_Q8_0) {
        *reinterpret_cast<float*>(dst + kScaleSlot) = f16_bits_to_f32(r.d);  // both halves store it
        uint32_t p[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int32_t v = (int32_t)r.q[i];
            p[2 * i] = pack_bf16x2((float)(int8_t)(v & 0xff), (float)(int8_t)((v >> 8) & 0xff));
            p[2 * i + 1] = pack_bf16x2((float)(int8_t)((v >> 16) & 0xff), (float)(int8_t)((v >> 24) & 0xff));
        }
        *reinterpret_cast<u32x4*>(dst + 16 * h) = u32x4{p[0], p[1], p[2], p[3]};
        *reinterpret_cast<u32x4*>(dst + 16 * h + 8) = u32x4{p[4], p[5], p[6], p[7]};
    } else if constexpr (QT == HIP_BRIDGE_BF16) {
        *reinterpret_cast<u32x4*>(dst + 16 * h) = r.v[0];
        *reinterpret_cast<u32x4*>(dst + 16 * h + 8) = r.v[1];
    } else if constexpr (QT == HIP_BRIDGE_F16) {
        uint32_t t[2][8];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t w4[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t s[2];
                split2(f16_bits_to_f32(w4[j] & 0xffffu), f16_bits_to_f32(w4[j] >> 16), s);
                t[0][4 * i + j] = s[0];
                t[1][4 * i + j] = s[1];
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            uint16_t* d = sw + u * plane + row * kLdsRow + 16 * h;
            *reinterpret_cast<u32x4*>(d) = u32x4{t[u][0], t[u][1], t[u][2], t[u][3]};
            *reinterpret_cast<u32x4*>(d + 8) = u32x4{t[u][4], t[u][5], t[u][6], t[u][7]};
        }
    } else {  // F32: elements [16h, 16h + 16)
        uint32_t t[3][8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t s[3];
            split3(__uint_as_float(r.v[i].x), __uint_as_float(r.v[i].y), s);
            t[0][2 * i] = s[0], t[1][2 * i] = s[1], t[2][2 * i] = s[2];
            split3(__uint_as_float(r.v[i].z), __uint_as_float(r.v[i].w), s);
            t[0][2 * i + 1] = s[0], t[1][2 * i + 1] = s[1], t[2][2 * i + 1] = s[2];
        }
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            uint16_t* d = sw + u * plane + row * kLdsRow + 16 * h;
            *reinterpret_cast<u32x4*>(d) = u32x4{t[u][0], t[u][1], t[u][2], t[u][3]};
            *reinterpret_cast<u32x4*>(d + 8) = u32x4{t[u][4], t[u][5], t[u][6], t[u][7]};
        }
    }
}

// The (x term, w term) products accumulated, largest first: down to relative size 2^-16
// (x in XT terms: 3 for f32 activations, 1 for bf16 ones, which are exact).
template <int XT, int NW>
struct TermPairs;
template <>
struct TermPairs<3, 1> {
    static constexpr int n = 3;
    static constexpr int xt[3] = {0, 1, 2}, wt[3] = {0, 0, 0};
};
template <>
struct TermPairs<3, 2> {
    static constexpr int n = 5;
    static constexpr int xt[5] = {0, 1, 0, 2, 1}, wt[5] = {0, 0, 1, 0, 1};
};
template <>
struct TermPairs<3, 3> {
    static constexpr int n = 6;
    static constexpr int xt[6] = {0, 1, 0, 2, 1, 0}, wt[6] = {0, 0, 1, 0, 1, 2};
};
template <int NW>
struct TermPairs<1, NW> {
    static constexpr int n = NW;
    static constexpr int xt[3] = {0, 0, 0}, wt[3] = {0, 1, 2};
};

// Workgroup order. Workgroups are dispatched to the 8 XCDs in turn (linear id i on XCD i % 8),
// and each XCD has its own L2. With ZL_GEMM_XCD the linear id is renumbered so that XCD k
// takes the k-th eighth of the tiles in row-fastest order (the workgroups of one XCD then
// share their token tile's activations in its L2). Measured neutral (within 2% either way
// over the prefill products: the kernel is bound by its instruction issue, not by operand
// fetches), so off by default.
#ifndef ZL_GEMM_XCD
#define ZL_GEMM_XCD 0
#endif
// Two operand buffers with f32 activations too (there the block-partial and total accumulators
// leave too few registers and the loop spills a few).
#ifndef ZL_GEMM_DB_F32X
#define ZL_GEMM_DB_F32X 0
#endif
// Wave priority raised while a wave issues its MFMAs (s_setprio 1 over the block's MFMAs, 0
// for the conversion and the scale products): taken for three-plane activations at 64-token
// tiles, where three workgroups share a CU (10240 x 2560 weights, 2048 tokens: 498 -> 407 us);
// at 128-token tiles it slows the products (292 -> 363 us), and elsewhere it is neutral.
// ZL_GEMM_PRIO=1 forces it everywhere, -1 turns it off.
#ifndef ZL_GEMM_PRIO
#define ZL_GEMM_PRIO 0
#endif

// XK: activation form (X_F32: f32, split into three terms while staging; X_BF16: bf16, one
// term; X_TERMS: three bf16 planes split beforehand, staged as they are). GE: gate.up GeGLU
// pairs (the W tile's first
// half holds gate rows, its second half the same rows of the up matrix; out = gelu(g) * u).
// YB: bf16 output (else f32).
enum XKind { X_F32 = 0, X_BF16 = 1, X_TERMS = 2 };

// Workgroups per CU the launch asks registers for: three (170 VGPRs a lane) for bf16
// activations when the LDS holds three, so a third wave per SIMD has MFMAs ready while the
// others read operands or wait at a barrier; two otherwise (the three-term activations' loop
// needs more registers: held to 170 it spills).
template <int QT, int XK, int WT, int WR>
constexpr int gemm_wgs_per_cu() {
    constexpr int bt = 64 * WT, br = 64 * WR;
    constexpr int oper = (bt + w_terms<QT>() * br) * kLdsRow * 2;  // bf16 activations: one term
    // (Q4_K's min term needs the registers: held to 170 its loop spills)
    return XK == X_BF16 && QT != HIP_BRIDGE_Q4_K && 2 * oper * 3 <= 160 * 1024 ? 3 : 2;
}

template <int QT, int XK, int WT, int WR, bool GE, bool YB>
__global__ __launch_bounds__(kGemmThreads, (gemm_wgs_per_cu<QT, XK, WT, WR>())) void k_gemm_mfma(GemmArgs a) {
    constexpr int XT = XK == X_BF16 ? 1 : 3;  // activation terms
    constexpr int NW = w_terms<QT>();
    constexpr bool SCALED = w_scaled<QT>();
    constexpr int BT = 2 * 32 * WT;  // tokens per workgroup
    constexpr int BR = 2 * 32 * WR;  // W rows per workgroup (GE: BR / 2 gate + BR / 2 up rows)
    constexpr int OR = GE ? BR / 2 : BR;  // output rows per workgroup
    constexpr int XPLANE = BT * kLdsRow, WPLANE = BR * kLdsRow;
    constexpr int OPER_BYTES = (XT * XPLANE + NW * WPLANE) * 2;
    // Two operand buffers (block kb read while block kb + 1 is written: one barrier per step)
    // when they fit two workgroups per CU in the 160 KB of LDS; else one (also for Q4_K with
    // three activation planes, whose two-buffer loop needs 284 registers: one wave per SIMD).
    constexpr bool DB = 2 * OPER_BYTES <= 80 * 1024 && (XK != X_F32 || ZL_GEMM_DB_F32X) &&
                        !(QT == HIP_BRIDGE_Q4_K && XK == X_TERMS);
    constexpr int NBUF = DB ? 2 : 1;
    constexpr int XCH_BYTES = GE ? 2 * WT * WR * 16 * kWave * 4 : 0;  // up accumulators, two waves
    // Q4_K: per-token sums of each K step's activations (f32 or bf16 x: one sum; pre-split
    // planes: one per plane, added in plane order), in two slots by step parity: step kb + 1's
    // sums are written while step kb's are read. (Summing f32 x's three terms instead, so that
    // both f32 forms agree bit for bit, cost 3 reductions a step: 10240 x 2560 x 2048, 531 us.)
    constexpr bool MIN = QT == HIP_BRIDGE_Q4_K;
    constexpr int XSP = XK == X_TERMS ? 3 : 1;  // sum planes
    constexpr int XS_FLOATS = MIN ? 2 * XSP * BT : 0;
    constexpr int MAIN_BYTES = NBUF * OPER_BYTES > XCH_BYTES ? NBUF * OPER_BYTES : XCH_BYTES;
    __shared__ __attribute__((aligned(16))) unsigned char s_raw[MAIN_BYTES + XS_FLOATS * 4];
    auto sx_of = [&](int b) { return reinterpret_cast<uint16_t*>(s_raw + b * OPER_BYTES); };
    auto sw_of = [&](int b) { return reinterpret_cast<uint16_t*>(s_raw + b * OPER_BYTES) + XT * XPLANE; };
    float* const s_xs = reinterpret_cast<float*>(s_raw + MAIN_BYTES);  // [slot][plane][token]

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    int tile = blockIdx.x;
    const int gx = (a.rows + OR - 1) / OR, nwg = (int)gridDim.x;
    if (ZL_GEMM_XCD && nwg % 8 == 0) tile = (tile % 8) * (nwg / 8) + tile / 8;
    const int r_base = (tile % gx) * OR, b_base = (tile / gx) * BT;
    // K steps [kbb, kbe): all of them, or with a split launch (gridDim.y = 2, f32 output,
    // added into zeroed y) one half per workgroup row
    const int nkb_all = a.cols / kKB;
    const int kbb = (int)((int64_t)nkb_all * blockIdx.y / gridDim.y);
    const int kbe = (int)((int64_t)nkb_all * (blockIdx.y + 1) / gridDim.y);

    // X staging. f32 x: chunk c = tid + 256 i is token c / 8, columns 4 (c % 8) .. (four
    // floats); bf16 x: token c / 4, columns 8 (c % 4) .. (eight bf16); term planes: chunk c of
    // plane c / (4 BT), as bf16 x within the plane. Loads through range-checked resources over
    // the workgroup's tokens: tokens past the batch read zeros.
    constexpr int XE = XK == X_F32 ? 4 : 8;          // elements per 16-byte chunk
    constexpr int XCPT = kKB / XE;                  // chunks per token per block (per plane)
    constexpr int XPL = XK == X_TERMS ? 3 : 1;      // planes loaded
    constexpr int XCH = XPL * BT * XCPT / kGemmThreads;
    const int xes = XK == X_F32 ? 4 : 2;
    const int64_t tok_left = (int64_t)a.batch - b_base;
    const int64_t xbytes = (tok_left < BT ? tok_left : BT) * (int64_t)a.cols * xes;
    const uint32_t xrange = (uint32_t)(xbytes < 0xffffffffLL ? xbytes : 0xffffffffLL);
    const int64_t plane_bytes = (int64_t)a.batch * a.cols * xes;
    __amdgpu_buffer_rsrc_t rsx[XPL];
#pragma unroll
    for (int u = 0; u < XPL; ++u)
        rsx[u] = buf_rsrc((const unsigned char*)a.x + u * plane_bytes + (int64_t)b_base * a.cols * xes, xrange);
    u32x4 xr[XCH];
    // A plane is a whole number of 256-chunk passes, so pass i's plane is a constant of the
    // unrolled loop: the resource it selects stays in scalar registers (a plane index
    // computed from tid would make each load a loop over the lanes' distinct resources).
    static_assert((BT * XCPT) % kGemmThreads == 0, "X plane not a whole number of passes");
    auto load_x = [&](int kb) {
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            constexpr int PC = BT * XCPT;  // chunks per plane
            const int pl = kGemmThreads * i / PC, cc = tid + kGemmThreads * i % PC, tok = cc / XCPT;
            const uint32_t off = (uint32_t)(((int64_t)tok * a.cols + kb * kKB + XE * (cc % XCPT)) * xes);
            xr[i] = bldp<POL_DEFAULT>(rsx[pl], off);
        }
    };
    auto store_x = [&](int buf, int slot) {
        uint16_t* const sx = sx_of(buf);
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            constexpr int PC = BT * XCPT;
            const int pl = kGemmThreads * i / PC, cc = tid + kGemmThreads * i % PC;
            const int tok = cc / XCPT, k = XE * (cc % XCPT);
            // (MIN) the token's sum over the step's 32 columns of one term: pairs, then the
            // XCPT consecutive lanes holding its chunks (8 of 4 f32 or 4 of 8 bf16: the same
            // tree over the 32 values)
            auto put_sum = [&](float cs, int plane) {
                cs = group_sum<XCPT>(cs);
                if (cc % XCPT == 0) s_xs[(slot * XSP + plane) * BT + tok] = cs;
            };
            if constexpr (XK == X_F32) {
                uint32_t t0[3], t1[3];
                split3(__uint_as_float(xr[i].x), __uint_as_float(xr[i].y), t0);
                split3(__uint_as_float(xr[i].z), __uint_as_float(xr[i].w), t1);
#pragma unroll
                for (int u = 0; u < 3; ++u)
                    *reinterpret_cast<u32x2*>(sx + u * XPLANE + tok * kLdsRow + k) = u32x2{t0[u], t1[u]};
                if constexpr (MIN)
                    put_sum((__uint_as_float(xr[i].x) + __uint_as_float(xr[i].y)) +
                                (__uint_as_float(xr[i].z) + __uint_as_float(xr[i].w)),
                            0);
            } else {
                *reinterpret_cast<u32x4*>(sx + pl * XPLANE + tok * kLdsRow + k) = xr[i];
                if constexpr (MIN)
                    put_sum(((bf16_lo(xr[i].x) + bf16_hi(xr[i].x)) + (bf16_lo(xr[i].y) + bf16_hi(xr[i].y))) +
                                ((bf16_lo(xr[i].z) + bf16_hi(xr[i].z)) + (bf16_lo(xr[i].w) + bf16_hi(xr[i].w))),
                            pl);
            }
        }
    };
    // W staging: half rows (BR rows x 2 halves over 256 threads: BR / 128 passes, or the
    // first 2 BR threads when BR < 128). GE: tile rows [0, OR) are gate rows, [OR, BR) the
    // same rows of the up matrix.
    constexpr int WPASS = BR * 2 >= kGemmThreads ? BR * 2 / kGemmThreads : 1;
    // bytes per K step (K-quants: per super-block of 8 steps)
    constexpr int64_t blk_bytes = QT == HIP_BRIDGE_Q4_0 ? 18 : QT == HIP_BRIDGE_Q8_0 ? 34 : QT == HIP_BRIDGE_F32 ? 128
                                  : QT == HIP_BRIDGE_Q4_K ? 144 : QT == HIP_BRIDGE_Q6_K ? 210 : 64;
    WRaw<QT> wr[WPASS];
    auto load_wt = [&](int kb) {
        const int64_t boff = k_quant<QT>() ? (int64_t)(kb >> 3) * blk_bytes : (int64_t)kb * blk_bytes;
#pragma unroll
        for (int i = 0; i < WPASS; ++i) {
            const int hr = tid + kGemmThreads * i, row = hr >> 1, h = hr & 1;
            const bool up = GE && row >= OR;
            const int gr = r_base + (up ? row - OR : row);
            const bool ok = hr < 2 * BR && gr < a.rows;
            const unsigned char* wm = up ? a.wu : a.w;
            load_w<QT>(wm + (int64_t)min(gr, a.rows - 1) * a.row_bytes + boff, kb & 7, h, ok, wr[i]);
        }
    };
    auto store_wt = [&](int buf) {
        uint16_t* const swb = sw_of(buf);
#pragma unroll
        for (int i = 0; i < WPASS; ++i) {
            const int hr = tid + kGemmThreads * i;
            if (2 * BR >= kGemmThreads || hr < 2 * BR) store_w<QT>(wr[i], hr & 1, swb, WPLANE, hr >> 1);
        }
    };

    const int wt0 = (wave >> 1) * 32 * WT;  // the wave's first token (within the workgroup)
    const int wr0 = (wave & 1) * 32 * WR;   // the wave's first W row (GE: wave & 1 = up)
    f32x16 acc[WT][WR];
    f32x16 part[WT][WR];
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WR; ++j) acc[i][j] = f32x16{};

    using TP = TermPairs<XT, NW>;
    constexpr int NP = TP::n;
    constexpr bool PRIO = ZL_GEMM_PRIO > 0 || (ZL_GEMM_PRIO == 0 && XK == X_TERMS && WT == 1);
    // One K step: block kb's operands from LDS buffer `buf` into registers, its MFMAs (into the
    // block partial when SCALED), then `convert` (block kb + 1 into the LDS and the loads of
    // kb + 2), then the block scale products.
    auto step = [&](int buf, int slot, bool single, auto convert) {
        const uint16_t* const sx = sx_of(buf);
        const uint16_t* const sw = sw_of(buf);
        // with one buffer every wave holds all of block kb's operands before the barrier;
        // with two, each K = 16 half's operands are read just before its MFMAs (half the
        // registers)
        constexpr int KH = DB ? 1 : 2;
        constexpr bool HALVES = w_halves<QT>();
        bf16x8 xa[KH][WT][XT], wb[KH][WR][NW];
        float dv[WR], bv[MIN ? WR : 1], dv1[HALVES ? WR : 1];
        auto read_ops = [&](int ks, int slot) {
            const int ko = 16 * ks + 8 * (lane >> 5);
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int u = 0; u < XT; ++u)
                    xa[slot][i][u] = *reinterpret_cast<const bf16x8*>(sx + u * XPLANE + (wt0 + 32 * i + (lane & 31)) * kLdsRow + ko);
#pragma unroll
            for (int j = 0; j < WR; ++j)
#pragma unroll
                for (int u = 0; u < NW; ++u)
                    wb[slot][j][u] = *reinterpret_cast<const bf16x8*>(sw + u * WPLANE + (wr0 + 32 * j + (lane & 31)) * kLdsRow + ko);
        };
        auto mfmas = [&](int ks, int slot) {
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int j = 0; j < WR; ++j)
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        const bf16x8 A = xa[slot][i][TP::xt[p]], Bv = wb[slot][j][TP::wt[p]];
                        if constexpr (SCALED) {
                            part[i][j] = ((ks == 0 || HALVES) && p == 0)
                                             ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Bv, f32x16{}, 0, 0, 0)
                                             : __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Bv, part[i][j], 0, 0, 0);
                        } else {
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Bv, acc[i][j], 0, 0, 0);
                        }
                    }
        };
        if constexpr (SCALED) {
#pragma unroll
            for (int j = 0; j < WR; ++j) {
                dv[j] = *reinterpret_cast<const float*>(sw + (wr0 + 32 * j + (lane & 31)) * kLdsRow + kScaleSlot);
                if constexpr (MIN)
                    bv[j] = *reinterpret_cast<const float*>(sw + (wr0 + 32 * j + (lane & 31)) * kLdsRow + kMinSlot);
                if constexpr (HALVES)
                    dv1[j] = *reinterpret_cast<const float*>(sw + (wr0 + 32 * j + (lane & 31)) * kLdsRow + kScaleSlot + 2);
            }
        }
        // HALVES: the first half's partial sums scaled into acc before the second half's MFMAs
        auto scale_first_half = [&]() {
            if constexpr (HALVES) {
#pragma unroll
                for (int j = 0; j < WR; ++j)
#pragma unroll
                    for (int i = 0; i < WT; ++i)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(dv[j], part[i][j][r], acc[i][j][r]);
            }
        };
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
        if constexpr (DB) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                read_ops(ks, 0);
                mfmas(ks, 0);
                if (ks == 0) scale_first_half();
            }
        } else {
            read_ops(0, 0);
            read_ops(1, 1);
            if (single) __syncthreads();
            mfmas(0, 0);
            scale_first_half();
            mfmas(1, 1);
        }
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
        convert();
        if constexpr (MIN) {
            // acc += A_j * part - B_j * (sum of the token's x over the step: its terms' sums
            // added in order); lane (l, r) of tile i holds token 32 i + 8 (r / 4) + 4 (l / 32) +
            // r % 4: four runs of four
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int t0 = wt0 + 32 * i + 8 * q + 4 * (lane >> 5);
                    f32x4 v = *reinterpret_cast<const f32x4*>(s_xs + slot * XSP * BT + t0);
#pragma unroll
                    for (int u = 1; u < XSP; ++u) {
                        const f32x4 w = *reinterpret_cast<const f32x4*>(s_xs + (slot * XSP + u) * BT + t0);
                        v.x += w.x, v.y += w.y, v.z += w.z, v.w += w.w;
                    }
                    const float xs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int j = 0; j < WR; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int r = 4 * q + e;
                            acc[i][j][r] = fmaf(dv[j], part[i][j][r], fmaf(-bv[j], xs[e], acc[i][j][r]));
                        }
                }
        } else if constexpr (SCALED) {
#pragma unroll
            for (int j = 0; j < WR; ++j)
#pragma unroll
                for (int i = 0; i < WT; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(HALVES ? dv1[j] : dv[j], part[i][j][r], acc[i][j][r]);
        }
    };

    // Pipeline. The raw registers hold block kb + 1 while the MFMAs of block kb run; they are
    // converted into the LDS (the other buffer with DB, else the same one once every wave has
    // read block kb's operands) and block kb + 2's loads are issued, so the matrix cores work
    // during the conversion rather than after it. Past the end: the last block again, unused.
    load_x(kbb);
    load_wt(kbb);
    store_x(0, kbb & 1);
    store_wt(0);
    __syncthreads();
    load_x(min(kbb + 1, kbe - 1));
    load_wt(min(kbb + 1, kbe - 1));
    for (int it = 0; it < kbe - kbb; ++it) {
        const int kb = kbb + it;
        const int cur = DB ? (it & 1) : 0, nxt = DB ? (cur ^ 1) : 0;
        step(cur, kb & 1, !DB, [&]() {
            store_x(nxt, (kb + 1) & 1);
            store_wt(nxt);
            load_x(min(kb + 2, kbe - 1));
            load_wt(min(kb + 2, kbe - 1));
        });
        __syncthreads();  // block kb + 1 is in the LDS (DB: and block kb's buffer is free)
    }

    // Epilogue: lane (l, r) of tile (i, j) holds token 8 (r / 4) + 4 (l / 32) + r % 4 and row
    // l % 32. GE: the up waves pass their accumulators through the (now free) LDS to the gate
    // waves of the same tokens, which write gelu(g) * u.
    if constexpr (GE) {
        float* const xch = reinterpret_cast<float*>(s_raw) + (wave >> 1) * (WT * WR * 16 * kWave);
        if (wave & 1) {
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int j = 0; j < WR; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) xch[((i * WR + j) * 16 + r) * kWave + lane] = acc[i][j][r];
        }
        __syncthreads();
        if (wave & 1) return;
#pragma unroll
        for (int i = 0; i < WT; ++i)
#pragma unroll
            for (int j = 0; j < WR; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    acc[i][j][r] = gelu_fast(acc[i][j][r]) * xch[((i * WR + j) * 16 + r) * kWave + lane];
    }
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WR; ++j) {
            const int row = r_base + (GE ? 0 : wr0) + 32 * j + (lane & 31);
            if (row >= a.rows) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tok = b_base + wt0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (tok < a.batch) {
                    if constexpr (YB)
                        ((uint16_t*)a.y)[(int64_t)tok * a.rows + row] = (uint16_t)(pack_bf16x2(acc[i][j][r], 0.0f) & 0xffffu);
                    else if (gridDim.y > 1)  // two K halves into zeroed y: 0 + a + b in either order
                        unsafeAtomicAdd((float*)a.y + (int64_t)tok * a.rows + row, acc[i][j][r]);
                    else
                        ((float*)a.y)[(int64_t)tok * a.rows + row] = acc[i][j][r];
                }
            }
        }
}

// Workgroup tile: the largest of 128 x 128, 64 x 128 and 64 x 64 (tokens x W rows) that still
// gives at least two workgroups per CU (bigger tiles convert each operand for more MFMAs;
// smaller ones fill the chip at small batches).
// Split K (ZL_GEMM_SPLITK, zl_host.h: two halves of the K steps per output tile, summed into
// zeroed y by float atomic adds; with exactly two addends the sum does not depend on their
// order, so results stay bit-reproducible) for deep products with f32 output that give fewer
// than two rounds of workgroups: 2560 x 10240 x 2048, 640 -> 1280 workgroups: Q4_0 435 -> 401
// us, Q4_K 520 -> 479, Q6_K 634 -> 559; at 128 tokens Q4_0 250 -> 129 us.
__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) y[i] = 0.0f;
}
void launch_zero_f32(float* y, int64_t n, hipStream_t s) {
    k_zero_f32<<<(unsigned)std::min<int64_t>(cdiv(n, 256), 8192), 256, 0, s>>>(y, n);
}
template <int QT, int XK, bool GE, bool YB>
static void launch_qt(const GemmArgs& a, hipStream_t s) {
    constexpr int64_t kFill = 512;
    auto wgs = [&](int bt, int br) { return cdiv(a.rows, GE ? br / 2 : br) * cdiv(a.batch, bt); };
    const int64_t n = wgs(128, 128) >= kFill ? wgs(128, 128) : wgs(64, 128) >= kFill ? wgs(64, 128) : wgs(64, 64);
    // Deep products with f32 output and fewer than two rounds of workgroups: two K halves per
    // tile, added into zeroed y
    unsigned ky = 1;
    if constexpr (!GE && !YB) {
        if (ZL_GEMM_SPLITK && n < 2 * kFill && a.cols >= ZL_GEMM_SPLITK_MIN_COLS) {
            ky = 2;
            launch_zero_f32((float*)a.y, (int64_t)a.batch * a.rows, s);
        }
    }
    const dim3 grid((unsigned)n, ky);
    if (wgs(128, 128) >= kFill) {
        k_gemm_mfma<QT, XK, 2, 2, GE, YB><<<grid, kGemmThreads, 0, s>>>(a);
    } else if (wgs(64, 128) >= kFill) {
        k_gemm_mfma<QT, XK, 1, 2, GE, YB><<<grid, kGemmThreads, 0, s>>>(a);
    } else {
        k_gemm_mfma<QT, XK, 1, 1, GE, YB><<<grid, kGemmThreads, 0, s>>>(a);
    }
}

template <int QT, int XK>
static void launch_qx(const GemmArgs& a, bool ge, bool y_bf16, hipStream_t s) {
    if (ge) y_bf16 ? launch_qt<QT, XK, true, true>(a, s) : launch_qt<QT, XK, true, false>(a, s);
    else y_bf16 ? launch_qt<QT, XK, false, true>(a, s) : launch_qt<QT, XK, false, false>(a, s);
}
template <int QT>
static void launch_q(const GemmArgs& a, int xk, bool ge, bool y_bf16, hipStream_t s) {
    if (xk == X_F32) launch_qx<QT, X_F32>(a, ge, y_bf16, s);
    else if (xk == X_BF16) launch_qx<QT, X_BF16>(a, ge, y_bf16, s);
    else launch_qx<QT, X_TERMS>(a, ge, y_bf16, s);
}

// 0 = launched; otherwise why not (the caller decides between a fallback and an error).
int launch_gemm_mfma_ex(int qtype, const void* w, const void* wu, int64_t row_bytes, int x_dtype, const void* x,
                        int y_dtype, void* y, int rows, int cols, int batch, hipStream_t s) {
    const bool kq = qtype == HIP_BRIDGE_Q4_K || qtype == HIP_BRIDGE_Q6_K;
    const bool types = qtype == HIP_BRIDGE_Q4_0 || qtype == HIP_BRIDGE_Q8_0 || qtype == HIP_BRIDGE_F16 ||
                       qtype == HIP_BRIDGE_BF16 || qtype == HIP_BRIDGE_F32 || kq;
    if (!types || (x_dtype != HIP_BRIDGE_F32 && x_dtype != HIP_BRIDGE_BF16 && x_dtype != HIP_BRIDGE_F32_TERMS) ||
        (y_dtype != HIP_BRIDGE_F32 && y_dtype != HIP_BRIDGE_BF16))
        return HIP_BRIDGE_EUNSUPPORTED;
    // dense rows must be 16-byte aligned for the 128-bit loads; block rows need 2 bytes
    const bool dense = qtype == HIP_BRIDGE_F16 || qtype == HIP_BRIDGE_BF16 || qtype == HIP_BRIDGE_F32;
    auto w_ok = [&](const void* p) {
        const uintptr_t wa = reinterpret_cast<uintptr_t>(p);
        return dense ? (wa % 16 == 0 && row_bytes % 16 == 0) : (wa % 2 == 0);
    };
    if (cols % (kq ? 256 : kKB) != 0 || !aligned16(x) || !w_ok(w) || (wu && !w_ok(wu))) return HIP_BRIDGE_EUNSUPPORTED;
    // 32-bit byte offsets within a token tile's activations (per plane)
    if ((int64_t)128 * cols * (x_dtype == HIP_BRIDGE_F32 ? 4 : 2) > 0xffffffffLL) return HIP_BRIDGE_EUNSUPPORTED;
    const GemmArgs a{(const unsigned char*)w, (const unsigned char*)wu, x, y, row_bytes, rows, cols, batch};
    const int xk = x_dtype == HIP_BRIDGE_BF16 ? X_BF16 : x_dtype == HIP_BRIDGE_F32_TERMS ? X_TERMS : X_F32;
    const bool ge = wu != nullptr, yb = y_dtype == HIP_BRIDGE_BF16;
    switch (qtype) {
        case HIP_BRIDGE_Q4_0: launch_q<HIP_BRIDGE_Q4_0>(a, xk, ge, yb, s); break;
        case HIP_BRIDGE_Q8_0: launch_q<HIP_BRIDGE_Q8_0>(a, xk, ge, yb, s); break;
        case HIP_BRIDGE_F16: launch_q<HIP_BRIDGE_F16>(a, xk, ge, yb, s); break;
        case HIP_BRIDGE_BF16: launch_q<HIP_BRIDGE_BF16>(a, xk, ge, yb, s); break;
        case HIP_BRIDGE_Q4_K: launch_q<HIP_BRIDGE_Q4_K>(a, xk, ge, yb, s); break;
        case HIP_BRIDGE_Q6_K: launch_q<HIP_BRIDGE_Q6_K>(a, xk, ge, yb, s); break;
        default: launch_q<HIP_BRIDGE_F32>(a, xk, ge, yb, s); break;
    }
    check_launch();
    return 0;
}

// x (f32) -> three bf16 planes h, m, l (h = bf16(x), m = bf16(x - h), l = bf16(x - h - m)):
// the activation form the K loop stages without converting. Four elements per thread.
__global__ __launch_bounds__(256) void k_split_terms(const float* __restrict__ x, uint16_t* __restrict__ planes,
                                                     int64_t n) {
    const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;  // n % 4 == 0
    if (i4 >= n) return;
    const u32x4 v = lds16(x + i4);
    uint32_t t0[3], t1[3];
    split3(__uint_as_float(v.x), __uint_as_float(v.y), t0);
    split3(__uint_as_float(v.z), __uint_as_float(v.w), t1);
#pragma unroll
    for (int u = 0; u < 3; ++u) *reinterpret_cast<u32x2*>(planes + u * n + i4) = u32x2{t0[u], t1[u]};
}

bool launch_gemm_mfma(int qtype, const void* w, int64_t row_bytes, const float* x, float* y, int rows, int cols,
                      int batch, hipStream_t s) {
    if (batch < gemm_mfma_min_batch(qtype, rows, cols) || !y) return false;
    return launch_gemm_mfma_ex(qtype, w, nullptr, row_bytes, HIP_BRIDGE_F32, x, HIP_BRIDGE_F32, y, rows, cols, batch,
                               s) == 0;
}

}  // namespace zl

using namespace zl;

extern "C" void hip_split_terms(const float* x, void* planes, int64_t n, HipStream_t stream) {
    if (n <= 0) return;
    if (!x || !planes) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    if (!aligned16(x) || (reinterpret_cast<uintptr_t>(planes) & 7u) || n % 4) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    k_split_terms<<<(unsigned)cdiv(n, 1024), 256, 0, stream_of(stream)>>>(x, (uint16_t*)planes, n);
    check_launch();
}
