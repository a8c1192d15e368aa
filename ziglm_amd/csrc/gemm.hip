// Prefill-sized GEMM on the matrix cores (gfx950 MFMA): Y[b][r] = sum_c W[r][c] * X[b][c] for
// Q4_0, Q8_0, F16, BF16 and F32 weights and f32 activations (replaces cuda_bridge.cu:1179-1445,
// k_gemm_q4_0 / k_gemm_q8_0 / k_gemm_f16, used by ziglm's batched prefill at
// cuda_model.zig:1264-1383), with ziglm's CPU arithmetic (math.zig:440-616): weights dequantised
// exactly, activations kept in f32, f32 sums.
//
// Exact operands on a bf16 matrix core. The MFMA multiplies bf16 operands exactly into f32
// accumulators, so every operand is written as a short sum of bf16 terms that is exact or
// nearly so:
//   x (f32) = h + m + l, h = bf16(x), m = bf16(x - h), l = bf16(x - h - m): the three terms
//     carry x's 24 significant bits (the remainder is below 2^-24 |x|);
//   Q4_0 / Q8_0 quants (integers -8..7 / -127..127) are exact in bf16; the block's f16 scale d
//     multiplies the block's f32 partial sum, sum_k q_k x_k, afterwards (the CPU's
//     (q * d) * x products are all exact-integer-times-f16 values, so applying d after the sum
//     changes only the f32 rounding);
//   BF16 weights are exact; F16 weights (11 significant bits) are hi + lo, both exact in bf16;
//   F32 weights are split like x.
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
// k as bf16 terms (rows padded to 80 bytes against bank conflicts) while registers hold block
// k + 1's raw X (f32) and W; each wave reads all of block k's MFMA operands into registers, one
// barrier frees the LDS, and block k's MFMAs then run from registers while the same waves
// convert block k + 1 into the LDS and issue block k + 2's global loads, so the matrix cores
// work during the conversion rather than after it. Loads take clamped (always valid) addresses
// and select zeros afterwards, so the loop body has no branches and the compiler interleaves
// the MFMAs with the conversion. Per 32-column block a 128 x 128 workgroup moves ~97 KB
// through the LDS (80 KB of operand reads), about as many cycles at 128 bytes per clock as its
// MFMAs take: LDS bandwidth bounds the kernel with the matrix cores.
#include "zl_common.h"
#include "zl_host.h"

namespace zl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmThreads = 256;
constexpr int kKB = 32;       // columns per K step (one Q4_0 / Q8_0 block)
constexpr int kLdsRow = 40;   // bf16 per LDS row: 32 + 8 padding (80 bytes)

template <int QT>
constexpr int w_terms() {
    return QT == HIP_BRIDGE_F16 ? 2 : QT == HIP_BRIDGE_F32 ? 3 : 1;
}
template <int QT>
constexpr bool w_scaled() {
    return QT == HIP_BRIDGE_Q4_0 || QT == HIP_BRIDGE_Q8_0;
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
    const float* x;
    float* y;
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

// 32-bit load from a 2-byte aligned address (block quants sit at offset 2 of 18 / 34-byte
// blocks): one global_load_dword, which gfx950 serves unaligned.
typedef uint32_t u32_a2 __attribute__((aligned(2)));
__device__ __forceinline__ uint32_t ld_u32_unaligned(const unsigned char* p) {
    return *reinterpret_cast<const u32_a2*>(p);
}

// `blk` is always a valid block address (the caller clamps it); `ok` false gives zeros, selected
// after the loads so that no load sits under a branch.
__device__ __forceinline__ u32x4 sel4(bool ok, u32x4 v) { return ok ? v : u32x4{0, 0, 0, 0}; }
template <int QT>
__device__ __forceinline__ void load_w(const unsigned char* blk, int h, bool ok, WRaw<QT>& r) {
    if constexpr (QT == HIP_BRIDGE_Q4_0) {
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

// Convert the thread's half row into bf16 terms: sw[t][row][...] (and the scale into sd[row]).
template <int QT>
__device__ __forceinline__ void store_w(const WRaw<QT>& r, int h, uint16_t* sw, int plane, int row, float* sd) {
    uint16_t* dst = sw + row * kLdsRow;
    if constexpr (QT == HIP_BRIDGE_Q4_0) {
        sd[row] = f16_bits_to_f32(r.d);  // both halves store the same value
        // byte j: low nibble = element j, high nibble = element j + 16 (value - 8)
        uint32_t lo[4], hi[4];
        const uint32_t q[2] = {r.q0, r.q1};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
#pragma unroll
            for (int b = 0; b < 4; b += 2) {
                const uint32_t b0 = (q[w] >> (8 * b)) & 0xffu, b1 = (q[w] >> (8 * b + 8)) & 0xffu;
                lo[w * 2 + b / 2] = pack_bf16x2((float)(int)(b0 & 15u) - 8.0f, (float)(int)(b1 & 15u) - 8.0f);
                hi[w * 2 + b / 2] = pack_bf16x2((float)(int)(b0 >> 4) - 8.0f, (float)(int)(b1 >> 4) - 8.0f);
            }
        }
        *reinterpret_cast<u32x4*>(dst + 8 * h) = u32x4{lo[0], lo[1], lo[2], lo[3]};
        *reinterpret_cast<u32x4*>(dst + 16 + 8 * h) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    } else if constexpr (QT == HIP_BRIDGE_Q8_0) {
        sd[row] = f16_bits_to_f32(r.d);  // both halves store the same value
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

// The (x term, w term) products accumulated, largest first: down to relative size 2^-16.
template <int NW>
struct TermPairs;
template <>
struct TermPairs<1> {
    static constexpr int n = 3;
    static constexpr int xt[3] = {0, 1, 2}, wt[3] = {0, 0, 0};
};
template <>
struct TermPairs<2> {
    static constexpr int n = 5;
    static constexpr int xt[5] = {0, 1, 0, 2, 1}, wt[5] = {0, 0, 1, 0, 1};
};
template <>
struct TermPairs<3> {
    static constexpr int n = 6;
    static constexpr int xt[6] = {0, 1, 0, 2, 1, 0}, wt[6] = {0, 0, 1, 0, 1, 2};
};

template <int QT, int WT, int WR>
__global__ __launch_bounds__(kGemmThreads, 2) void k_gemm_mfma(GemmArgs a) {
    constexpr int NW = w_terms<QT>();
    constexpr bool SCALED = w_scaled<QT>();
    constexpr int BT = 2 * 32 * WT;  // tokens per workgroup
    constexpr int BR = 2 * 32 * WR;  // rows per workgroup
    constexpr int XPLANE = BT * kLdsRow, WPLANE = BR * kLdsRow;
    __shared__ __attribute__((aligned(16))) uint16_t sx[3 * XPLANE];
    __shared__ __attribute__((aligned(16))) uint16_t sw[NW * WPLANE];
    __shared__ float sd[SCALED ? BR : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int r_base = blockIdx.x * BR, b_base = blockIdx.y * BT;
    const int nkb = a.cols / kKB;

    // X staging: chunk c = tid + 256 i (i < BT * 8 / 256) is token c / 8, columns 4 (c % 8) ...
    constexpr int XCH = BT * 8 / kGemmThreads;
    f32x4 xr[XCH];
    auto load_x = [&](int kb) {  // kb < nkb; tokens past the batch read the last token, then zeros
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + kGemmThreads * i, tok = b_base + c / 8;
            const f32x4 v = ldf4(a.x + (int64_t)min(tok, a.batch - 1) * a.cols + kb * kKB + 4 * (c % 8));
            xr[i] = tok < a.batch ? v : f32x4{0, 0, 0, 0};
        }
    };
    auto store_x = [&]() {
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int c = tid + kGemmThreads * i, tok = c / 8, k = 4 * (c % 8);
            uint32_t t0[3], t1[3];
            split3(xr[i].x, xr[i].y, t0);
            split3(xr[i].z, xr[i].w, t1);
#pragma unroll
            for (int u = 0; u < 3; ++u)
                *reinterpret_cast<u32x2*>(sx + u * XPLANE + tok * kLdsRow + k) = u32x2{t0[u], t1[u]};
        }
    };
    // W staging: half rows (BR rows x 2 halves over 256 threads: BR / 128 passes, or the
    // first 2 BR threads when BR < 128)
    constexpr int WPASS = BR * 2 >= kGemmThreads ? BR * 2 / kGemmThreads : 1;
    WRaw<QT> wr[WPASS];
    auto load_wt = [&](int kb) {
#pragma unroll
        for (int i = 0; i < WPASS; ++i) {
            const int hr = tid + kGemmThreads * i, row = hr >> 1, h = hr & 1;
            const int gr = r_base + row;
            const bool ok = hr < 2 * BR && gr < a.rows;
            const int64_t blk_bytes = QT == HIP_BRIDGE_Q4_0 ? 18 : QT == HIP_BRIDGE_Q8_0 ? 34 : QT == HIP_BRIDGE_F32 ? 128 : 64;
            load_w<QT>(a.w + (int64_t)min(gr, a.rows - 1) * a.row_bytes + (int64_t)kb * blk_bytes, h, ok, wr[i]);
        }
    };
    auto store_wt = [&]() {
#pragma unroll
        for (int i = 0; i < WPASS; ++i) {
            const int hr = tid + kGemmThreads * i;
            if (2 * BR >= kGemmThreads || hr < 2 * BR) store_w<QT>(wr[i], hr & 1, sw, WPLANE, hr >> 1, sd);
        }
    };

    const int wt0 = (wave >> 1) * 32 * WT;  // the wave's first token (within the workgroup)
    const int wr0 = (wave & 1) * 32 * WR;   // the wave's first row
    f32x16 acc[WT][WR];
    f32x16 part[WT][WR];
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WR; ++j) acc[i][j] = f32x16{};

    // Pipeline: LDS holds block kb while the raw registers hold block kb + 1. Each wave reads
    // all of block kb's MFMA operands (and scales) from LDS into registers, one barrier frees
    // the LDS, and then block kb's MFMAs run from registers while the same waves convert block
    // kb + 1 into the LDS (and issue block kb + 2's loads): the MFMAs overlap the conversion's
    // VALU and LDS work instead of following it.
    constexpr int NP = TermPairs<NW>::n;
    load_x(0);
    load_wt(0);
    store_x();
    store_wt();
    __syncthreads();
    load_x(min(1, nkb - 1));
    load_wt(min(1, nkb - 1));
    for (int kb = 0; kb < nkb; ++kb) {
        bf16x8 xa[2][WT][3], wb[2][WR][NW];
        float dv[WR];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {  // two K = 16 halves of the block
            const int ko = 16 * ks + 8 * (lane >> 5);
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int u = 0; u < 3; ++u)
                    xa[ks][i][u] = *reinterpret_cast<const bf16x8*>(sx + u * XPLANE + (wt0 + 32 * i + (lane & 31)) * kLdsRow + ko);
#pragma unroll
            for (int j = 0; j < WR; ++j)
#pragma unroll
                for (int u = 0; u < NW; ++u)
                    wb[ks][j][u] = *reinterpret_cast<const bf16x8*>(sw + u * WPLANE + (wr0 + 32 * j + (lane & 31)) * kLdsRow + ko);
        }
        if constexpr (SCALED) {
#pragma unroll
            for (int j = 0; j < WR; ++j) dv[j] = sd[wr0 + 32 * j + (lane & 31)];
        }
        __syncthreads();  // every wave holds block kb's operands: the LDS is free
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int j = 0; j < WR; ++j)
#pragma unroll
                    for (int p = 0; p < NP; ++p) {
                        const bf16x8 A = xa[ks][i][TermPairs<NW>::xt[p]], Bv = wb[ks][j][TermPairs<NW>::wt[p]];
                        if constexpr (SCALED) {
                            part[i][j] = (ks == 0 && p == 0)
                                             ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Bv, f32x16{}, 0, 0, 0)
                                             : __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Bv, part[i][j], 0, 0, 0);
                        } else {
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, Bv, acc[i][j], 0, 0, 0);
                        }
                    }
        // block kb + 1 into the LDS (after the last block: a copy nobody reads), block kb + 2's
        // loads in flight (past the end: the last block again, unused)
        store_x();
        store_wt();
        load_x(min(kb + 2, nkb - 1));
        load_wt(min(kb + 2, nkb - 1));
        if constexpr (SCALED) {
#pragma unroll
            for (int j = 0; j < WR; ++j)
#pragma unroll
                for (int i = 0; i < WT; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(dv[j], part[i][j][r], acc[i][j][r]);
        }
        __syncthreads();  // block kb + 1 is in the LDS
    }

    // Epilogue: lane (l, r) of tile (i, j) holds token 8 (r / 4) + 4 (l / 32) + r % 4 and row l % 32.
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WR; ++j) {
            const int row = r_base + wr0 + 32 * j + (lane & 31);
            if (row >= a.rows) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int tok = b_base + wt0 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (tok < a.batch) a.y[(int64_t)tok * a.rows + row] = acc[i][j][r];
            }
        }
}

// Workgroup tile: the largest of 128 x 128, 64 x 128 and 64 x 64 (tokens x rows) that still
// gives at least two workgroups per CU (bigger tiles convert each operand for more MFMAs;
// smaller ones fill the chip at small batches).
template <int QT>
static void launch_qt(const GemmArgs& a, hipStream_t s) {
    constexpr int64_t kFill = 512;
    auto wgs = [&](int bt, int br) { return cdiv(a.rows, br) * cdiv(a.batch, bt); };
    if (wgs(128, 128) >= kFill) {
        k_gemm_mfma<QT, 2, 2><<<dim3((unsigned)cdiv(a.rows, 128), (unsigned)cdiv(a.batch, 128)), kGemmThreads, 0, s>>>(a);
    } else if (wgs(64, 128) >= kFill) {
        k_gemm_mfma<QT, 1, 2><<<dim3((unsigned)cdiv(a.rows, 128), (unsigned)cdiv(a.batch, 64)), kGemmThreads, 0, s>>>(a);
    } else {
        k_gemm_mfma<QT, 1, 1><<<dim3((unsigned)cdiv(a.rows, 64), (unsigned)cdiv(a.batch, 64)), kGemmThreads, 0, s>>>(a);
    }
}

bool launch_gemm_mfma(int qtype, const void* w, int64_t row_bytes, const float* x, float* y, int rows, int cols,
                      int batch, hipStream_t s) {
    const bool types = qtype == HIP_BRIDGE_Q4_0 || qtype == HIP_BRIDGE_Q8_0 || qtype == HIP_BRIDGE_F16 ||
                       qtype == HIP_BRIDGE_BF16 || qtype == HIP_BRIDGE_F32;
    // dense rows must be 16-byte aligned for the 128-bit loads; block rows need 2 bytes
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    const bool dense = qtype == HIP_BRIDGE_F16 || qtype == HIP_BRIDGE_BF16 || qtype == HIP_BRIDGE_F32;
    const bool aligned = aligned16(x) && (dense ? (wa % 16 == 0 && row_bytes % 16 == 0) : (wa % 2 == 0));
    if (!types || cols % kKB != 0 || batch < kGemmMfmaMinBatch || !aligned || !y) return false;
    const GemmArgs a{(const unsigned char*)w, x, y, row_bytes, rows, cols, batch};
    switch (qtype) {
        case HIP_BRIDGE_Q4_0: launch_qt<HIP_BRIDGE_Q4_0>(a, s); break;
        case HIP_BRIDGE_Q8_0: launch_qt<HIP_BRIDGE_Q8_0>(a, s); break;
        case HIP_BRIDGE_F16: launch_qt<HIP_BRIDGE_F16>(a, s); break;
        case HIP_BRIDGE_BF16: launch_qt<HIP_BRIDGE_BF16>(a, s); break;
        default: launch_qt<HIP_BRIDGE_F32>(a, s); break;
    }
    check_launch();
    return true;
}

}  // namespace zl
