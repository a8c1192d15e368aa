// Embedding-row gather + dequant + scale (replaces cuda_bridge.cu:1559-1940).
//
// Arithmetic is ziglm's CPU order (quant.zig:73-79, 119-130, 357-385, 413-512 and
// model.zig:494-503): out = fl(fl(f32(q) * d) * scale). For Q8_0/Q4_0 q*d is exact, so every
// output is one IEEE rounding and the result is bit-exact; Q6_K keeps the CPU's
// ((d * scale_j) * q) * scale order and Q4_K its (q * (d * sc_j) - dmin * m_j) * scale.
//
// Layout: one wave per segment of consecutive outputs of one row (K * 64 16-byte chunks for
// Q8_0 / Q4_0 / dense types, 2048 outputs for K-quants), four independent waves per
// workgroup (no block barrier). Every lane produces 16 bytes of output per step (4 f32 or 8
// bf16), so each store instruction of a wave writes 1 KB of whole, contiguous cache lines.
// Q8_0 / Q4_0 (34 / 18 B blocks, 2-byte aligned): each lane loads the f16 scale and the
// quant bytes behind its outputs straight from global memory (a 16-bit load and 32-bit loads
// from 2-byte aligned addresses); the lanes of a wave read a contiguous span of the row, so
// the loads coalesce into that span's cache lines (measured on MI355X at 4096 x 2560: 9.4 us
// against 12.9 us for staging the row through LDS first).
// Q6_K / Q4_K (210 / 144 B super-blocks): the segment (8 super-blocks) is staged in LDS, then
// decoded.
// Dense types (F32, F16, BF16): each lane converts the elements behind its 16-byte stores,
// all loads (range-checked, so none waits behind another's bounds branch) issued before the
// first store.
#include "zl_common.h"
#include "zl_host.h"

namespace zl {

#ifndef ZL_GATHER_WAVES
#define ZL_GATHER_WAVES 4
#endif
constexpr int kGatherWaves = ZL_GATHER_WAVES;  // independent waves (segments) per workgroup
#ifndef ZL_GATHER_ROW_WG
#define ZL_GATHER_ROW_WG 0
#endif

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint32_t lds_u16(const unsigned char* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}


// Outputs per lane per step: one 16-byte store (4 f32 or 8 bf16), so each store instruction
// of a wave writes 64 x 16 B of contiguous, whole cache lines.
template <typename OutT>
__host__ __device__ constexpr int out_epl() {
    return 16 / (int)sizeof(OutT);
}

template <typename OutT>
__device__ __forceinline__ void store16(OutT* p, const float* v) {
    sts16(p, Chunk<OutT>::pack(v));
}
// Output stores of the Q8_0 / Q4_0 / dense gathers: cache policy ZL_GATHER_SP (zl_common.h
// POL_*), through a resource `r` over the output row at byte offset `off` (p = row + off).
#ifndef ZL_GATHER_SP
#define ZL_GATHER_SP POL_NT
#endif
template <typename OutT>
__device__ __forceinline__ void store16p(OutT* p, __amdgpu_buffer_rsrc_t r, uint32_t off, const float* v) {
    strow16<ZL_GATHER_SP>(p - off / sizeof(OutT), r, off, Chunk<OutT>::pack(v));
}

// Dequantise elements [e, e+N) (N = 4 or 8, e a multiple of N) of a block row staged at
// `row` in LDS, multiplied by `scale`.
template <int QT, int N>
__device__ __forceinline__ void dequant(const unsigned char* row, int e, float scale, float* v) {
    if constexpr (QT == HIP_BRIDGE_Q8_0) {
        const unsigned char* blk = row + (e >> 5) * 34;
        const float d = f16_bits_to_f32(lds_u16(blk));
        const unsigned char* qs = blk + 2 + (e & 31);
#pragma unroll
        for (int j = 0; j < N / 2; ++j) {
            const uint32_t w = lds_u16(qs + 2 * j);
            v[2 * j] = ((float)(int8_t)(w & 0xff) * d) * scale;
            v[2 * j + 1] = ((float)(int8_t)(w >> 8) * d) * scale;
        }
    } else if constexpr (QT == HIP_BRIDGE_Q4_0) {
        const unsigned char* blk = row + (e >> 5) * 18;
        const float d = f16_bits_to_f32(lds_u16(blk));
        const int o = e & 31;
        const unsigned char* qs = blk + 2 + (o & 15);
        const int shift = o < 16 ? 0 : 4;  // low nibbles -> elements 0..15, high -> 16..31
#pragma unroll
        for (int j = 0; j < N / 2; ++j) {
            const uint32_t w = lds_u16(qs + 2 * j);
            const int q0 = (int)((w >> shift) & 0xf) - 8;
            const int q1 = (int)((w >> (8 + shift)) & 0xf) - 8;
            v[2 * j] = ((float)q0 * d) * scale;
            v[2 * j + 1] = ((float)q1 * d) * scale;
        }
    } else if constexpr (QT == HIP_BRIDGE_Q4_K) {
        // Q4_K super-block of 256: d, dmin (f16), scales[12] (packed 6-bit scales / mins),
        // qs[128] = 144 B (types.zig:170-175); element order and arithmetic as
        // quant.zig:276-309: f32(q) * (d * sc_j) - dmin * m_j, then * scale.
        const unsigned char* sb = row + (e >> 8) * 144;
        const float d = f16_bits_to_f32(lds_u16(sb)), dmin = f16_bits_to_f32(lds_u16(sb + 2));
        const int w = e & 255;
        const int jj = w >> 6;            // pair of 32-element sub-blocks sharing qs[32 jj ..]
        const int hi = (w >> 5) & 1;      // high nibbles: the pair's second sub-block
        const int j = 2 * jj + hi;        // sub-block 0..7
        const unsigned char* sc = sb + 4;
        int s6, m6;
        if (j < 4) {
            s6 = sc[j] & 63;
            m6 = sc[j + 4] & 63;
        } else {
            s6 = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
            m6 = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
        }
        const float dj = d * (float)s6, mj = dmin * (float)m6;
        const unsigned char* qs = sb + 16 + 32 * jj + (w & 31);
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int q = hi ? (qs[k] >> 4) : (qs[k] & 0x0F);
            v[k] = ((float)q * dj - mj) * scale;
        }
    } else {
        // Q6_K super-block of 256: ql[128] qh[64] scales[16] (int8) d (f16) = 210 B
        // (types.zig:187-192); element order as quant.zig:357-385.
        const unsigned char* sb = row + (e >> 8) * 210;
        const float d = f16_bits_to_f32(lds_u16(sb + 208));
        const int w = e & 255;
        const int half = w >> 7;        // n in quant.zig:359
        const int grp = (w & 127) >> 5; // which of q1..q4
        const int l0 = w & 31;          // N consecutive l, same is = l/16
        const unsigned char* ql = sb + half * 64 + l0 + ((grp & 1) ? 32 : 0);
        const unsigned char* qh = sb + 128 + half * 32 + l0;
        const int8_t sc = (int8_t)sb[192 + half * 8 + (l0 >> 4) + 2 * grp];
        const float dsc = d * (float)sc;  // exact (11-bit x 8-bit)
        const int nshift = (grp & 2) ? 4 : 0;
        const int hshift = 2 * grp;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int lo = (ql[j] >> nshift) & 0xf;
            const int hi = (qh[j] >> hshift) & 3;
            const int q = (lo | (hi << 4)) - 32;
            v[j] = (dsc * (float)q) * scale;
        }
    }
}

template <int QT>
__host__ __device__ constexpr int64_t block_bytes() {
    return QT == HIP_BRIDGE_Q8_0 ? 34 : QT == HIP_BRIDGE_Q4_0 ? 18 : QT == HIP_BRIDGE_Q4_K ? 144 : 210;
}
template <int QT>
__host__ __device__ constexpr int block_elems() {
    return QT == HIP_BRIDGE_Q6_K || QT == HIP_BRIDGE_Q4_K ? 256 : 32;
}

template <int QT>
__host__ __device__ constexpr int seg_elems() {
    return QT == HIP_BRIDGE_Q6_K || QT == HIP_BRIDGE_Q4_K ? 2048 : 512;
}


// Steps per wave of the Q8_0 / Q4_0 (K_Q) and dense (K_D) gathers: a wave takes K * 64
// consecutive 16-byte output chunks of one row (K * 256 f32 or K * 512 bf16 outputs) and
// reads its row's id once. Measured at 4096 x 2560 -> f32 (us, K = 2 / 3 / 5 / 10): Q8_0
// 10.2 / 10.5 / 11.0 / 12.2, Q4_0 8.66 / 8.83 / 9.2 / 8.95, BF16 12.3 / 12.3 / 12.1 / 12.2;
// K = 1 and 4 retaken later against 10.3 / 8.7 for K = 2: Q8_0 17.5 / 11.1, Q4_0 16.6 / 8.9.
// Not taken: a persistent grid whose waves walk segments with the next segment's table loads
// and the id after it in flight (bit-equal): Q8_0 / Q4_0 10.28 / 8.71 -> 10.45 / 9.14 us at 8
// workgroups per CU (2, 4, 6: slower still).
#ifndef ZL_GATHER_STEPS
#define ZL_GATHER_STEPS 2
#endif
#ifndef ZL_GATHER_STEPS_DENSE
#define ZL_GATHER_STEPS_DENSE 5
#endif
constexpr int kGatherSteps = ZL_GATHER_STEPS;
constexpr int kGatherStepsDense = ZL_GATHER_STEPS_DENSE;

typedef uint32_t u32_a2 __attribute__((aligned(2)));
// 32-bit load from a 2-byte aligned address (one global_load_dword; gfx950 serves it
// unaligned).
__device__ __forceinline__ uint32_t ld32_a2(const unsigned char* p) {
    return *reinterpret_cast<const u32_a2*>(p);
}

// Q8_0 / Q4_0: per 16-byte output chunk (N = 4 f32 or 8 bf16 outputs of one block) a lane
// loads the block's f16 scale (16-bit) and the quant bytes behind its outputs as 32-bit
// words from 2-byte aligned addresses (Q8_0: N bytes; Q4_0: 4 bytes for N = 4, 8 for N = 8,
// low nibbles for elements 0..15 of the block, high for 16..31). Every address is clamped
// into the table (id 0, element 0 for lanes past the row or an invalid id) and the values
// are dropped afterwards, so no load sits under a branch and all 2K of a lane's loads are in
// flight before its first store.
template <int QT, typename OutT, int K>
__global__ __launch_bounds__(ZL_GATHER_ROW_WG ? 512 : 64 * kGatherWaves) void k_gather_q(const unsigned char* __restrict__ table,
                                                  const int32_t* __restrict__ ids,
                                                  OutT* __restrict__ out, int64_t n_rows,
                                                  int64_t n_tokens, int dim, float scale, int nseg,
                                                  int64_t single_id) {
    constexpr int N = out_epl<OutT>();  // outputs per lane per step
    constexpr int S = K * kWave * N;    // outputs per wave
    constexpr int BB = (int)block_bytes<QT>();
    constexpr int NW = N / 4;  // quant words per chunk: one byte per output (Q4_0: a nibble of it)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t wg = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
    const int64_t t = wg / nseg;
    if (t >= n_tokens) return;
    const int e0 = (int)(wg - t * nseg) * S;
    const int64_t id = ids ? (int64_t)ids[t] : single_id;  // wave-uniform: a scalar load
    const bool valid = id >= 0 && id < n_rows;
    const unsigned char* grow = table + (valid ? id : 0) * (int64_t)(dim / 32) * BB;
    uint32_t dq[K], w[K][NW];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int e = e0 + kWave * N * k + lane * N;
        const int ec = e < dim ? e : 0;
        const unsigned char* blk = grow + (ec >> 5) * BB;
        dq[k] = lds_u16(blk);
        const unsigned char* qs = blk + 2 + (QT == HIP_BRIDGE_Q8_0 ? (ec & 31) : (ec & 15));
#pragma unroll
        for (int j = 0; j < NW; ++j) w[k][j] = ld32_a2(qs + 4 * j);
    }
    OutT* orow = out + t * (int64_t)dim;
    const auto ro = buf_rsrc(orow, (uint32_t)dim * sizeof(OutT));
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int e = e0 + kWave * N * k + lane * N;
        if (e >= dim) break;
        float v[N];
        const float d = f16_bits_to_f32(dq[k]);
        const int shift = (e & 31) < 16 ? 0 : 4;  // Q4_0: low or high nibbles of the block
#pragma unroll
        for (int j = 0; j < N; ++j) {
            // element j of the chunk: byte j of the lane's quant span
            const uint32_t byte = w[k][j >> 2] >> (8 * (j & 3));
            const int q = QT == HIP_BRIDGE_Q8_0 ? (int)(int8_t)(byte & 0xff) : (int)((byte >> shift) & 0xf) - 8;
            v[j] = ((float)q * d) * scale;
        }
        if (!valid) {
#pragma unroll
            for (int j = 0; j < N; ++j) v[j] = 0.0f;
        }
        store16p<OutT>(orow + e, ro, (uint32_t)e * sizeof(OutT), v);
    }
}

// Q6_K, and Q8_0 / Q4_0 tables at an odd address: the segment's bytes are staged in LDS
// (128-bit loads when the row is 16-byte aligned, byte loads otherwise), then decoded.
// Segments hold whole blocks and start at multiples of 16 bytes within the row.
template <int QT, typename OutT>
__global__ __launch_bounds__(64 * kGatherWaves) void k_gather_blocks(const unsigned char* __restrict__ table,
                                                       const int32_t* __restrict__ ids,
                                                       OutT* __restrict__ out, int64_t n_rows,
                                                       int64_t n_tokens, int dim, float scale,
                                                       int row_bytes, int nseg, int vec16,
                                                       int64_t single_id) {
    constexpr int SEG = seg_elems<QT>();
    constexpr int SEG_BYTES = SEG / block_elems<QT>() * (int)block_bytes<QT>();
    constexpr int LDS_STRIDE = (SEG_BYTES + 15) & ~15;
    static_assert(SEG_BYTES % 16 == 0, "segments must start 16-byte aligned");
    __shared__ __attribute__((aligned(16))) unsigned char s_seg[kGatherWaves * LDS_STRIDE];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t wg = (int64_t)blockIdx.x * kGatherWaves + wave;
    const int64_t t = wg / nseg;
    const int sg = (int)(wg - t * nseg);
    unsigned char* sseg = s_seg + wave * LDS_STRIDE;
    const int e0 = sg * SEG;
    const int e1 = dim - e0 < SEG ? dim : e0 + SEG;
    int64_t id = -1;
    if (t < n_tokens) {
        id = ids ? (int64_t)ids[t] : single_id;
        if (id >= 0 && id < n_rows) {
            const int b0 = sg * SEG_BYTES;
            const int b1 = (e1 / block_elems<QT>()) * (int)block_bytes<QT>();
            const unsigned char* gseg = table + id * (int64_t)row_bytes + b0;
            if (vec16) {
                // row_bytes % 16 == 0: the rounded-up last chunk stays inside the row
                const int n16 = (b1 - b0 + 15) >> 4;
                constexpr int UN = (SEG_BYTES / 16 + kWave - 1) / kWave;
                u32x4 tmp[UN];
#pragma unroll
                for (int u = 0; u < UN; ++u) {
                    const int i = lane + kWave * u;
                    if (i < n16) tmp[u] = ld16(gseg + 16 * i);
                }
#pragma unroll
                for (int u = 0; u < UN; ++u) {
                    const int i = lane + kWave * u;
                    if (i < n16) st16(sseg + 16 * i, tmp[u]);
                }
            } else {
                for (int i = lane; i < b1 - b0; i += kWave) sseg[i] = gseg[i];
            }
        }
    }
    // Each wave reads only the segment it staged: a wave-scope fence + barrier (LDS writes
    // complete and ordered before the reads) instead of a block barrier, so the four waves of
    // a workgroup do not wait for each other's HBM latency.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (t >= n_tokens) return;
    OutT* orow = out + t * (int64_t)dim;
    const bool valid = id >= 0 && id < n_rows;
    constexpr int N = out_epl<OutT>();
    for (int e = e0 + lane * N; e < e1; e += kWave * N) {
        float v[N];
        if (valid) {
            dequant<QT, N>(sseg, e - e0, scale, v);
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) v[j] = 0.0f;
        }
        store16<OutT>(orow + e, v);
    }
}

// Dense types: one wave per 512-output segment; per step each lane converts the N inputs
// behind one 16-byte output store (f32 -> f32: 16 B loads; 16-bit -> f32: 8 B; 16-bit ->
// bf16: 16 B; f32 -> bf16: 2 x 16 B), every load and store instruction contiguous across
// the wave, all of a lane's loads issued before its first store.
template <int QT, int N>
struct DenseIn {
    static constexpr int ES = QT == HIP_BRIDGE_F32 ? 4 : 2;
    static constexpr int WORDS = N * ES / 4;  // 32-bit words behind N outputs
    uint32_t w[WORDS];
    // rs: the row's resource; off: byte offset of the first input (past the row: zeros).
    // Plain (cached) loads: for rows at random addresses they measured faster than
    // nontemporal ones (BF16 -> f32 at 4096 x 2560: 11.4 against 13.3 us).
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
        if constexpr (WORDS == 2) {
            const auto r = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
            w[0] = r.x;
            w[1] = r.y;
        } else {
#pragma unroll
            for (int c = 0; c < WORDS / 4; ++c) {
                const auto r = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u * c, 0, 0));
                w[4 * c] = r.x;
                w[4 * c + 1] = r.y;
                w[4 * c + 2] = r.z;
                w[4 * c + 3] = r.w;
            }
        }
    }
    __device__ __forceinline__ void convert(float scale, float* v) const {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            float x;
            if constexpr (QT == HIP_BRIDGE_F32) {
                x = __uint_as_float(w[j]);
            } else {
                const uint32_t h = (j & 1) ? w[j >> 1] >> 16 : w[j >> 1] & 0xffff;
                x = QT == HIP_BRIDGE_BF16 ? __uint_as_float(h << 16) : f16_bits_to_f32(h);
            }
            v[j] = x * scale;
        }
    }
};

template <int QT, typename OutT, int K>
__global__ __launch_bounds__(64 * kGatherWaves) void k_gather_dense(const unsigned char* __restrict__ table,
                                                      const int32_t* __restrict__ ids,
                                                      OutT* __restrict__ out, int64_t n_rows,
                                                      int64_t n_tokens, int dim, float scale,
                                                      int nseg, int64_t single_id) {
    constexpr int N = out_epl<OutT>();
    using In = DenseIn<QT, N>;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t wg = (int64_t)blockIdx.x * kGatherWaves + wave;
    const int64_t t = wg / nseg;
    if (t >= n_tokens) return;
    const int e0 = (int)(wg - t * nseg) * (K * kWave * N);
    const int64_t id = ids ? (int64_t)ids[t] : single_id;  // wave-uniform: a scalar load
    const bool valid = id >= 0 && id < n_rows;
    const int64_t rbytes = (int64_t)dim * In::ES;
    const auto rs = buf_rsrc(table + (valid ? id : 0) * rbytes, valid ? (uint32_t)rbytes : 0u);
    In in[K];
#pragma unroll
    for (int k = 0; k < K; ++k) in[k].load(rs, (uint32_t)(e0 + lane * N + kWave * N * k) * In::ES);
    OutT* orow = out + t * (int64_t)dim;
    const auto ro = buf_rsrc(orow, (uint32_t)dim * sizeof(OutT));
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int e = e0 + lane * N + kWave * N * k;
        if (e >= dim) break;
        float v[N];
        if (valid) {
            in[k].convert(scale, v);
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) v[j] = 0.0f;
        }
        store16p<OutT>(orow + e, ro, (uint32_t)e * sizeof(OutT), v);
    }
}

// Any dense row layout / alignment: one thread per output element (scalar loads).
template <int QT, typename OutT>
__global__ __launch_bounds__(256) void k_gather_dense_scalar(const unsigned char* __restrict__ table,
                                                             const int32_t* __restrict__ ids,
                                                             OutT* __restrict__ out, int64_t n_rows,
                                                             int64_t n_tokens, int dim, float scale,
                                                             int64_t single_id) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_tokens * (int64_t)dim) return;
    const int64_t t = i / dim, c = i - t * dim;
    const int64_t id = ids ? (int64_t)ids[t] : single_id;
    float v = 0.0f;
    if (id >= 0 && id < n_rows) {
        if constexpr (QT == HIP_BRIDGE_F32) {
            const unsigned char* p = table + (id * dim + c) * 4;
            v = __uint_as_float((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                                ((uint32_t)p[3] << 24));
        } else {
            const unsigned char* p = table + (id * dim + c) * 2;
            const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
            v = QT == HIP_BRIDGE_BF16 ? bf16_lo(h) : f16_bits_to_f32(h);
        }
        v = v * scale;
    }
    if constexpr (sizeof(OutT) == 4) {
        out[i] = v;
    } else {
        out[i] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffff);
    }
}

static int64_t row_bytes_of(int qtype, int dim) {
    switch (qtype) {
        case HIP_BRIDGE_F32: return (int64_t)dim * 4;
        case HIP_BRIDGE_F16:
        case HIP_BRIDGE_BF16: return (int64_t)dim * 2;
        case HIP_BRIDGE_Q8_0: return dim % 32 ? -1 : (int64_t)(dim / 32) * 34;
        case HIP_BRIDGE_Q4_0: return dim % 32 ? -1 : (int64_t)(dim / 32) * 18;
        case HIP_BRIDGE_Q4_K: return dim % 256 ? -1 : (int64_t)(dim / 256) * 144;
        case HIP_BRIDGE_Q6_K: return dim % 256 ? -1 : (int64_t)(dim / 256) * 210;
        default: return -1;
    }
}

template <int QT, typename OutT>
static void launch_blocks(const void* table, const int32_t* ids, int64_t single_id, void* out,
                          int64_t n_rows, int64_t n_tokens, int dim, float scale, hipStream_t s) {
    const int64_t rb = row_bytes_of(QT, dim);
    const int vec16 = (rb % 16 == 0) && aligned16(table);
    const int nseg = (int)cdiv(dim, seg_elems<QT>());
    const int64_t grid = cdiv(n_tokens * nseg, kGatherWaves);
    if (grid > INT32_MAX) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    k_gather_blocks<QT, OutT><<<(unsigned)grid, 64 * kGatherWaves, 0, s>>>(
        (const unsigned char*)table, ids, (OutT*)out, n_rows, n_tokens, dim, scale, (int)rb,
        nseg, vec16, single_id);
    check_launch();
}

template <int QT, typename OutT>
static void launch_q(const void* table, const int32_t* ids, int64_t single_id, void* out,
                     int64_t n_rows, int64_t n_tokens, int dim, float scale, hipStream_t s) {
    constexpr int S = kGatherSteps * kWave * out_epl<OutT>();
    const int nseg = (int)cdiv(dim, S);
    // A row's segments share the 128-byte lines at their boundaries (rows of 34- or 18-byte
    // blocks start anywhere within a line), and workgroups that split a row across XCDs fetch
    // each shared line once per L2. ZL_GATHER_ROW_WG=1 puts every segment of a row in one
    // workgroup (nseg waves): at 4096 x 2560 -> f32 it cuts the table bytes fetched by 3.3%
    // (Q8_0) and 5.7% (Q4_0) but runs slower (10.72 against 10.28 us, 8.89 against 8.72 us),
    // so the default keeps kGatherWaves segments per workgroup.
    const int wpw = ZL_GATHER_ROW_WG && nseg <= 8 ? nseg : kGatherWaves;
    const int64_t grid = cdiv(n_tokens * nseg, wpw);
    if (grid > INT32_MAX) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    k_gather_q<QT, OutT, kGatherSteps><<<(unsigned)grid, 64 * wpw, 0, s>>>(
        (const unsigned char*)table, ids, (OutT*)out, n_rows, n_tokens, dim, scale, nseg, single_id);
    check_launch();
}

template <int QT, typename OutT>
static void launch_dense(const void* table, const int32_t* ids, int64_t single_id, void* out,
                         int64_t n_rows, int64_t n_tokens, int dim, float scale, hipStream_t s) {
    const bool vec = dim % 8 == 0 && aligned16(table) && aligned16(out);
    if (vec) {
        const int nseg = (int)cdiv(dim, kGatherStepsDense * kWave * out_epl<OutT>());
        const int64_t grid = cdiv(n_tokens * nseg, kGatherWaves);
        if (grid > INT32_MAX) {
            set_error(HIP_BRIDGE_EUNSUPPORTED);
            return;
        }
        k_gather_dense<QT, OutT, kGatherStepsDense><<<(unsigned)grid, 64 * kGatherWaves, 0, s>>>(
            (const unsigned char*)table, ids, (OutT*)out, n_rows, n_tokens, dim, scale, nseg,
            single_id);
    } else {
        const int64_t grid = cdiv(n_tokens * (int64_t)dim, 256);
        if (grid > INT32_MAX) {
            set_error(HIP_BRIDGE_EUNSUPPORTED);
            return;
        }
        k_gather_dense_scalar<QT, OutT><<<(unsigned)grid, 256, 0, s>>>(
            (const unsigned char*)table, ids, (OutT*)out, n_rows, n_tokens, dim, scale, single_id);
    }
    check_launch();
}

template <typename OutT>
static void gather(const void* table, int qtype, int64_t n_rows, const int32_t* ids,
                   int64_t single_id, void* out, int64_t n_tokens, int dim, float scale,
                   hipStream_t s) {
    const int out_es = (int)sizeof(OutT);
    const bool block_ok = dim % 8 == 0 && aligned16(out) && ((int64_t)dim * out_es) % 16 == 0;
    const bool even = (reinterpret_cast<uintptr_t>(table) & 1u) == 0;
    switch (qtype) {
        case HIP_BRIDGE_Q8_0:
            if (!block_ok) break;
            if (even) return launch_q<HIP_BRIDGE_Q8_0, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
            return launch_blocks<HIP_BRIDGE_Q8_0, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_Q4_0:
            if (!block_ok) break;
            if (even) return launch_q<HIP_BRIDGE_Q4_0, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
            return launch_blocks<HIP_BRIDGE_Q4_0, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_Q6_K:
            if (!block_ok) break;
            return launch_blocks<HIP_BRIDGE_Q6_K, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_Q4_K:
            if (!block_ok) break;
            return launch_blocks<HIP_BRIDGE_Q4_K, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_F32:
            return launch_dense<HIP_BRIDGE_F32, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_F16:
            return launch_dense<HIP_BRIDGE_F16, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_BF16:
            return launch_dense<HIP_BRIDGE_BF16, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        default:
            break;
    }
    set_error(HIP_BRIDGE_EUNSUPPORTED);
}

}  // namespace zl

using namespace zl;

extern "C" {

void hip_embed_gather(const void* table, int qtype, int64_t n_rows, const int32_t* ids,
                      int out_dtype, void* out, int64_t n_tokens, int dim, float scale,
                      HipStream_t stream) {
    if (n_tokens <= 0 || dim <= 0) return;
    if (!table || !ids || !out) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    if (row_bytes_of(qtype, dim) < 0) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    if (out_dtype == HIP_BRIDGE_F32)
        gather<float>(table, qtype, n_rows, ids, 0, out, n_tokens, dim, scale, stream_of(stream));
    else if (out_dtype == HIP_BRIDGE_BF16)
        gather<uint16_t>(table, qtype, n_rows, ids, 0, out, n_tokens, dim, scale, stream_of(stream));
    else
        set_error(HIP_BRIDGE_EUNSUPPORTED);
}

void hip_embed_lookup_batch(const void* emb_weights, int qtype, const int* token_ids, float* out,
                            int n_tokens, int dim, float scale, HipStream_t stream) {
    // The reference ABI carries no vocabulary size: ids are trusted (negative ids give a
    // zero row).
    hip_embed_gather(emb_weights, qtype, INT64_MAX, token_ids, HIP_BRIDGE_F32, out, n_tokens,
                     dim, scale, stream);
}

}  // extern "C"

extern "C" void hip_embed_lookup(const void* emb_weights, int qtype, int token_id, float* out,
                                 int dim, float scale, HipStream_t stream) {
    // Single token: the id is a host value and travels as a kernel argument.
    if (!emb_weights || dim <= 0) return;
    if (!out) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    if (row_bytes_of(qtype, dim) < 0) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    gather<float>(emb_weights, qtype, INT64_MAX, nullptr, token_id, out, 1, dim, scale,
                  stream_of(stream));
}
