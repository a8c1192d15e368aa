// Embedding-row gather + dequant + scale (replaces cuda_bridge.cu:1559-1940).
//
// Arithmetic is ziglm's CPU order (quant.zig:73-79, 119-130, 357-385, 413-512 and
// model.zig:494-503): out = fl(fl(f32(q) * d) * scale). For Q8_0/Q4_0 q*d is exact, so every
// output is one IEEE rounding and the result is bit-exact; Q6_K keeps the CPU's
// ((d * scale_j) * q) * scale order.
//
// Layout: one wave per segment of consecutive outputs of one row (512 outputs; 2048 for
// Q6_K), four independent waves per workgroup (no block barrier). Block formats (Q8_0 34 B,
// Q4_0 18 B, Q6_K 210 B per block) are not 16-byte aligned per block, but segments of 16
// (Q8_0/Q4_0) or 8 (Q6_K) blocks are (544 / 288 / 1680 B), and so are whole rows at the
// usual widths (2720 / 1440 B at 2560 columns). A wave copies its segment into LDS with
// 128-bit loads (byte loads when the row is not 16-byte aligned), then each lane dequantises
// 8 consecutive outputs from LDS and writes them with 128-bit stores: one HBM read of the
// row, one HBM write of the output, the per-block scale read once per 8 outputs.
// Dense types (F32, F16, BF16) skip LDS: each lane converts 8 consecutive elements.
#include "zl_common.h"
#include "zl_host.h"

namespace zl {

constexpr int kGatherWaves = 4;  // rows per workgroup

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint32_t lds_u16(const unsigned char* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// Writes 8 consecutive outputs starting at element e of row `orow`.
template <typename OutT>
__device__ __forceinline__ void store8(OutT* orow, int64_t e, const float* v);
template <>
__device__ __forceinline__ void store8<float>(float* orow, int64_t e, const float* v) {
    sts16(orow + e, Chunk<float>::pack(v));
    sts16(orow + e + 4, Chunk<float>::pack(v + 4));
}
template <>
__device__ __forceinline__ void store8<uint16_t>(uint16_t* orow, int64_t e, const float* v) {
    sts16(orow + e, Chunk<uint16_t>::pack(v));
}

// Dequantise elements [e, e+8) of a row staged at `row` in LDS, multiplied by `scale`.
template <int QT>
__device__ __forceinline__ void dequant8(const unsigned char* row, int e, float scale, float* v);

template <>
__device__ __forceinline__ void dequant8<HIP_BRIDGE_Q8_0>(const unsigned char* row, int e, float scale,
                                                    float* v) {
    const unsigned char* blk = row + (e >> 5) * 34;
    const float d = f16_bits_to_f32(lds_u16(blk));
    const unsigned char* qs = blk + 2 + (e & 31);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t w = lds_u16(qs + 2 * j);
        v[2 * j] = ((float)(int8_t)(w & 0xff) * d) * scale;
        v[2 * j + 1] = ((float)(int8_t)(w >> 8) * d) * scale;
    }
}

template <>
__device__ __forceinline__ void dequant8<HIP_BRIDGE_Q4_0>(const unsigned char* row, int e, float scale,
                                                    float* v) {
    const unsigned char* blk = row + (e >> 5) * 18;
    const float d = f16_bits_to_f32(lds_u16(blk));
    const int o = e & 31;
    const unsigned char* qs = blk + 2 + (o & 15);
    const int shift = o < 16 ? 0 : 4;  // low nibbles -> elements 0..15, high -> 16..31
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t w = lds_u16(qs + 2 * j);
        const int q0 = (int)((w >> shift) & 0xf) - 8;
        const int q1 = (int)((w >> (8 + shift)) & 0xf) - 8;
        v[2 * j] = ((float)q0 * d) * scale;
        v[2 * j + 1] = ((float)q1 * d) * scale;
    }
}

template <>
__device__ __forceinline__ void dequant8<HIP_BRIDGE_Q6_K>(const unsigned char* row, int e, float scale,
                                                    float* v) {
    // Super-block of 256: ql[128] qh[64] scales[16] (int8) d (f16) = 210 B (types.zig:187-192).
    const unsigned char* sb = row + (e >> 8) * 210;
    const float d = f16_bits_to_f32(lds_u16(sb + 208));
    const int w = e & 255;
    const int half = w >> 7;        // n in quant.zig:359
    const int grp = (w & 127) >> 5; // which of q1..q4
    const int l0 = w & 31;          // 8 consecutive l, same is = l/16
    const unsigned char* ql = sb + half * 64 + l0 + ((grp & 1) ? 32 : 0);
    const unsigned char* qh = sb + 128 + half * 32 + l0;
    const int8_t sc = (int8_t)sb[192 + half * 8 + (l0 >> 4) + 2 * grp];
    const float dsc = d * (float)sc;  // exact (11-bit x 8-bit)
    const int nshift = (grp & 2) ? 4 : 0;
    const int hshift = 2 * grp;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int lo = (ql[j] >> nshift) & 0xf;
        const int hi = (qh[j] >> hshift) & 3;
        const int q = (lo | (hi << 4)) - 32;
        v[j] = (dsc * (float)q) * scale;
    }
}

template <int QT>
__host__ __device__ constexpr int64_t block_bytes() {
    return QT == HIP_BRIDGE_Q8_0 ? 34 : QT == HIP_BRIDGE_Q4_0 ? 18 : 210;
}
template <int QT>
__host__ __device__ constexpr int block_elems() {
    return QT == HIP_BRIDGE_Q6_K ? 256 : 32;
}

// Work split: one wave per segment of kSegElems[QT] consecutive outputs of one row
// (n_tokens * ceil(dim / seg) waves, four per workgroup, independent of each other), so a
// 2048-4096-token gather puts tens of thousands of waves in flight instead of one per row.
// Segments hold whole blocks and start at multiples of 16 bytes within the row.
template <int QT>
__host__ __device__ constexpr int seg_elems() {
    return QT == HIP_BRIDGE_Q6_K ? 2048 : 512;  // Q8_0 544 B, Q4_0 288 B, Q6_K 1680 B
}

// Block formats: the segment's bytes are staged in LDS, then dequantised 8 outputs per lane.
template <int QT, typename OutT>
__global__ __launch_bounds__(256) void k_gather_blocks(const unsigned char* __restrict__ table,
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
                    if (i < n16) tmp[u] = lds16(gseg + 16 * i);
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
    for (int e = e0 + lane * 8; e < e1; e += kWave * 8) {
        float v[8];
        if (valid) {
            dequant8<QT>(sseg, e - e0, scale, v);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = 0.0f;
        }
        store8<OutT>(orow, e, v);
    }
}

// Dense types: one wave per 512-output segment, each lane converts 8 consecutive elements
// (one 16-byte load of f16/bf16, two of f32).
template <int QT, typename OutT>
__global__ __launch_bounds__(256) void k_gather_dense(const unsigned char* __restrict__ table,
                                                      const int32_t* __restrict__ ids,
                                                      OutT* __restrict__ out, int64_t n_rows,
                                                      int64_t n_tokens, int dim, float scale,
                                                      int nseg, int64_t single_id) {
    constexpr int ES = QT == HIP_BRIDGE_F32 ? 4 : 2;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t wg = (int64_t)blockIdx.x * kGatherWaves + wave;
    const int64_t t = wg / nseg;
    if (t >= n_tokens) return;
    const int e = (int)(wg - t * nseg) * 512 + lane * 8;
    if (e >= dim) return;
    const int64_t id = ids ? (int64_t)ids[t] : single_id;
    float v[8];
    if (id >= 0 && id < n_rows) {
        const unsigned char* p = table + (id * (int64_t)dim + e) * ES;
        if constexpr (QT == HIP_BRIDGE_F32) {
            const u32x4 r0 = lds16(p), r1 = lds16(p + 16);
            Chunk<float>::unpack(r0, v);
            Chunk<float>::unpack(r1, v + 4);
        } else if constexpr (QT == HIP_BRIDGE_BF16) {
            Chunk<uint16_t>::unpack(lds16(p), v);
        } else {
            const u32x4 r = lds16(p);
            const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = f16_bits_to_f32(w[j] & 0xffff);
                v[2 * j + 1] = f16_bits_to_f32(w[j] >> 16);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = v[j] * scale;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.0f;
    }
    store8<OutT>(out + t * (int64_t)dim, e, v);
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
    k_gather_blocks<QT, OutT><<<(unsigned)grid, 256, 0, s>>>(
        (const unsigned char*)table, ids, (OutT*)out, n_rows, n_tokens, dim, scale, (int)rb,
        nseg, vec16, single_id);
    check_launch();
}

template <int QT, typename OutT>
static void launch_dense(const void* table, const int32_t* ids, int64_t single_id, void* out,
                         int64_t n_rows, int64_t n_tokens, int dim, float scale, hipStream_t s) {
    const bool vec = dim % 8 == 0 && aligned16(table) && aligned16(out);
    if (vec) {
        const int nseg = (int)cdiv(dim, 512);
        const int64_t grid = cdiv(n_tokens * nseg, kGatherWaves);
        if (grid > INT32_MAX) {
            set_error(HIP_BRIDGE_EUNSUPPORTED);
            return;
        }
        k_gather_dense<QT, OutT><<<(unsigned)grid, 256, 0, s>>>(
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
    switch (qtype) {
        case HIP_BRIDGE_Q8_0:
            if (!block_ok) break;
            return launch_blocks<HIP_BRIDGE_Q8_0, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_Q4_0:
            if (!block_ok) break;
            return launch_blocks<HIP_BRIDGE_Q4_0, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
        case HIP_BRIDGE_Q6_K:
            if (!block_ok) break;
            return launch_blocks<HIP_BRIDGE_Q6_K, OutT>(table, ids, single_id, out, n_rows, n_tokens, dim, scale, s);
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
