// Reference streaming kernel: the practical HBM ceiling of an op's byte mix. It reads n_in
// streams and writes n_out streams of `bytes` each (out_j[i] = in0[i] ^ in1[i], or in0[i]),
// so an op that reads R tensors and writes W tensors of one size can be set beside a kernel
// that moves exactly the same bytes and does nothing else. out0 may be in0 (a read-modify-
// write of one tensor in place, as the residual-stream updates x += ... do). Launch shapes
// combine threads per workgroup, 128-bit chunks per thread and the load / store cache
// policies the ops choose among (zl_common.h POL_*); the benchmark times each and takes the
// fastest as the ceiling of that size and mix.
//
// A second form, hip_stream_ref_copies, copies up to three (source, destination, size)
// pairs in one launch, for ops whose streams differ in size: the QK op reads Q, K and V and
// writes Q in place and K / V into the caches. Its workgroups take the pairs one after the
// other, or interleaved in proportion to their sizes (as an op that moves all three per
// token does).
//
// Every shape issues all of a thread's loads before its first store; accesses go through
// range-checked buffer resources over the workgroup's span.
#include "zl_common.h"
#include "zl_host.h"

namespace zl {

struct StreamArgs {
    const uint8_t* in0;
    const uint8_t* in1;
    uint8_t* out0;
    uint8_t* out1;
    int64_t nch;  // 16-byte chunks per stream
    // copies form (NIN == 0): pair p copies pch[p] chunks src[p] -> dst[p] with workgroups
    // [wg0[p], wg0[p + 1])
    const uint8_t* src[3];
    uint8_t* dst[3];
    int64_t pch[3];
    uint32_t wg0[4];
    int ilv;  // interleave the pairs' workgroups
};

// Interleaved order: workgroup b of n = n0 + n1 + n2 goes to pair 0 when the count of pair-0
// workgroups among the first b + 1, floor((b + 1) n0 / n), steps there (as Bresenham's line
// spreads its steps), else to pairs 1 / 2 the same way over the remaining index. Every pair
// gets exactly its count, each local index once.
__device__ __forceinline__ void ilv_pair(uint32_t b, const uint32_t* wg0, int& p, uint32_t& local) {
    const uint64_t n0 = wg0[1], n1 = wg0[2] - wg0[1], n = wg0[3];
    const uint64_t a1 = ((uint64_t)b + 1) * n0 / n, a0 = (uint64_t)b * n0 / n;
    if (a1 > a0) {
        p = 0;
        local = (uint32_t)a0;
        return;
    }
    const uint64_t r = b - a1, m = n - n0;
    const uint64_t c1 = (r + 1) * n1 / m, c0 = r * n1 / m;
    p = c1 > c0 ? 1 : 2;
    local = (uint32_t)(c1 > c0 ? c0 : r - c1);
}

// Store policy kGlobalNt: nt stores as global (per-lane address) stores, the form the norm
// kernels use (buffer nt stores are the other nt form).
constexpr int kGlobalNt = -1;

// U chunks per thread, consecutive by workgroup: chunk (block * U + u) * THREADS + thread.
// NIN == 0: the copies form (one read and one write stream per pair).
template <int NIN, int NOUT, int THREADS, int U, int LP, int SP>
__global__ __launch_bounds__(THREADS) void k_stream(StreamArgs a) {
    const uint8_t* in0 = a.in0;
    const uint8_t* in1 = a.in1;
    uint8_t* out0 = a.out0;
    uint8_t* out1 = a.out1;
    int64_t nch = a.nch;
    uint32_t blk = blockIdx.x;
    if constexpr (NIN == 0) {  // the workgroup's pair (uniform)
        int p;
        if (a.ilv) {
            ilv_pair(blk, a.wg0, p, blk);
        } else {
            p = blk < a.wg0[1] ? 0 : blk < a.wg0[2] ? 1 : 2;
            blk -= p == 0 ? 0u : p == 1 ? a.wg0[1] : a.wg0[2];
        }
        in0 = p == 0 ? a.src[0] : p == 1 ? a.src[1] : a.src[2];
        out0 = p == 0 ? a.dst[0] : p == 1 ? a.dst[1] : a.dst[2];
        nch = p == 0 ? a.pch[0] : p == 1 ? a.pch[1] : a.pch[2];
    }
    const int64_t c0 = (int64_t)blk * U * THREADS;
    const int64_t left = nch - c0;
    const uint32_t bytes = (uint32_t)(left < U * THREADS ? left : U * THREADS) * 16u;
    const auto r0 = buf_rsrc(in0 + c0 * 16, bytes);
    const auto r1 = buf_rsrc(NIN == 2 ? in1 + c0 * 16 : in0, NIN == 2 ? bytes : 0u);
    const auto w0 = buf_rsrc(out0 + c0 * 16, bytes);
    const auto w1 = buf_rsrc(NOUT == 2 ? out1 + c0 * 16 : out0, NOUT == 2 ? bytes : 0u);
    u32x4 x[U], y[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t off = (uint32_t)(u * THREADS + threadIdx.x) * 16u;
        x[u] = bldp<LP>(r0, off);
        if constexpr (NIN == 2) y[u] = bldp<LP>(r1, off);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t off = (uint32_t)(u * THREADS + threadIdx.x) * 16u;
        const u32x4 v = NIN == 2 ? (x[u] ^ y[u]) : x[u];
        if constexpr (SP == kGlobalNt) {
            if (off < bytes) {
                sts16(out0 + c0 * 16 + off, v);
                if constexpr (NOUT == 2) sts16(out1 + c0 * 16 + off, v);
            }
        } else {
            bstp<SP>(w0, off, v);
            if constexpr (NOUT == 2) bstp<SP>(w1, off, v);
        }
    }
}

// The launch shapes the ceiling is the best of: {threads, chunks per thread} x load policy
// {default, nt} x store policy {nt (buffer store), sc1}, and nt loads with nt global stores. The 3-, 5- and 6-chunk shapes follow the norm
// kernels' layout (a 128- or 256-thread group over 3 chunks per lane of a row, two rows per
// group).
struct Shape {
    int threads, unroll;
};
constexpr Shape kGeo[] = {{64, 1}, {256, 1}, {256, 2}, {256, 4}, {512, 2}, {128, 3}, {256, 3}, {256, 5}, {256, 6}};
constexpr int kNumGeo = sizeof(kGeo) / sizeof(kGeo[0]);
constexpr int kNumShapes = kNumGeo * 5;

template <int NIN, int NOUT, int THREADS, int U, int LP, int SP>
static void launch_one(const StreamArgs& a, hipStream_t s) {
    if constexpr (NIN == 0) {
        StreamArgs c = a;
        c.wg0[0] = 0;
        for (int p = 0; p < 3; ++p) c.wg0[p + 1] = c.wg0[p] + (uint32_t)cdiv(c.pch[p], (int64_t)THREADS * U);
        if (c.wg0[3] > 0) k_stream<0, 1, THREADS, U, LP, SP><<<c.wg0[3], THREADS, 0, s>>>(c);
    } else {
        const int64_t grid = cdiv(a.nch, (int64_t)THREADS * U);
        k_stream<NIN, NOUT, THREADS, U, LP, SP><<<(unsigned)grid, THREADS, 0, s>>>(a);
    }
}

template <int NIN, int NOUT, int LP, int SP>
static void launch_geo(int geo, const StreamArgs& a, hipStream_t s) {
    switch (geo) {
        case 0: launch_one<NIN, NOUT, 64, 1, LP, SP>(a, s); break;
        case 1: launch_one<NIN, NOUT, 256, 1, LP, SP>(a, s); break;
        case 2: launch_one<NIN, NOUT, 256, 2, LP, SP>(a, s); break;
        case 3: launch_one<NIN, NOUT, 256, 4, LP, SP>(a, s); break;
        case 4: launch_one<NIN, NOUT, 512, 2, LP, SP>(a, s); break;
        case 5: launch_one<NIN, NOUT, 128, 3, LP, SP>(a, s); break;
        case 6: launch_one<NIN, NOUT, 256, 3, LP, SP>(a, s); break;
        case 7: launch_one<NIN, NOUT, 256, 5, LP, SP>(a, s); break;
        default: launch_one<NIN, NOUT, 256, 6, LP, SP>(a, s); break;
    }
}

template <int NIN, int NOUT>
static void launch_shape(int shape, const StreamArgs& a, hipStream_t s) {
    const int geo = shape % kNumGeo, pol = shape / kNumGeo;
    switch (pol) {
        case 0: launch_geo<NIN, NOUT, POL_NT, POL_NT>(geo, a, s); break;
        case 1: launch_geo<NIN, NOUT, POL_DEFAULT, POL_NT>(geo, a, s); break;
        case 2: launch_geo<NIN, NOUT, POL_NT, POL_SC1>(geo, a, s); break;
        case 3: launch_geo<NIN, NOUT, POL_DEFAULT, POL_SC1>(geo, a, s); break;
        default: launch_geo<NIN, NOUT, POL_NT, kGlobalNt>(geo, a, s); break;
    }
}

}  // namespace zl

using namespace zl;

extern "C" {

int hip_stream_ref_shapes(void) { return kNumShapes; }

int hip_stream_ref(int n_in, int n_out, const void* in0, const void* in1, void* out0, void* out1, int64_t bytes,
                   int shape, HipStream_t stream) {
    if (bytes <= 0) return 0;
    if (n_in < 1 || n_in > 2 || n_out < 1 || n_out > 2 || shape < 0 || shape >= kNumShapes || bytes % 16 ||
        !in0 || !out0 || (n_in == 2 && !in1) || (n_out == 2 && !out1) || !aligned16(in0) || !aligned16(out0) ||
        (n_in == 2 && !aligned16(in1)) || (n_out == 2 && !aligned16(out1)))
        return HIP_BRIDGE_EINVAL;
    if (bytes / 16 > 0xffffffffLL) return HIP_BRIDGE_EUNSUPPORTED;
    StreamArgs a{};
    a.in0 = (const uint8_t*)in0;
    a.in1 = (const uint8_t*)in1;
    a.out0 = (uint8_t*)out0;
    a.out1 = (uint8_t*)out1;
    a.nch = bytes / 16;
    const hipStream_t s = stream_of(stream);
    if (n_in == 1 && n_out == 1) launch_shape<1, 1>(shape, a, s);
    else if (n_in == 2 && n_out == 1) launch_shape<2, 1>(shape, a, s);
    else if (n_in == 1 && n_out == 2) launch_shape<1, 2>(shape, a, s);
    else launch_shape<2, 2>(shape, a, s);
    return (int)hipGetLastError();
}

int hip_stream_ref_copies(const void* src0, void* dst0, int64_t bytes0, const void* src1, void* dst1,
                          int64_t bytes1, const void* src2, void* dst2, int64_t bytes2, int interleave,
                          int shape, HipStream_t stream) {
    const void* src[3] = {src0, src1, src2};
    void* dst[3] = {dst0, dst1, dst2};
    const int64_t bytes[3] = {bytes0, bytes1, bytes2};
    if (shape < 0 || shape >= kNumShapes) return HIP_BRIDGE_EINVAL;
    StreamArgs a{};
    int64_t wgs = 0;
    for (int p = 0; p < 3; ++p) {
        if (bytes[p] < 0 || bytes[p] % 16) return HIP_BRIDGE_EINVAL;
        if (bytes[p] == 0) continue;
        if (!src[p] || !dst[p] || !aligned16(src[p]) || !aligned16(dst[p])) return HIP_BRIDGE_EINVAL;
        if (bytes[p] / 16 > 0xffffffffLL) return HIP_BRIDGE_EUNSUPPORTED;
        a.src[p] = (const uint8_t*)src[p];
        a.dst[p] = (uint8_t*)dst[p];
        a.pch[p] = bytes[p] / 16;
        wgs += cdiv(a.pch[p], (int64_t)64);  // the most workgroups any shape takes
    }
    if (wgs > 0xffffffffLL) return HIP_BRIDGE_EUNSUPPORTED;
    a.ilv = interleave != 0;
    launch_shape<0, 1>(shape, a, stream_of(stream));
    return (int)hipGetLastError();
}

}  // extern "C"
