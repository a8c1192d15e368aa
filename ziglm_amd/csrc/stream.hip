// Reference streaming kernel: the practical HBM ceiling of an op's byte mix. It reads n_in
// streams and writes n_out streams of `bytes` each (out_j[i] = in0[i] ^ in1[i], or in0[i]),
// so an op that reads R tensors and writes W tensors of one size can be set beside a kernel
// that moves exactly the same bytes and does nothing else. out0 may be in0 (a read-modify-
// write of one tensor in place, as the residual-stream updates x += ... do). Launch shapes
// combine threads per workgroup, 128-bit chunks per thread and the load / store cache
// policies the ops choose among (zl_common.h POL_*); the benchmark times each and takes the
// fastest as the ceiling of that size and mix.
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
};

// Store policy kGlobalNt: nt stores as global (per-lane address) stores, the form the norm
// kernels use (buffer nt stores are the other nt form).
constexpr int kGlobalNt = -1;

// U chunks per thread, consecutive by workgroup: chunk (block * U + u) * THREADS + thread.
template <int NIN, int NOUT, int THREADS, int U, int LP, int SP>
__global__ __launch_bounds__(THREADS) void k_stream(StreamArgs a) {
    const int64_t c0 = (int64_t)blockIdx.x * U * THREADS;
    const int64_t left = a.nch - c0;
    const uint32_t bytes = (uint32_t)(left < U * THREADS ? left : U * THREADS) * 16u;
    const auto r0 = buf_rsrc(a.in0 + c0 * 16, bytes);
    const auto r1 = buf_rsrc(NIN == 2 ? a.in1 + c0 * 16 : a.in0, NIN == 2 ? bytes : 0u);
    const auto w0 = buf_rsrc(a.out0 + c0 * 16, bytes);
    const auto w1 = buf_rsrc(NOUT == 2 ? a.out1 + c0 * 16 : a.out0, NOUT == 2 ? bytes : 0u);
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
                sts16(a.out0 + c0 * 16 + off, v);
                if constexpr (NOUT == 2) sts16(a.out1 + c0 * 16 + off, v);
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
    const int64_t grid = cdiv(a.nch, (int64_t)THREADS * U);
    k_stream<NIN, NOUT, THREADS, U, LP, SP><<<(unsigned)grid, THREADS, 0, s>>>(a);
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
    const StreamArgs a{(const uint8_t*)in0, (const uint8_t*)in1, (uint8_t*)out0, (uint8_t*)out1, bytes / 16};
    const hipStream_t s = stream_of(stream);
    if (n_in == 1 && n_out == 1) launch_shape<1, 1>(shape, a, s);
    else if (n_in == 2 && n_out == 1) launch_shape<2, 1>(shape, a, s);
    else if (n_in == 1 && n_out == 2) launch_shape<1, 2>(shape, a, s);
    else launch_shape<2, 2>(shape, a, s);
    return (int)hipGetLastError();
}

}  // extern "C"
