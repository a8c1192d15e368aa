// Reference streaming kernel: the practical HBM ceiling of an op's byte mix. It reads n_in
// streams and writes n_out streams of `bytes` each (out_j[i] = in0[i] ^ in1[i], or in0[i]),
// so an op that reads R tensors and writes W tensors of one size can be set beside a kernel
// that moves exactly the same bytes and does nothing else. Several launch shapes are built;
// the benchmark times each and takes the fastest as the ceiling of that size and mix.
//
// Every shape issues all of a thread's 128-bit loads before its first store, with the same
// nontemporal policy the ops use for single-use activations (zl_common.h lds16 / sts16).
#include "zl_common.h"
#include "zl_host.h"

namespace zl {

struct StreamArgs {
    const u32x4* in0;
    const u32x4* in1;
    u32x4* out0;
    u32x4* out1;
    int64_t nch;  // 16-byte chunks per stream
};

// U chunks per thread, consecutive by workgroup: chunk (block * U + u) * THREADS + thread.
template <int NIN, int NOUT, int THREADS, int U>
__global__ __launch_bounds__(THREADS) void k_stream(StreamArgs a) {
    u32x4 r0[U], r1[U];
    int64_t idx[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        idx[u] = ((int64_t)blockIdx.x * U + u) * THREADS + threadIdx.x;
        if (idx[u] < a.nch) {
            r0[u] = lds16(a.in0 + idx[u]);
            if constexpr (NIN == 2) r1[u] = lds16(a.in1 + idx[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (idx[u] < a.nch) {
            const u32x4 v = NIN == 2 ? (r0[u] ^ r1[u]) : r0[u];
            sts16(a.out0 + idx[u], v);
            if constexpr (NOUT == 2) sts16(a.out1 + idx[u], v);
        }
    }
}

struct Shape {
    int threads, unroll;
};
// The launch shapes the ceiling is the best of.
constexpr Shape kShapes[] = {{64, 1}, {128, 1}, {256, 1}, {256, 2}, {256, 4}, {512, 1}, {1024, 1}, {64, 4}};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);

template <int NIN, int NOUT, int THREADS, int U>
static void launch_one(const StreamArgs& a, hipStream_t s) {
    const int64_t grid = cdiv(a.nch, (int64_t)THREADS * U);
    k_stream<NIN, NOUT, THREADS, U><<<(unsigned)grid, THREADS, 0, s>>>(a);
}

template <int NIN, int NOUT>
static void launch_shape(int shape, const StreamArgs& a, hipStream_t s) {
    switch (shape) {
        case 0: launch_one<NIN, NOUT, 64, 1>(a, s); break;
        case 1: launch_one<NIN, NOUT, 128, 1>(a, s); break;
        case 2: launch_one<NIN, NOUT, 256, 1>(a, s); break;
        case 3: launch_one<NIN, NOUT, 256, 2>(a, s); break;
        case 4: launch_one<NIN, NOUT, 256, 4>(a, s); break;
        case 5: launch_one<NIN, NOUT, 512, 1>(a, s); break;
        case 6: launch_one<NIN, NOUT, 1024, 1>(a, s); break;
        default: launch_one<NIN, NOUT, 64, 4>(a, s); break;
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
    const StreamArgs a{(const u32x4*)in0, (const u32x4*)in1, (u32x4*)out0, (u32x4*)out1, bytes / 16};
    const hipStream_t s = stream_of(stream);
    if (n_in == 1 && n_out == 1) launch_shape<1, 1>(shape, a, s);
    else if (n_in == 2 && n_out == 1) launch_shape<2, 1>(shape, a, s);
    else if (n_in == 1 && n_out == 2) launch_shape<1, 2>(shape, a, s);
    else launch_shape<2, 2>(shape, a, s);
    return (int)hipGetLastError();
}

}  // extern "C"
