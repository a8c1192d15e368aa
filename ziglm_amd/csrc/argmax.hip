// Greedy token selection on the device (replaces cuda_bridge.cu:2943-3077 cuda_argmax)
// with ziglm's CPU definition (sampler.zig:158-170 sampleGreedy), which the decode loop
// uses: index 0 (the pad token) is never chosen; the result is the first index of the
// greatest value from index 1 on; NaN never compares greater, so a NaN at index 1 is kept
// and NaNs elsewhere are skipped; n <= 1 gives 0.
//
// Two stages, no atomics: kArgmaxBlocks workgroups each reduce a contiguous range to
// (value, index) with "greater, or equal and smaller index" (NaNs skipped) and store it in a
// device-global partial array; one workgroup then reduces the partials in order and writes
// the index. The partial arrays are referenced only from device code. As with the
// reference's global scratch, concurrent calls on different streams race on them.
#include <algorithm>

#include "zl_common.h"
#include "zl_host.h"

namespace zl {

constexpr int kArgmaxBlocks = 512;
constexpr int kArgmaxThreads = 256;

__device__ float g_argmax_val[kArgmaxBlocks];
__device__ uint32_t g_argmax_idx[kArgmaxBlocks];

struct Best {
    float v;
    uint32_t i;  // UINT32_MAX: none yet
};

// a better than b: greater value, or equal value and smaller index (a real index beats none).
__device__ __forceinline__ bool better(const Best& a, const Best& b) {
    if (a.i == UINT32_MAX) return false;
    if (b.i == UINT32_MAX) return true;
    return a.v > b.v || (a.v == b.v && a.i < b.i);
}

__device__ __forceinline__ Best wave_best(Best x) {
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        Best y;
        y.v = __shfl_xor(x.v, o);
        y.i = __shfl_xor(x.i, o);
        if (better(y, x)) x = y;
    }
    return x;
}

__device__ __forceinline__ Best block_best(Best x, Best* s) {
    x = wave_best(x);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = x;
    __syncthreads();
    Best r = s[0];
#pragma unroll
    for (int w = 1; w < kArgmaxThreads / kWave; ++w)
        if (better(s[w], r)) r = s[w];
    return r;
}

// Stage 1: workgroup b reduces indices [1 + b*span, 1 + (b+1)*span) of [1, n).
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_partial(const float* __restrict__ x, int64_t n,
                                                                   int64_t span) {
    __shared__ Best s[kArgmaxThreads / kWave];
    const int64_t lo = 1 + (int64_t)blockIdx.x * span;
    const int64_t hi = min(n, lo + span);
    Best b{0.0f, UINT32_MAX};
    for (int64_t i = lo + threadIdx.x; i < hi; i += kArgmaxThreads) {
        const float v = x[i];
        // NaN is never greater (sampler.zig:165): skip it
        if (v == v) {
            const Best c{v, (uint32_t)i};
            if (better(c, b)) b = c;
        }
    }
    b = block_best(b, s);
    if (threadIdx.x == 0) {
        g_argmax_val[blockIdx.x] = b.v;
        g_argmax_idx[blockIdx.x] = b.i;
    }
}

// Stage 2: reduce the partials; the CPU keeps index 1 when logits[1] is NaN.
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_final(const float* __restrict__ x, int nblocks,
                                                                 uint32_t* __restrict__ out) {
    __shared__ Best s[kArgmaxThreads / kWave];
    Best b{0.0f, UINT32_MAX};
    for (int j = threadIdx.x; j < nblocks; j += kArgmaxThreads) {
        const Best c{g_argmax_val[j], g_argmax_idx[j]};
        if (better(c, b)) b = c;
    }
    b = block_best(b, s);
    if (threadIdx.x == 0) {
        const float x1 = x[1];
        *out = (x1 != x1 || b.i == UINT32_MAX) ? 1u : b.i;
    }
}

}  // namespace zl

using namespace zl;

extern "C" void hip_argmax(const float* logits, int n, unsigned int* out_idx, HipStream_t stream) {
    if (!logits || !out_idx) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    hipStream_t s = stream_of(stream);
    if (n <= 1) {
        // sampleGreedy returns 0; write it with a one-thread kernel (stream-ordered, no memset)
        hip_fill_u8(out_idx, 0, sizeof(unsigned int), stream);
        return;
    }
    const int64_t m = (int64_t)n - 1;  // indices 1 .. n-1
    const int64_t span = std::max<int64_t>(kArgmaxThreads * 4, cdiv(m, kArgmaxBlocks));
    const int blocks = (int)cdiv(m, span);
    k_argmax_partial<<<blocks, kArgmaxThreads, 0, s>>>(logits, n, span);
    k_argmax_final<<<1, kArgmaxThreads, 0, s>>>(logits, blocks, out_idx);
    check_launch();
}
