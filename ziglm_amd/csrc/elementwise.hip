// Elementwise ops: GeGLU (replaces cuda_bridge.cu:2247-2269), SwiGLU (2275-2291), tanh
// soft-cap (2319-2330), residual add and scale (2293-2317), the per-layer-embedding (PLE)
// gate and context fuse (2885-2937), and an out-of-place scale (scale 1: a kernel copy,
// which a captured graph replays like any other kernel).
//
// Streaming layout: one wave per workgroup, each thread owns U consecutive-by-wave 128-bit
// chunks (chunk = (block*U + u)*64 + thread), so every load/store instruction of a wave
// covers 1 KiB of contiguous memory; all loads of a thread are issued before any math.
// Elements that do not fill a whole chunk (n % E) are done by a scalar tail in block 0.
// Launch shape measured on MI355X for bf16 GeGLU (2048 x 10240 / 8192 x 21504): 64 threads
// and U = 1 take 20.2 / 155 us, against 22.1 / 169 us for 256 threads and U = 2, and against
// 21.2-23.7 / 166-187 us for a persistent grid of one-wave workgroups walking blocks of 64 or
// more chunks with the next block's loads in flight (4-32 waves per CU, 1-4 chunks per thread).
//
// GeGLU: out = gelu_tanh(gate) * up (math.zig:1119-1130) with the logistic form of GELU
// (zl_common.h gelu_fast). SwiGLU: out = silu(gate) * up (math.zig:1108-1117, silu_fast).
// Soft-cap: x = cap * tanh(x / cap) (model.zig:805-810) with the IEEE quotient x/cap
// (div_by_uniform) and tanh_fast. PLE context fuse (model.zig:525-535): ctx = (ctx + s) * c
// with c = f32(1/sqrt(2)), two roundings as the CPU's, or ctx = s.
#include "zl_common.h"
#include "zl_host.h"

namespace zl {

#ifndef ZL_EW_THREADS
#define ZL_EW_THREADS 64
#endif
#ifndef ZL_EW_UNROLL
#define ZL_EW_UNROLL 1
#endif
#ifndef ZL_EW_LP
#define ZL_EW_LP POL_NT
#endif
#ifndef ZL_EW_SP
#define ZL_EW_SP POL_NT
#endif
constexpr int kEwThreads = ZL_EW_THREADS;
constexpr int kEwUnroll = ZL_EW_UNROLL;
constexpr int kEwLP = ZL_EW_LP, kEwSP = ZL_EW_SP;  // load / store cache policy (zl_common.h POL_*)

enum EwOp { EW_GEGLU = 0, EW_SOFTCAP = 1, EW_ADD = 2, EW_SCALE = 3, EW_SWIGLU = 4, EW_PLE_FUSE = 5 };

// Ops with a second input stream.
template <int OP>
constexpr bool ew_two() { return OP == EW_GEGLU || OP == EW_ADD || OP == EW_SWIGLU || OP == EW_PLE_FUSE; }

struct EwArgs {
    const void* a;  // gate | x | x
    const void* b;  // up   | -  | residual
    void* out;
    int64_t n;
    float p0, p1;   // softcap: cap, 1/cap; scale: factor; PLE fuse: factor, 1 = add (0 = copy b)
};

template <int OP>
__device__ __forceinline__ float ew1(float a, float b, const EwArgs& args) {
    if constexpr (OP == EW_GEGLU) return gelu_fast(a) * b;
    else if constexpr (OP == EW_SOFTCAP) return args.p0 * tanh_fast(div_by_uniform(a, args.p0, args.p1));
    else if constexpr (OP == EW_ADD) return a + b;
    else if constexpr (OP == EW_SWIGLU) return silu_fast(a) * b;
    else if constexpr (OP == EW_PLE_FUSE) return args.p1 != 0.0f ? (a + b) * args.p0 : b;
    else return a * args.p0;
}

template <typename T, int OP>
__global__ __launch_bounds__(kEwThreads) void k_ew(EwArgs args) {
    using C = Chunk<T>;
    constexpr int E = C::E;
    constexpr bool kTwo = ew_two<OP>();
    const int64_t nch = args.n / E;
    const T* A = (const T*)args.a;
    const T* B = (const T*)args.b;
    T* O = (T*)args.out;
    // The workgroup's chunks through range-checked buffer resources (chunks past the end read
    // zeros and are not stored), with the streaming cache policies.
    const int64_t c0 = (int64_t)blockIdx.x * kEwUnroll * kEwThreads;
    const int64_t left = nch - c0;
    const uint32_t bytes = (uint32_t)(left < kEwUnroll * kEwThreads ? left : kEwUnroll * kEwThreads) * 16u;
    const auto rsa = buf_rsrc(A + c0 * E, bytes);
    const auto rsb = buf_rsrc(kTwo ? B + c0 * E : A, kTwo ? bytes : 0u);
    const auto rso = buf_rsrc(O + c0 * E, bytes);
    u32x4 ra[kEwUnroll], rb[kEwUnroll];
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        const uint32_t off = (uint32_t)(u * kEwThreads + threadIdx.x) * 16u;
        ra[u] = bldp<kEwLP>(rsa, off);
        if constexpr (kTwo) rb[u] = bldp<kEwLP>(rsb, off);
    }
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) {
        float x[E], y[E];
        C::unpack(ra[u], x);
        if constexpr (kTwo) C::unpack(rb[u], y);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = ew1<OP>(x[j], kTwo ? y[j] : 0.0f, args);
        bstp<kEwSP>(rso, (uint32_t)(u * kEwThreads + threadIdx.x) * 16u, C::pack(x));
    }
    // scalar tail
    const int64_t tail0 = nch * E;
    const int64_t ti = tail0 + (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
    if (blockIdx.x == 0 && ti < args.n) {
        float x, y = 0.0f;
        if constexpr (sizeof(T) == 4) {
            x = ((const float*)A)[ti];
            if constexpr (kTwo) y = ((const float*)B)[ti];
        } else {
            x = bf16_lo(((const uint16_t*)A)[ti]);
            if constexpr (kTwo) y = bf16_lo(((const uint16_t*)B)[ti]);
        }
        const float r = ew1<OP>(x, y, args);
        if constexpr (sizeof(T) == 4) ((float*)O)[ti] = r;
        else ((uint16_t*)O)[ti] = (uint16_t)(pack_bf16x2(r, 0.0f) & 0xffffu);
    }
}

// Unaligned buffers: one element per thread.
template <typename T, int OP>
__global__ __launch_bounds__(kEwThreads) void k_ew_scalar(EwArgs args) {
    constexpr bool kTwo = ew_two<OP>();
    const int64_t i = (int64_t)blockIdx.x * kEwThreads + threadIdx.x;
    if (i >= args.n) return;
    float x, y = 0.0f;
    if constexpr (sizeof(T) == 4) {
        x = ((const float*)args.a)[i];
        if constexpr (kTwo) y = ((const float*)args.b)[i];
    } else {
        x = bf16_lo(((const uint16_t*)args.a)[i]);
        if constexpr (kTwo) y = bf16_lo(((const uint16_t*)args.b)[i]);
    }
    const float r = ew1<OP>(x, y, args);
    if constexpr (sizeof(T) == 4) ((float*)args.out)[i] = r;
    else ((uint16_t*)args.out)[i] = (uint16_t)(pack_bf16x2(r, 0.0f) & 0xffffu);
}

template <typename T, int OP>
static void launch_ew_t(const EwArgs& a, hipStream_t s) {
    constexpr int E = Chunk<T>::E;
    constexpr bool kTwo = ew_two<OP>();
    const bool vec = aligned16(a.a) && aligned16(a.out) && (!kTwo || aligned16(a.b));
    if (vec) {
        const int64_t nch = a.n / E;
        int64_t grid = cdiv(nch, (int64_t)kEwThreads * kEwUnroll);
        if (grid < 1) grid = 1;  // the tail still needs block 0
        k_ew<T, OP><<<(unsigned)grid, kEwThreads, 0, s>>>(a);
    } else {
        k_ew_scalar<T, OP><<<(unsigned)cdiv(a.n, kEwThreads), kEwThreads, 0, s>>>(a);
    }
    check_launch();
}

template <int OP>
static void launch_ew(int dtype, const EwArgs& a, hipStream_t s) {
    if (a.n <= 0) return;
    if (!a.a || !a.out || (ew_two<OP>() && !a.b)) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    if (dtype == HIP_BRIDGE_F32) launch_ew_t<float, OP>(a, s);
    else if (dtype == HIP_BRIDGE_BF16) launch_ew_t<uint16_t, OP>(a, s);
    else set_error(HIP_BRIDGE_EUNSUPPORTED);
}

}  // namespace zl

using namespace zl;

extern "C" {

void hip_geglu_ex(int dtype, const void* gate, const void* up, void* out, int64_t n,
                  HipStream_t stream) {
    EwArgs a{gate, up, out, n, 0.0f, 0.0f};
    launch_ew<EW_GEGLU>(dtype, a, stream_of(stream));
}

void hip_tanh_softcap_ex(int dtype, void* x, float cap, int64_t n, HipStream_t stream) {
    // 1/cap rounded once (IEEE f32 divide on the host) for the correctly rounded quotient.
    EwArgs a{x, nullptr, x, n, cap, 1.0f / cap};
    launch_ew<EW_SOFTCAP>(dtype, a, stream_of(stream));
}

void hip_geglu(const float* gate, const float* up, float* out, int n, HipStream_t stream) {
    hip_geglu_ex(HIP_BRIDGE_F32, gate, up, out, n, stream);
}

void hip_tanh_softcap(float* x, float cap, int n, HipStream_t stream) {
    hip_tanh_softcap_ex(HIP_BRIDGE_F32, x, cap, n, stream);
}

void hip_add(float* x, const float* residual, int n, HipStream_t stream) {
    EwArgs a{x, residual, x, n, 0.0f, 0.0f};
    launch_ew<EW_ADD>(HIP_BRIDGE_F32, a, stream_of(stream));
}

void hip_scale(float* x, float scale, int n, HipStream_t stream) {
    EwArgs a{x, nullptr, x, n, scale, 0.0f};
    launch_ew<EW_SCALE>(HIP_BRIDGE_F32, a, stream_of(stream));
}

void hip_scale_ex(int dtype, const void* x, float scale, void* out, int64_t n, HipStream_t stream) {
    EwArgs a{x, nullptr, out, n, scale, 0.0f};
    launch_ew<EW_SCALE>(dtype, a, stream_of(stream));
}

void hip_swiglu_ex(int dtype, const void* gate, const void* up, void* out, int64_t n,
                   HipStream_t stream) {
    EwArgs a{gate, up, out, n, 0.0f, 0.0f};
    launch_ew<EW_SWIGLU>(dtype, a, stream_of(stream));
}

void hip_swiglu(const float* gate, const float* up, float* out, int n, HipStream_t stream) {
    hip_swiglu_ex(HIP_BRIDGE_F32, gate, up, out, n, stream);
}

// ple_buf = gelu_tanh(gate) * slice: the GeGLU kernel with the slice as the up operand
// (model.zig:765-768 computes slice * gelu(gate); the product commutes exactly).
void hip_ple_gate_gelu(const float* ple_gate_in, const float* ple_slice, float* ple_buf_out,
                       int ple_dim, HipStream_t stream) {
    hip_geglu_ex(HIP_BRIDGE_F32, ple_gate_in, ple_slice, ple_buf_out, ple_dim, stream);
}

void hip_ple_ctx_fuse(float* ctx_ple_buf, const float* ctx_scratch, int n, int add_token_embd,
                      HipStream_t stream) {
    // 1/sqrt(2) rounded to f32 (0x3F3504F3), the value of model.zig:528's
    // `1.0 / @sqrt(2.0)` coerced to f32.
    EwArgs a{ctx_ple_buf, ctx_scratch, ctx_ple_buf, n, 0.70710677f, add_token_embd ? 1.0f : 0.0f};
    launch_ew<EW_PLE_FUSE>(HIP_BRIDGE_F32, a, stream_of(stream));
}

}  // extern "C"
