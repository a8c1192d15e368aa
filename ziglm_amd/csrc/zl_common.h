// Device helpers shared by the hip_bridge kernels (gfx950, wave64).
//
// All sources are compiled with -ffp-contract=off: a*b+c is never fused implicitly, so the
// f32 expressions that mirror ziglm's CPU arithmetic round exactly as written. Where a
// kernel wants an FMA (sums of squares, polynomial evaluation) it calls fmaf explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zl {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---- bf16 <-> f32 ------------------------------------------------------------------
// bf16 is stored as uint16 bit patterns; a 32-bit word holds elements (2j, 2j+1) in its
// (low, high) halves (little endian).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even of two f32 values to bf16 (v_cvt_pk_bf16_f32 on gfx950). For every
// non-NaN input this equals ziglm's quant.f32ToBf16 ((bits + 0x7FFF + lsb) >> 16); NaN inputs
// stay NaN here, where the reference formula can carry a NaN payload into +-Inf.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// ---- 16-byte chunk <-> f32 lanes ---------------------------------------------------
// A "chunk" is one 128-bit load: 4 f32 or 8 bf16 elements.
template <typename T> struct Chunk;
template <> struct Chunk<float> {
    static constexpr int E = 4;
    __device__ static __forceinline__ void unpack(const u32x4& r, float* v) {
        v[0] = __uint_as_float(r.x);
        v[1] = __uint_as_float(r.y);
        v[2] = __uint_as_float(r.z);
        v[3] = __uint_as_float(r.w);
    }
    __device__ static __forceinline__ u32x4 pack(const float* v) {
        u32x4 r;
        r.x = __float_as_uint(v[0]);
        r.y = __float_as_uint(v[1]);
        r.z = __float_as_uint(v[2]);
        r.w = __float_as_uint(v[3]);
        return r;
    }
};
template <> struct Chunk<uint16_t> {
    static constexpr int E = 8;
    __device__ static __forceinline__ void unpack(const u32x4& r, float* v) {
        v[0] = bf16_lo(r.x);
        v[1] = bf16_hi(r.x);
        v[2] = bf16_lo(r.y);
        v[3] = bf16_hi(r.y);
        v[4] = bf16_lo(r.z);
        v[5] = bf16_hi(r.z);
        v[6] = bf16_lo(r.w);
        v[7] = bf16_hi(r.w);
    }
    __device__ static __forceinline__ u32x4 pack(const float* v) {
        u32x4 r;
        r.x = pack_bf16x2(v[0], v[1]);
        r.y = pack_bf16x2(v[2], v[3]);
        r.z = pack_bf16x2(v[4], v[5]);
        r.w = pack_bf16x2(v[6], v[7]);
        return r;
    }
};

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// Streaming (single-use) activations: nontemporal 128-bit loads and stores (the "nt" cache
// policy: no retention in L2 for data read or written exactly once). Measured on MI355X
// for GeGLU-shaped traffic: +8% bandwidth at 126 MB, +7% at 1 GB.
#ifndef ZL_STREAM_NT
#define ZL_STREAM_NT 1
#endif
__device__ __forceinline__ u32x4 lds16(const void* p) {
#if ZL_STREAM_NT
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#else
    return *reinterpret_cast<const u32x4*>(p);
#endif
}
__device__ __forceinline__ void sts16(void* p, const u32x4& v) {
#if ZL_STREAM_NT
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
#else
    *reinterpret_cast<u32x4*>(p) = v;
#endif
}
__device__ __forceinline__ f32x4 ldf4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
// A wave-uniform global pointer held in scalar registers and opaque to the optimiser, so
// that a per-lane choice among several such pointers stays a register select (the asm is
// not volatile and touches no memory, so loads around it keep their scalar / global forms).
template <typename P>
__device__ __forceinline__ P* sreg(P* p) {
    typedef __attribute__((address_space(1))) P* GP;
    uint64_t v = (uint64_t)p;
    asm("" : "+s"(v));
    return (P*)(GP)v;
}

// Range-checked loads through a buffer resource over [base, base + bytes): a raw buffer load
// at a byte offset past the end returns zeros and makes no memory access (CDNA buffer range
// checking), so lanes whose chunk lies outside a row need no branch around their load. A
// conditional load makes the compiler wait for it before the next one is issued (the value
// is merged at the branch's end), one memory round trip per chunk; these keep every load of
// a row in flight together. Word 3 of the resource is the gfx9-family raw-buffer format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes at `off`; nt: the streaming (nontemporal) policy of lds16.
__device__ __forceinline__ u32x4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, ZL_STREAM_NT ? 2 : 0));
}
__device__ __forceinline__ f32x4 bldf4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Cache policy of a buffer access (the instruction's cache-policy bits on gfx950): bit 0 sc0,
// bit 1 nt (streaming: not retained), bit 4 sc1 (for stores, sc1 alone is device scope). The
// streaming kernels take their load / store policy as compile-time constants; measured on
// MI355X with every op's inputs rotated past the Infinity Cache, nt loads and nt stores are
// the fastest for each of them (2048 x 2560 bf16: norm + add with default-policy loads 6.55
// -> 8.8 us; 4096 x 2560 gathers with sc1 or default-policy stores 8.7 -> 15.0-15.4 us for
// Q4_0). The reference streaming kernel (stream.hip), whose best shape defines an op's
// ceiling, also tries default-policy loads and sc1 stores, which a plain stream of some
// byte mixes prefers.
enum : int { POL_DEFAULT = 0, POL_SC0 = 1, POL_NT = 2, POL_SC1 = 16 };
template <int POL>
__device__ __forceinline__ u32x4 bldp(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL));
}
template <int POL>
__device__ __forceinline__ void bstp(__amdgpu_buffer_rsrc_t r, uint32_t off, const u32x4& v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, POL);
}
// A 128-bit store at byte offset `off` of a row (base `p`, range-checked resource `r` over
// the same row) with policy POL: POL_NT as a global nontemporal store (measured faster than
// the buffer form for the norm kernels: 2048 x 2560 bf16 norm + add + norm 8.60 -> 8.26 us),
// other policies as buffer stores.
template <int POL>
__device__ __forceinline__ void strow16(void* p, __amdgpu_buffer_rsrc_t r, uint32_t off, const u32x4& v) {
    if constexpr (POL == POL_NT) sts16((uint8_t*)p + off, v);
    else bstp<POL>(r, off, v);
}
// Global (per-lane address) 128-bit accesses with the nt policy or the default one.
template <bool NT>
__device__ __forceinline__ u32x4 ldg16(const void* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else return *reinterpret_cast<const u32x4*>(p);
}
template <bool NT>
__device__ __forceinline__ void stg16(void* p, const u32x4& v) {
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
    else *reinterpret_cast<u32x4*>(p) = v;
}

// ---- lane-group reductions -----------------------------------------------------------
// Sum over aligned groups of G lanes (G a power of two <= 64); every lane of a group gets
// the bit-identical group total (each step adds a pair in the same order on both sides).
// Within a 16-lane row: DPP quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror.
// Across rows: gfx950 v_permlane16_swap / v_permlane32_swap, whose two results are this
// lane's row (half) and its partner's, so their sum is the pair total. The second operand
// goes through an identity DPP move first: the compiler folds swap(x, x) into (x, x), which
// is wrong for these partial-row swaps.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "group size");
    if constexpr (G >= 2) v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (G >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (G >= 8) v += dpp<0x141>(v);  // row_half_mirror
    if constexpr (G >= 16) v += dpp<0x140>(v); // row_mirror
    if constexpr (G >= 32) {
        const unsigned a = __builtin_bit_cast(unsigned, v);
        const unsigned b = __builtin_bit_cast(unsigned, dpp<0xE4>(v));  // identity move
        const auto p = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        v = __builtin_bit_cast(float, (unsigned)p[0]) + __builtin_bit_cast(float, (unsigned)p[1]);
    }
    if constexpr (G >= 64) {
        const unsigned a = __builtin_bit_cast(unsigned, v);
        const unsigned b = __builtin_bit_cast(unsigned, dpp<0xE4>(v));
        const auto p = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        v = __builtin_bit_cast(float, (unsigned)p[0]) + __builtin_bit_cast(float, (unsigned)p[1]);
    }
    return v;
}

// ---- RMSNorm scalar: inv = 1.0 / sqrt(mean + eps) (math.zig:894-895) --------------------
// sqrtf and '/' are the correctly rounded IEEE operations under hipcc's defaults
// (-fhip-fp32-correctly-rounded-divide-sqrt), the same as Zig's @sqrt and '/'.
__device__ __forceinline__ float rms_inv(float sum_sq, int n, float eps) {
    float mean = sum_sq / (float)n;
    return 1.0f / sqrtf(mean + eps);
}
// The same with the hardware reciprocal square root for 1/sqrt (within 1 ulp of the IEEE
// sqrt and divide above, ~20 instructions shorter): the row kernels whose arithmetic is
// exposed at prefill sizes take it.
__device__ __forceinline__ float rms_inv_hw(float sum_sq, int n, float eps) {
    return __builtin_amdgcn_rsqf(sum_sq / (float)n + eps);
}

// Norm weights: raw 128-bit loads issued early (load_w), turned into the per-element factor
// 1 + w, w, or 1 (no weight) only where used (w_factor), so that no wait on the weight loads
// sits between the activation loads and independent work. Multiplying by 1.0 is exact, so
// (x*inv)*1 equals the reference's no-scale x*inv bit for bit.
template <int E>
__device__ __forceinline__ void load_w(const float* w, int64_t e0, bool has_w, float* f) {
    if (has_w) {
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            const f32x4 v = ldf4(w + e0 + 4 * q);
            f[4 * q + 0] = v.x;
            f[4 * q + 1] = v.y;
            f[4 * q + 2] = v.z;
            f[4 * q + 3] = v.w;
        }
    }
}
// The same from a range-checked resource (a weight-less resource reads zeros, unused).
template <int E>
__device__ __forceinline__ void load_wb(__amdgpu_buffer_rsrc_t r, uint32_t off, float* f) {
#pragma unroll
    for (int q = 0; q < E / 4; ++q) {
        const f32x4 v = bldf4(r, off + 16u * q);
        f[4 * q + 0] = v.x;
        f[4 * q + 1] = v.y;
        f[4 * q + 2] = v.z;
        f[4 * q + 3] = v.w;
    }
}
__device__ __forceinline__ float w_factor(float w, bool has_w, int uo) {
    return has_w ? (uo ? 1.0f + w : w) : 1.0f;
}

// RoPE denominator D_i = f32(base^(f32(2i)/f32(eff))) evaluated in double precision as
// exp2(e_i * log2(base)), with log2(base) computed once on the host (double). The double
// result is within ~1e-15 relative of the exact power, so its f32 rounding equals the
// oracle's f32(pow(base, e_i)) except within ~1e-15 of an f32 rounding tie (the GPU parity
// tests check RoPE outputs bit for bit). Computed per lane, no memory access.
__device__ __forceinline__ float rope_denom(int i, int eff, double log2_base) {
    const float e = (float)(2 * i) / (float)eff;
    return (float)exp2((double)e * log2_base);
}

// cos and sin of a RoPE angle theta = pos / D_i (f32). theta = k * pi/2 + r with
// k = rint(theta * 2/pi) and r = theta - k * pi/2 in double precision, pi/2 as a two-double
// sum, so r is exact to about 2^-53 for |theta| < 2^21 (positions up to ~3 million at
// D_0 = 1); then, with z = r^2 and |r| <= pi/4,
//   sin r = r + (r z) P(z),  cos r = (1 - z/2) + z^2 Q(z),
// P and Q quadratics fitted in relative error on [0, pi/4] (f32 evaluation: at most 0.7 ulp
// for sin, 1.3 ulp for cos), and k mod 4 maps (sin r, cos r) to (sin theta, cos theta).
// No memory operand and few registers, unlike the library sincos with its large-argument path.
__device__ __forceinline__ void rope_sincos(float theta, float* sn, float* cs) {
    const double t = (double)theta;
    const double k = rint(t * 0.63661977236758134);
    double rd = fma(-k, 1.5707963267948966, t);
    rd = fma(-k, 6.123233995736766e-17, rd);
    const float r = (float)rd;
    const float z = r * r;
    float ps = fmaf(z, -1.951538579305634e-4f, 8.332161232829094e-3f);
    ps = fmaf(z, ps, -1.6666655242443085e-1f);
    const float sr = fmaf(r * z, ps, r);
    float pc = fmaf(z, 2.4433236831100658e-5f, -1.3887316454201937e-3f);
    pc = fmaf(z, pc, 4.166664555668831e-2f);
    const float cr = fmaf(z * z, pc, 1.0f - 0.5f * z);
    const int q = (int)(int64_t)k & 3;
    float s = (q & 1) ? cr : sr;
    float c = (q & 1) ? sr : cr;
    if (q == 1 || q == 2) c = -c;
    if (q >= 2) s = -s;
    *sn = s;
    *cs = c;
}

// ---- tanh / GELU / soft-cap ------------------------------------------------------------
// Kernel tanh (a fast formulation, not the oracle's musl algorithm; both are accurate to a
// few ulp, so they agree within the tolerances the tests state):
//   |x| < 0.625: tanh(x) = x - x^3 q(x^2), q a degree-4 polynomial fitted (Lawson-weighted
//                least squares in relative error) on [0, 0.625]; <= 0.7 ulp in f32.
//   otherwise:   1 - 2/(exp(2|x|) + 1) with the hardware exp2 and reciprocal (a few ulp),
//                sign restored; exp2 overflows to +inf for |x| > 44, giving exactly +-1.
__device__ __forceinline__ float tanh_fast(float x) {
    const float ax = fabsf(x);
    const float x2 = x * x;
    float q = fmaf(x2, 0.005704984534531832f, -0.02063908614218235f);
    q = fmaf(x2, q, 0.05373971536755562f);
    q = fmaf(x2, q, -0.13331441581249237f);
    q = fmaf(x2, q, 0.3333328068256378f);
    const float small = fmaf(-x * x2, q, x);
    const float e = __builtin_amdgcn_exp2f(ax * 2.885390043258667f);  // exp(2|x|)
    const float big = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
    return ax < 0.625f ? small : copysignf(big, x);
}

// GELU, tanh approximation (math.zig:1119-1123), in the algebraically equal logistic form
//   0.5 x (1 + tanh(z)) = x / (1 + exp(-2z)),  z = 0.7978845608 (x + 0.044715 x^3),
// with -2z*log2(e) = x (A + B x^2), A = -2*0.7978845608*log2(e), B = 0.044715*A.
// No cancellation: relative error a few ulp everywhere. The reference's own 1 + tanh(z)
// loses up to ~2^-23 absolute for z << 0, which is what the tests' absolute floor covers.
// x -> -inf: exp2 -> +inf, rcp -> 0, result -0 (the reference gives 0.5x*0 = -0 too).
__device__ __forceinline__ float gelu_fast(float x) {
    const float x2 = x * x;
    const float y = x * fmaf(x2, -0.10294324159622192f, -2.302208185195923f);
    const float e = __builtin_amdgcn_exp2f(y);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// SiLU x / (1 + exp(-x)) (math.zig:1108-1110). exp(-x) = 2^y with y = -x*log2(e): the
// rounding error of y (FMA residual plus the low part of log2(e)) is folded back in to first
// order, so the exponential is accurate to ~2 ulp for every |x| (a plain exp2 of the rounded
// product loses up to |x|*2^-24 relative); the quotient is rcp plus one Newton step. exp(-x)
// overflowing (x < -88.7) gives x / inf = -0, as the CPU's division does.
__device__ __forceinline__ float silu_fast(float x) {
    const float nx = -x;
    const float y = nx * 1.44269502f;                                // RN(-x * log2 e)
    const float dy = fmaf(nx, 1.44269502f, -y) + nx * 1.92596299e-8f;  // -x*log2(e) - y
    const float e0 = __builtin_amdgcn_exp2f(y);
    const float e = fmaf(e0, dy * 0.693147181f, e0);
    const float d = 1.0f + e;
    const float r = __builtin_amdgcn_rcpf(d);
    const float q = x * r;
    const float qc = fmaf(fmaf(-d, q, x), r, q);
    return (__builtin_isinf(e0) || __builtin_isinf(e)) ? copysignf(0.0f, x) : qc;
}

// Correctly rounded x / b for a divisor b shared by all lanes, given rb = RN(1/b) computed on
// the host: q0 = x*rb, r = x - b*q0 (exact by FMA), q = q0 + r*rb (Markstein's correction;
// valid when no intermediate over/underflows, which holds for |x| < 2^100 and
// 2^-100 < |b| < 2^100). Equals the IEEE quotient the reference computes.
__device__ __forceinline__ float div_by_uniform(float x, float b, float rb) {
    const float q0 = x * rb;
    const float r = fmaf(-b, q0, x);
    return fmaf(r, rb, q0);
}

}  // namespace zl
