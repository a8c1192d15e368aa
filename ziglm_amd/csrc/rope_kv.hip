// Fused attention prologue: per-head RMSNorm of Q and K (and the Gemma-4 no-scale norm of
// V), half-split RoPE, and the KV-cache append, in one launch. Replaces cuda_bridge.cu
// k_rmsnorm_batched (1504-1553) x3, k_rope{,_ind,_batched} (2070-2245) and
// k_kv_cache_put{,_ind,_batched} (2336-2460), which in the reference are six launches and
// five extra HBM round trips of Q and K.
//
// Numerics follow ziglm's CPU path:
//   norm  math.zig:850-988 ((x*inv)*(1+w); inv = 1.0/sqrt(mean + eps), in the fused kernel
//         by the hardware reciprocal square root, within 1 ulp of it);
//   RoPE  math.zig:1019-1078 .normal: pairs (i, i + r/2); theta = (f32(pos)*freq_scale)/D_i
//         (IEEE f32 division); D_i = f32(pow(base, f32(2i)/f32(r))), the oracle's value (in
//         the fused kernel evaluated per lane in double precision, rope_denom; in the generic
//         kernel computed on the host and passed in the arguments); cos/sin by rope_sincos,
//         within 1.3 ulp of the correctly rounded values the oracle uses; the rotation is
//         v0*c - v1*s, v0*s + v1*c with no FMA;
//   KV    kv_cache_put (cuda_bridge.cu:2349; kv_cache.zig:63-85): row-contiguous copy.
//
// Fast path (head_dim in {64, 128, 256, 512}, rotary_dim/2 a multiple of E, 16-byte aligned
// buffers): LH = head_dim/(2E) lanes per head (E = elements per 128-bit chunk), 64/LH heads
// per wave, one workgroup per token (per token and pass of head rows when there are few
// tokens). Each lane holds two chunks of a head row: with R = rotary_dim/(2E), lanes l < R
// chunks l and l + R (elements i and i + rotary_dim/2, so every RoPE pair is inside one
// lane), the others two adjacent chunks of the unrotated tail; with full rotary that is
// chunk l and chunk l + LH. The norm statistic is an LH-lane butterfly. The token's cos/sin
// table (rotary_dim/2 entries) is computed once in LDS while the first head's loads are in
// flight; its denominators are evaluated per lane (rope_denom) and its cos/sin by
// rope_sincos, so that phase has no memory operand to wait for. Measured at c2 (2048 tokens,
// 8/4 heads x 256, bf16): 6.7 us, against 6.6 us for a plain stream of the same bytes. Not
// taken: a variant without the workgroup barrier (each wave computing its own angles and
// staging its own weights in LDS, 8.6-9.0 us when the kernel took 7.9); each lane loading
// the norm weights of its own chunks into registers instead of the LDS staging (7.3 us, the
// weight loads as many load instructions as the rows'); one or four tokens per workgroup
// (8.9 / 8.7 us); a persistent form whose workgroups walk the tokens with the next token's
// head rows in flight (as the row norms do at 8192 rows), bit-equal to this one: Gemma-27B
// heads at 8192 tokens 44.8 -> 48.7 us at its best grid (3-4 workgroups per CU; 2, 6 and 8
// were slower still).
// Generic path (other head sizes up to 512, any alignment): one wave per head row (Q, K or V
// head), head staged in LDS, four rows per workgroup.
#include <math.h>
#include <algorithm>
#include <string.h>

#include "zl_common.h"
#include "zl_host.h"

namespace zl {

constexpr int kMaxHalf = 256;  // head_dim <= 512
// A head row of zeros that loads with nothing to read point at (k_qk_fused issues every
// load of its first pass on every path).
__device__ __attribute__((aligned(16))) float g_qk_pad_row[2 * kMaxHalf];

#ifndef ZL_QK_TPW
#define ZL_QK_TPW 2
#endif
// launches of at most this many tokens take a workgroup per token and pass of head rows (for
// all token counts: Gemma-27B heads at 8192 tokens 43.9 -> 46.3 us, so not for prefill)
#ifndef ZL_QK_GY_TOKENS
#define ZL_QK_GY_TOKENS 64
#endif
#ifndef ZL_QK_NP2
#define ZL_QK_NP2 0
#endif
#ifndef ZL_QK_TPW_MIN
#define ZL_QK_TPW_MIN 1024
#endif

struct RopeTab {
    float denom[kMaxHalf];
};


struct QkArgs {
    void* q;
    const void* k;
    const void* v;
    const float* wq;
    const float* wk;
    void* kdst;
    void* vdst;
    int64_t cache_rows;     // rows available in kdst/vdst (0: not checked)
    int64_t row_stride;     // elements between destination rows
    const int32_t* pos;     // device positions (pos_mode 1, 2)
    int pos_mode;           // 0: pos_base + t; 1: pos[t]; 2: pos[0] + t
    int pos_base;
    const int64_t* slot;    // device cache rows (slot_mode 1)
    int slot_mode;          // 0: layer_base + position, position in [0, max_seq); 1: slot[t]; 2: row t
    int64_t layer_base;
    int max_seq;
    int n_tokens, nh, nkv, D, half;
    int do_qnorm, do_knorm, v_norm, do_rope, uo;
    float freq_scale, eps;
    double log2_base;
};

__device__ __forceinline__ int token_pos(const QkArgs& a, int t) {
    return a.pos_mode == 0 ? a.pos_base + t : a.pos_mode == 1 ? a.pos[t] : a.pos[0] + t;
}

// Destination row of token t in kdst/vdst, or -1 when it must not be written.
__device__ __forceinline__ int64_t token_row(const QkArgs& a, int t, int p) {
    int64_t row;
    if (a.slot_mode == 0) {
        if (p < 0 || p >= a.max_seq) return -1;
        row = a.layer_base + p;
    } else if (a.slot_mode == 1) {
        row = a.slot[t];
    } else {
        return t;
    }
    if (row < 0 || (a.cache_rows > 0 && row >= a.cache_rows)) return -1;
    return row;
}

// cos/sin of theta_i = pos_f / D_i for i < half, into LDS.
__device__ __forceinline__ void fill_cos_sin(const RopeTab& tab, float pos_f, int half, float* s_cos,
                                             float* s_sin) {
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        rope_sincos(pos_f / tab.denom[i], &s_sin[i], &s_cos[i]);
    }
}

// Cache policy of the head-row loads and stores (nt or the default; the rows are addressed
// per lane, so the buffer-only policies do not apply).
#ifndef ZL_QK_LD_NT
#define ZL_QK_LD_NT 1
#endif
#ifndef ZL_QK_ST_NT
#define ZL_QK_ST_NT 1
#endif
constexpr bool kQkLdNt = ZL_QK_LD_NT, kQkStNt = ZL_QK_ST_NT;

// Head rows one pass of a k_qk_fused workgroup takes (4 waves of 64 / LH heads).
template <typename T, int D>
__host__ __device__ constexpr int qk_slots() {
    return 4 * (kWave / (D / 2 / Chunk<T>::E));
}

template <typename T, int D, int TPW, int NP = 1>
__global__ __launch_bounds__(256) void k_qk_fused(QkArgs a) {
    using C = Chunk<T>;
    constexpr int E = C::E;
    constexpr int HALF = D / 2;
    constexpr int LH = HALF / E;  // lanes per head
    constexpr int G = kWave / LH; // heads per wave
    static_assert(LH >= 1 && LH <= kWave && (LH & (LH - 1)) == 0, "bad head layout");
    __shared__ float s_cos[TPW][HALF], s_sin[TPW][HALF];
    __shared__ __attribute__((aligned(16))) float s_wq[D], s_wk[D];

    const int tb = blockIdx.x * TPW;  // the workgroup's first token (TPW tokens each)
    const int lane = threadIdx.x & 63;
    const int hl = lane & (LH - 1);
    constexpr int kSlots = qk_slots<T, D>();
    // Workgroup (x, y) takes head rows y * kSlots + slot, + kSlots * gridDim.y, ... of each
    // of its tokens.
    const int gslot = blockIdx.y * kSlots + (threadIdx.x >> 6) * G + lane / LH;
    const int hstep = kSlots * gridDim.y;
    // The lane's two chunks of a head row (E elements each): with rotary width r = 2 * half,
    // lanes [0, R) (R = half / E) hold the RoPE pair (hl, hl + R) -- elements i and i + half --
    // and the others two adjacent chunks of the unrotated tail [r, D).
    const int R = a.half / E;
    const int c0 = hl < R ? hl : 2 * R + 2 * (hl - R);
    const int c1 = hl < R ? hl + R : c0 + 1;
    const int nq = a.q ? a.nh : 0;
    const int HR = a.nh + 2 * a.nkv;
    const bool has_wq = a.wq != nullptr, has_wk = a.wk != nullptr;
    // The base pointers as register values: a per-lane choice among them is then a select,
    // not a per-lane load of the chosen argument (which the compiler otherwise emits, with a
    // wait for it ahead of the row loads), nor, for the weights, a loop over the distinct
    // buffer resources of a wave.
    const T* const qb = sreg((const T*)a.q);
    const T* const kb = sreg((const T*)a.k);
    const T* const vb = sreg((const T*)a.v);
    const float* const wqb = sreg(a.wq);
    const float* const wkb = sreg(a.wk);

    // Head rows: [0, nh) Q, [nh, nh+nkv) K, [nh+nkv, nh+2nkv) V.
    auto src_of = [&](int hr, int t) -> const T* {
        if (hr < a.nh) return qb + ((int64_t)t * a.nh + hr) * D;
        if (hr < a.nh + a.nkv) return kb + ((int64_t)t * a.nkv + (hr - a.nh)) * D;
        return vb + ((int64_t)t * a.nkv + (hr - a.nh - a.nkv)) * D;
    };
    // Source rows exist for every token of the launch (whether a K / V row is then written
    // depends on its destination, known only after the position and slot reads below).
    auto readable = [&](int hr, int t) -> bool {
        if (t >= a.n_tokens) return false;
        if (hr < a.nh) return nq > 0;
        if (hr < a.nh + a.nkv) return a.k != nullptr;
        return a.v != nullptr;
    };
    // Issue order. First the norm weights, staged once per workgroup in LDS as factors (1+w),
    // w or 1 (threads [0, D/4) stage wq, [D/4, D/2) wk, one f32x4 each; L2 hits after the
    // first workgroups): the barrier below waits for them, and loads complete in issue order.
    // Then the first head row of every token (HBM), and only then the position / slot reads
    // and the tokens' cos/sin tables (no memory operand but the angles' positions), which run
    // while the rows are in flight (position reads issued ahead of the rows delay every row
    // request by their latency: c2 7.75 -> 6.69 us with this order and the register selects
    // above). Every thread issues all of these loads (from the zero row where there is nothing
    // to read): the compiler counts outstanding loads per path, and were some skipped on one
    // path, a wait for the earliest would become a wait for all of them.
    const int ti = threadIdx.x;
    const int wi = ti < D / 4 ? ti : ti - D / 4;
    const bool stage_q = ti < D / 4, stage_k = ti >= D / 4 && ti < D / 2;
    const float* ws = stage_q && has_wq ? wqb : stage_k && has_wk ? wkb : g_qk_pad_row;
    const f32x4 wstage = ldf4(ws + (stage_q || stage_k ? 4 * wi : 0));
    // (NP > 1: the head rows of the token's first NP passes, all requested here)
    u32x4 ra[TPW][NP], rb[TPW][NP];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
        for (int q = 0; q < NP; ++q) {
            const int hr = gslot + q * hstep;
            const bool row_ok = hr < HR && readable(hr, tb + tt);
            const T* src0 = row_ok ? src_of(hr, tb + tt) : (const T*)g_qk_pad_row;
            ra[tt][q] = ldg16<kQkLdNt>(src0 + c0 * E);
            rb[tt][q] = ldg16<kQkLdNt>(src0 + c1 * E);
        }

    int p[TPW];
    int64_t row[TPW];
    bool tok[TPW];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        tok[tt] = tb + tt < a.n_tokens;  // uniform
        p[tt] = tok[tt] ? token_pos(a, tb + tt) : 0;
        row[tt] = tok[tt] ? token_row(a, tb + tt, p[tt]) : -1;
    }
    auto active = [&](int hr, int tt) -> bool {
        if (!tok[tt]) return false;
        if (hr < a.nh) return nq > 0;
        if (hr < a.nh + a.nkv) return a.k != nullptr && row[tt] >= 0;
        return a.v != nullptr && row[tt] >= 0;
    };
    if (a.do_rope) {
        for (int i = ti; i < TPW * a.half; i += 256) {
            const int tt = i / a.half, k = i - tt * a.half;
            const float theta = ((float)p[tt] * a.freq_scale) / rope_denom(k, 2 * a.half, a.log2_base);
            rope_sincos(theta, &s_sin[tt][k], &s_cos[tt][k]);
        }
    }
    if (stage_q || stage_k) {
        const bool hw = stage_q ? has_wq : has_wk;
        f32x4 f;
        f.x = w_factor(wstage.x, hw, a.uo);
        f.y = w_factor(wstage.y, hw, a.uo);
        f.z = w_factor(wstage.z, hw, a.uo);
        f.w = w_factor(wstage.w, hw, a.uo);
        *reinterpret_cast<f32x4*>((stage_q ? s_wq : s_wk) + 4 * wi) = f;
    }
    __syncthreads();

    // One head row of token tb + tt: norm, RoPE, store.
    auto process = [&](int hr, int tt, u32x4 xa, u32x4 xb) {
        const int t = tb + tt;
        const int kind = hr < a.nh ? 0 : hr < a.nh + a.nkv ? 1 : 2;  // Q, K, V
        float x0[E], x1[E];
        C::unpack(xa, x0);
        C::unpack(xb, x1);
        const bool norm = kind == 0 ? a.do_qnorm : kind == 1 ? a.do_knorm : a.v_norm;
        if (norm) {
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < E; ++j) {
                ss = fmaf(x0[j], x0[j], ss);
                ss = fmaf(x1[j], x1[j], ss);
            }
            ss = group_sum<LH>(ss);
            // 1 / sqrt(mean + eps) by the hardware reciprocal square root (within 1 ulp
            // of the reference's IEEE sqrt and divide, and ~20 instructions shorter per
            // row: this kernel's arithmetic is exposed, c2 7.89 -> 7.72 us); D is a power
            // of two, so the mean is exact
            const float inv = __builtin_amdgcn_rsqf(ss * (1.0f / (float)D) + a.eps);
            if (kind == 2) {  // Gemma-4 V: no-scale norm
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    x0[j] = x0[j] * inv;
                    x1[j] = x1[j] * inv;
                }
            } else {
                const float* sw = kind == 0 ? s_wq : s_wk;  // factors (1+w), w or 1
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    x0[j] = (x0[j] * inv) * sw[c0 * E + j];
                    x1[j] = (x1[j] * inv) * sw[c1 * E + j];
                }
            }
        }
        if (a.do_rope && kind != 2 && hl < R) {
#pragma unroll
            for (int j = 0; j < E; ++j) {
                const float c = s_cos[tt][hl * E + j], s = s_sin[tt][hl * E + j];
                const float v0 = x0[j], v1 = x1[j];
                x0[j] = v0 * c - v1 * s;
                x1[j] = v0 * s + v1 * c;
            }
        }
        T* dst;
        if (kind == 0) dst = (T*)a.q + ((int64_t)t * a.nh + hr) * D;
        else if (kind == 1) dst = (T*)a.kdst + row[tt] * a.row_stride + (int64_t)(hr - a.nh) * D;
        else dst = (T*)a.vdst + row[tt] * a.row_stride + (int64_t)(hr - a.nh - a.nkv) * D;
        stg16<kQkStNt>(dst + c0 * E, C::pack(x0));
        stg16<kQkStNt>(dst + c1 * E, C::pack(x1));
    };
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
#pragma unroll
        for (int q = 0; q < NP; ++q) {
            const int hr = gslot + q * hstep;
            if (hr < HR && active(hr, tt)) process(hr, tt, ra[tt][q], rb[tt][q]);
        }
        // passes past the preloaded ones: their rows requested in turn
        for (int hr = gslot + NP * hstep; hr < HR; hr += hstep) {
            if (!active(hr, tt)) continue;
            const T* src = src_of(hr, tb + tt);
            process(hr, tt, ldg16<kQkLdNt>(src + c0 * E), ldg16<kQkLdNt>(src + c1 * E));
        }
    }
}

// ---- generic path ----------------------------------------------------------------------

template <typename T>
__device__ __forceinline__ float gld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float gld<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float gld<uint16_t>(const uint16_t* p, int64_t i) { return bf16_lo(p[i]); }
template <typename T>
__device__ __forceinline__ void gst(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void gst<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void gst<uint16_t>(uint16_t* p, int64_t i, float v) {
    p[i] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
}

template <typename T>
__global__ __launch_bounds__(256) void k_qk_generic(QkArgs a, RopeTab tab) {
    __shared__ float s_cos[kMaxHalf], s_sin[kMaxHalf];
    __shared__ float s_head[4][2 * kMaxHalf];
    const int t = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int D = a.D, half = a.half;
    const int HR = a.nh + 2 * a.nkv;
    const int p = token_pos(a, t);
    const int64_t row = token_row(a, t, p);
    if (a.do_rope) fill_cos_sin(tab, (float)p * a.freq_scale, half, s_cos, s_sin);
    __syncthreads();
    float* buf = s_head[wave];
    // Workgroup (t, y) takes head rows 4y .. 4y+3 of token t, one per wave.
    {
        const int hr = blockIdx.y * 4 + wave;
        int kind = -1;
        const T* src = nullptr;
        T* dst = nullptr;
        if (hr < a.nh) {
            if (a.q) {
                kind = 0;
                src = (const T*)a.q + ((int64_t)t * a.nh + hr) * D;
                dst = (T*)a.q + ((int64_t)t * a.nh + hr) * D;
            }
        } else if (hr < a.nh + a.nkv) {
            if (a.k && row >= 0) {
                kind = 1;
                src = (const T*)a.k + ((int64_t)t * a.nkv + (hr - a.nh)) * D;
                dst = (T*)a.kdst + row * a.row_stride + (int64_t)(hr - a.nh) * D;
            }
        } else if (hr < HR) {
            if (a.v && row >= 0) {
                kind = 2;
                src = (const T*)a.v + ((int64_t)t * a.nkv + (hr - a.nh - a.nkv)) * D;
                dst = (T*)a.vdst + row * a.row_stride + (int64_t)(hr - a.nh - a.nkv) * D;
            }
        }
        float ss = 0.0f;
        if (kind >= 0) {
            for (int i = lane; i < D; i += kWave) {
                const float x = gld(src, i);
                buf[i] = x;
                ss = fmaf(x, x, ss);
            }
        }
        ss = group_sum<kWave>(ss);
        __syncthreads();
        if (kind >= 0) {
            const bool norm = kind == 0 ? a.do_qnorm : kind == 1 ? a.do_knorm : a.v_norm;
            if (norm) {
                const float inv = rms_inv(ss, D, a.eps);
                const float* w = kind == 0 ? a.wq : kind == 1 ? a.wk : nullptr;
                for (int i = lane; i < D; i += kWave) {
                    const float y = buf[i] * inv;
                    buf[i] = w ? (a.uo ? y * (1.0f + w[i]) : y * w[i]) : y;
                }
            }
        }
        __syncthreads();
        if (kind >= 0 && kind != 2 && a.do_rope) {
            for (int i = lane; i < half; i += kWave) {
                const float c = s_cos[i], s = s_sin[i];
                const float v0 = buf[i], v1 = buf[i + half];
                buf[i] = v0 * c - v1 * s;
                buf[i + half] = v0 * s + v1 * c;
            }
        }
        __syncthreads();
        if (kind >= 0)
            for (int i = lane; i < D; i += kWave) gst(dst, i, buf[i]);
        __syncthreads();
    }
}

// ---- host side -------------------------------------------------------------------------

// D_i = f32(pow(f64 base, f64(f32(2i)/f32(eff)))): the same expression as the oracle's
// zo_rope_denominator. A few (base, eff) tables are cached per host thread.
static const RopeTab& rope_table(float base, int eff) {
    struct Entry {
        float base;
        int eff;
        RopeTab tab;
    };
    static thread_local Entry cache[4];
    static thread_local int used = 0, next = 0;
    for (int i = 0; i < used; ++i)
        if (cache[i].eff == eff && memcmp(&cache[i].base, &base, sizeof(float)) == 0) return cache[i].tab;
    Entry& e = cache[next];
    next = (next + 1) % 4;
    if (used < 4) ++used;
    e.base = base;
    e.eff = eff;
    memset(&e.tab, 0, sizeof(e.tab));
    for (int i = 0; i < eff / 2 && i < kMaxHalf; ++i) {
        const float ex = (float)(2 * i) / (float)eff;
        e.tab.denom[i] = (float)pow((double)base, (double)ex);
    }
    return e.tab;
}

template <typename T>
static void launch_qk_t(const QkArgs& a, const RopeTab& tab, hipStream_t s) {
    constexpr int E = Chunk<T>::E;
    const bool fast = (a.D == 64 || a.D == 128 || a.D == 256 || a.D == 512) && a.half % E == 0 &&
                      aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.kdst) &&
                      aligned16(a.vdst) && aligned16(a.wq) && aligned16(a.wk) && a.row_stride % E == 0;
    const unsigned grid = (unsigned)a.n_tokens;
    if (fast) {
        // Few tokens (decode): one workgroup per pass of head rows, so no workgroup loops
        // (each pass would wait for its own loads); many tokens: the token's rows in turn.
        const int HR = a.nh + 2 * a.nkv;
        auto gy = [&](int slots) {
            return (unsigned)(a.n_tokens <= ZL_QK_GY_TOKENS ? std::max<int64_t>(1, cdiv(HR, slots)) : 1);
        };
        // Two tokens per workgroup (the weight staging and the barrier shared by both) for
        // launches with many tokens whose head rows fit one pass (Gemma-4B at 2048 tokens:
        // 7.87 -> 7.76 us; with two passes per token the second token's passes follow the
        // first's: Gemma-27B heads at 8192 tokens 43.8 -> 49.8 us, so one token there).
        constexpr int TP = ZL_QK_TPW;
        const unsigned gridm = (unsigned)cdiv(a.n_tokens, TP);
        auto go = [&](auto d_c) {
            constexpr int DD = decltype(d_c)::value;
            constexpr int SL = qk_slots<T, DD>();
            const bool multi = TP > 1 && a.n_tokens >= ZL_QK_TPW_MIN && HR <= SL;
            // ZL_QK_NP2: a token's two passes of head rows requested at once (NP = 2); measured
            // slower for Gemma-27B heads at 8192 tokens (42.9 -> 45.0 us), so off by default
            const bool two_pass = ZL_QK_NP2 && !multi && cdiv(HR, SL * (int)gy(SL)) == 2;
            if (multi) k_qk_fused<T, DD, TP><<<dim3(gridm, gy(SL)), 256, 0, s>>>(a);
            else if (two_pass) k_qk_fused<T, DD, 1, 2><<<dim3(grid, gy(SL)), 256, 0, s>>>(a);
            else k_qk_fused<T, DD, 1><<<dim3(grid, gy(SL)), 256, 0, s>>>(a);
        };
        if (a.D == 64) go(std::integral_constant<int, 64>{});
        else if (a.D == 128) go(std::integral_constant<int, 128>{});
        else if (a.D == 256) go(std::integral_constant<int, 256>{});
        else go(std::integral_constant<int, 512>{});
    } else {
        const dim3 g2(grid, (unsigned)std::max<int64_t>(1, cdiv(a.nh + 2 * a.nkv, 4)));  // 4 head rows per workgroup
        k_qk_generic<T><<<g2, 256, 0, s>>>(a, tab);
    }
    check_launch();
}

static void launch_qk(int dtype, QkArgs& a, float base, int rotary_dim, hipStream_t s) {
    if (a.n_tokens <= 0 || a.D <= 0) return;
    if (a.D > 2 * kMaxHalf || (a.D & 1) || a.nh < 0 || a.nkv < 0) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    const int eff = (rotary_dim <= 0 || rotary_dim > a.D) ? a.D : rotary_dim;
    a.half = eff / 2;
    if ((a.k && !a.kdst) || (a.v && !a.vdst) || (a.pos_mode != 0 && !a.pos) ||
        (a.slot_mode == 1 && !a.slot)) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    static const RopeTab zero_tab = {};
    const RopeTab& tab = a.do_rope ? rope_table(base, eff) : zero_tab;
    a.log2_base = log2((double)base);
    if (dtype == HIP_BRIDGE_F32) launch_qk_t<float>(a, tab, s);
    else if (dtype == HIP_BRIDGE_BF16) launch_qk_t<uint16_t>(a, tab, s);
    else set_error(HIP_BRIDGE_EUNSUPPORTED);
}

static QkArgs base_args() {
    QkArgs a;
    memset(&a, 0, sizeof(a));
    a.freq_scale = 1.0f;
    return a;
}

}  // namespace zl

using namespace zl;

extern "C" {

void hip_qk_norm_rope_kv(int dtype, void* q, const void* k, const void* v,
                         const float* q_norm_w, const float* k_norm_w, int v_norm,
                         void* k_cache, void* v_cache, int64_t cache_rows, int layer_idx,
                         int max_seq, int max_kv_dim, const int32_t* d_pos, int pos_base,
                         const int64_t* d_slot, int n_tokens, int num_heads, int num_kv_heads,
                         int head_dim, int rotary_dim, float freq_base, float freq_scale,
                         float eps, int use_unit_offset, HipStream_t stream) {
    QkArgs a = base_args();
    a.q = q;
    a.k = k;
    a.v = v;
    a.wq = q_norm_w;
    a.wk = k_norm_w;
    a.kdst = k_cache;
    a.vdst = v_cache;
    a.cache_rows = cache_rows;
    a.row_stride = max_kv_dim;
    a.pos = d_pos;
    a.pos_mode = d_pos ? 1 : 0;
    a.pos_base = pos_base;
    a.slot = d_slot;
    a.slot_mode = d_slot ? 1 : 0;
    a.layer_base = (int64_t)layer_idx * max_seq;
    a.max_seq = max_seq;
    a.n_tokens = n_tokens;
    a.nh = q ? num_heads : 0;
    a.nkv = num_kv_heads;
    a.D = head_dim;
    a.do_qnorm = q_norm_w != nullptr;
    a.do_knorm = k_norm_w != nullptr;
    a.v_norm = v_norm;
    a.do_rope = 1;
    a.uo = use_unit_offset;
    a.freq_scale = freq_scale;
    a.eps = eps;
    if (max_kv_dim < num_kv_heads * head_dim || (k && !k_cache) || (v && !v_cache)) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    launch_qk(dtype, a, freq_base, rotary_dim, stream_of(stream));
}

// ---- reference-ABI RoPE (in place, f32) ------------------------------------------------

static void rope_common(float* q, float* k, const int* d_pos, int pos, int batch, int nh,
                        int nkv, int head_dim, int rotary_dim, float base, HipStream_t stream) {
    if (batch <= 0) return;
    QkArgs a = base_args();
    a.q = q;
    a.k = k;
    a.kdst = k;
    a.row_stride = (int64_t)nkv * head_dim;
    a.pos = d_pos;
    a.pos_mode = d_pos ? 2 : 0;
    a.pos_base = pos;
    a.slot_mode = 2;
    a.n_tokens = batch;
    a.nh = q ? nh : 0;
    a.nkv = k ? nkv : 0;
    a.D = head_dim;
    a.do_rope = 1;
    launch_qk(HIP_BRIDGE_F32, a, base, rotary_dim, stream_of(stream));
}

void hip_rope(float* q, float* k, int pos, int num_heads, int num_kv_heads, int head_dim,
              int rotary_dim, float freq_base, HipStream_t stream) {
    rope_common(q, k, nullptr, pos, 1, num_heads, num_kv_heads, head_dim, rotary_dim, freq_base, stream);
}

void hip_rope_ind(float* q, float* k, const int* d_pos, int num_heads, int num_kv_heads,
                  int head_dim, int rotary_dim, float freq_base, HipStream_t stream) {
    if (!d_pos) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    rope_common(q, k, d_pos, 0, 1, num_heads, num_kv_heads, head_dim, rotary_dim, freq_base, stream);
}

void hip_rope_batched(float* q, float* k, int pos, int batch_size, int num_heads,
                      int num_kv_heads, int head_dim, int rotary_dim, float freq_base,
                      HipStream_t stream) {
    rope_common(q, k, nullptr, pos, batch_size, num_heads, num_kv_heads, head_dim, rotary_dim,
                freq_base, stream);
}

// ---- reference-ABI KV append (f32) -----------------------------------------------------

static void kv_put_common(float* kc, float* vc, const float* k, const float* v, int layer,
                          const int* d_pos, int pos, int batch, int max_seq, int nkv,
                          int head_dim, int max_kv_dim, HipStream_t stream) {
    if (batch <= 0 || nkv <= 0 || head_dim <= 0) return;
    if (!kc || !vc || !k || !v || max_kv_dim < nkv * head_dim) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    QkArgs a = base_args();
    a.k = k;
    a.v = v;
    a.kdst = kc;
    a.vdst = vc;
    a.row_stride = max_kv_dim;
    a.pos = d_pos;
    a.pos_mode = d_pos ? 2 : 0;
    a.pos_base = pos;
    a.slot_mode = 0;
    a.layer_base = (int64_t)layer * max_seq;
    a.max_seq = max_seq;
    a.n_tokens = batch;
    a.nh = 0;
    a.nkv = nkv;
    a.D = head_dim;
    a.do_rope = 0;
    launch_qk(HIP_BRIDGE_F32, a, 0.0f, 0, stream_of(stream));
}

void hip_kv_cache_put(float* k_cache, float* v_cache, const float* k, const float* v,
                      int layer_idx, int pos, int max_seq, int n_kv_heads, int head_dim,
                      int max_kv_dim, HipStream_t stream) {
    kv_put_common(k_cache, v_cache, k, v, layer_idx, nullptr, pos, 1, max_seq, n_kv_heads,
                  head_dim, max_kv_dim, stream);
}

void hip_kv_cache_put_ind(float* k_cache, float* v_cache, const float* k, const float* v,
                          int layer_idx, const int* d_pos, int max_seq, int n_kv_heads,
                          int head_dim, int max_kv_dim, HipStream_t stream) {
    if (!d_pos) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    kv_put_common(k_cache, v_cache, k, v, layer_idx, d_pos, 0, 1, max_seq, n_kv_heads, head_dim,
                  max_kv_dim, stream);
}

void hip_kv_cache_put_batched(float* k_cache, float* v_cache, const float* k, const float* v,
                              int layer_idx, int pos, int batch_size, int max_seq,
                              int n_kv_heads, int head_dim, int max_kv_dim,
                              HipStream_t stream) {
    kv_put_common(k_cache, v_cache, k, v, layer_idx, nullptr, pos, batch_size, max_seq,
                  n_kv_heads, head_dim, max_kv_dim, stream);
}

}  // extern "C"
