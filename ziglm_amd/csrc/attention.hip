// Decode attention over the KV cache with soft-capped scores, sliding window and GQA
// (replaces cuda_bridge.cu:2466-2879: cuda_attention_forward, _ind, _batched; CPU
// definition model.zig:658-700 with math.softmax, math.zig:1088-1106).
//
// Query token b (of `batch`) at position p_b attends to positions [start_b, p_b], start_b =
// p_b + 1 - window when a window is set and exceeded: score_t = (q_h . k_t) * scale, then
// cap * tanh(score / cap) when cap > 0, softmax over t, out_h = sum_t w_t v_t; query head h
// reads kv head h / (n_heads / n_kv_heads).
//
// Layout (flash-decoding). One workgroup per (token b, kv head, head group, split s) covers
// one chunk of consecutive positions (the sequence's own length cut into nsplit chunks,
// split_chunk) for G query heads of the kv head (G = n_heads/n_kv_heads, or
// a fraction of it when there are few kv-head groups, choose_heads). Lanes come in groups of
// LT = D/8 (8 elements of a head row per lane), one group per position, so a wave works on
// 64/LT positions at a time and the K/V row loads of a position are one contiguous span; the
// workgroup's G query heads reuse each loaded K and V row. Each lane group keeps an online softmax state per
// query head (running max m, sum l, accumulator a = sum exp(s - m) v); the groups and waves
// are merged through LDS. With one split the workgroup writes out = a / l; otherwise it
// writes (m, l, a) to the caller's workspace and a second kernel merges the splits.
// Arithmetic: f32 throughout, exp via exp2; results agree with the CPU's (which exponentiates
// after a full max pass and normalises the weights before the weighted sum) within the f32
// rounding of the scores, not bit for bit.
#include <math.h>
#include <algorithm>
#include <mutex>

#include "zl_common.h"
#include "zl_host.h"

namespace zl {

#ifndef ZL_ATTN_THREADS
#define ZL_ATTN_THREADS 256
#endif
constexpr int kAttnThreads = ZL_ATTN_THREADS;  // k_attn workgroup
constexpr int kMergeThreads = 256;             // k_attn_merge workgroup
constexpr float kLog2e = 1.4426950408889634f;
// A head row of zeros (head_dim <= 512) that loads with nothing to read point at.
__device__ __attribute__((aligned(16))) float g_attn_pad_row[512];

struct AttnArgs {
    const float* q;           // [batch][n_heads][D]
    const void* kc;           // cache rows of row_stride elements (f32 or bf16)
    const void* vc;
    float* out;               // [batch][n_heads][D]
    float* ws;                // [batch][n_heads][nsplit][D + 2] partials (nsplit > 1)
    const int32_t* pos;       // per-token positions, or null: pos_base + b
    const int64_t* row_base;  // per-token cache row of position 0, or null: row0
    int64_t row0;
    int64_t cache_rows;       // > 0: rows outside [0, cache_rows) give a zero output
    int64_t row_stride;
    int pos_base;
    int max_len;              // positions must be < max_len
    int batch, nh, nkv, D;
    int window;
    int nsplit;               // splits per sequence (split_chunk)
    int chunk_min;            // shortest split (split_chunk)
    int gq;                   // query heads per kv head (nh / nkv)
    int hg;                   // workgroups per (token, kv head, split): each takes gq / hg heads
    float scale, softcap, inv_cap;
    // QK mode (k_attn<..., true>): the query heads arrive raw and are normalised and rotated
    // here, and the token's own K/V row is formed from the raw projections (not read from the
    // cache) and written to the cache by one workgroup per kv head.
    const float* qk_k;        // raw K / V of the tokens [batch][nkv][D], or null: reads only
    const float* qk_v;
    const float* qk_wq;       // per-head norm weights [D], or null: no norm
    const float* qk_wk;
    int qk_vnorm, qk_uo, qk_half;  // V no-scale norm; (1 + w) weights; rotary_dim / 2 (0: none)
    float qk_eps, qk_freq_scale;
    double qk_log2_base;
};

// Position range of token b, or an empty range when its rows fall outside the cache.
__device__ __forceinline__ void attn_range(const AttnArgs& a, int b, int& start, int& end, int64_t& rb) {
    const int p = a.pos ? a.pos[b] : a.pos_base + b;
    rb = a.row_base ? a.row_base[b] : a.row0;
    start = 0;
    end = 0;
    if (p < 0 || p >= a.max_len || rb < 0) return;
    if (a.cache_rows > 0 && rb + p >= a.cache_rows) return;
    end = p + 1;
    start = (a.window > 0 && end > a.window) ? end - a.window : 0;
}

// Positions per split for a sequence of `len` positions: the sequence's own length is cut
// into nsplit equal chunks (the host sized nsplit for the longest possible sequence), no
// chunk shorter than a.chunk_min, so a short context spreads over fewer splits and the rest
// stay empty. Returns the number of non-empty splits in `used`.
#ifndef ZL_ATTN_CHUNK_MIN
#define ZL_ATTN_CHUNK_MIN 8
#endif
__device__ __forceinline__ int split_chunk(const AttnArgs& a, int len, int& used) {
    const int chunk = max((len + a.nsplit - 1) / a.nsplit, a.chunk_min);
    used = len > 0 ? min(a.nsplit, (len + chunk - 1) / chunk) : 0;
    return chunk;
}

template <typename KT>
__device__ __forceinline__ void load8(const KT* row, float* v) {
    if constexpr (sizeof(KT) == 4) {
        const f32x4 x = ldf4((const float*)row), y = ldf4((const float*)row + 4);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
        v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
    } else {
        Chunk<uint16_t>::unpack(ld16(row), v);
    }
}

// QK mode: RMSNorm of a head row held as 8 elements per lane over LT lanes (the norm
// kernels' arithmetic: inv = rms_inv(sum of squares), then (x * inv) * factor).
template <int LT>
__device__ __forceinline__ void qk_norm8(float* x, int D, float eps, const float* wf) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
    const float inv = rms_inv(group_sum<LT>(ss), D, eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (x[e] * inv) * wf[e];
}
// Half-split RoPE of a head row held as 8 elements per lane: element i < half pairs with
// i + half, which lives hl = half / 8 lanes further (hl a power of two, so the partner is
// lane ^ hl within the row's lane group); cos / sin of pair i come from the LDS table. The
// rotation is the QK kernel's: v0*c - v1*s, v0*s + v1*c.
__device__ __forceinline__ void qk_rope8(float* x, int li, int half, const float* s_cos, const float* s_sin) {
    const int hl = half >> 3;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = __shfl_xor(x[e], hl);
    if (li < 2 * hl) {
        const int base = (li & (hl - 1)) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float c = s_cos[base + e], sn = s_sin[base + e];
            x[e] = li < hl ? x[e] * c - y[e] * sn : y[e] * sn + x[e] * c;
        }
    }
}

template <typename KT, int D, int G, bool QK, bool DB>
__global__ __launch_bounds__(kAttnThreads) void k_attn(AttnArgs a) {
    constexpr int LT = D / 8;                  // lanes per position
    constexpr int SLOTS = kAttnThreads / LT;   // positions in flight per workgroup
    constexpr int GM = G < 4 ? G : 4;          // query heads merged per LDS pass
    // Per-slot states for the merge: m, l per query head, a per (head, element); the G heads
    // go through in passes of GM (LDS = SLOTS * GM * D * 4 <= 32 KB for every D).
    __shared__ float s_m[SLOTS][GM], s_l[SLOTS][GM];
    __shared__ float s_a[SLOTS][GM][D];
    __shared__ float s_cos[QK ? D / 2 : 1], s_sin[QK ? D / 2 : 1];
    const int tid = threadIdx.x;
    const int slot = tid / LT;
    const int li = tid % LT;                   // 8-element slice of the head row
    const int split = blockIdx.x % a.nsplit;
    const int r = blockIdx.x / a.nsplit;
    const int hgi = r % a.hg;
    const int bk = r / a.hg;
    const int kvh = bk % a.nkv;
    const int b = bk / a.nkv;
    const int h0 = kvh * a.gq + hgi * G;       // first query head of this workgroup

    // The query rows (and in QK mode their norm factors) do not depend on the token's
    // position: they go out first, ahead of the position read and of the K/V rows, so that
    // the query is normalised and rotated while the K/V rows are in flight (waits count loads
    // in issue order: issued after the K/V rows, the query would wait for all of them).
    float q[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float* qh = a.q + ((int64_t)b * a.nh + h0 + g) * D + li * 8;
        const f32x4 x = ldf4(qh), y = ldf4(qh + 4);
        q[g][0] = x.x; q[g][1] = x.y; q[g][2] = x.z; q[g][3] = x.w;
        q[g][4] = y.x; q[g][5] = y.y; q[g][6] = y.z; q[g][7] = y.w;
    }
    // QK mode: the Q norm weights of this lane's slice
    // (raw: the factors are formed where they are used, so nothing waits for these loads
    // before the K/V rows are requested; a null weight reads as zeros through an empty range)
    f32x4 wq0{}, wq1{};
    if constexpr (QK) {
        const auto rs = buf_rsrc(a.qk_wq, a.qk_wq ? (uint32_t)D * 4u : 0u);
        wq0 = bldf4(rs, (uint32_t)li * 32u);
        wq1 = bldf4(rs, (uint32_t)li * 32u + 16u);
    }

    int start, end;
    int64_t rb;
    attn_range(a, b, start, end, rb);
    int used;
    const int chunk = split_chunk(a, end - start, used);
    // Splits past the sequence's length hold nothing: the merge reads only the first `used`
    // (block-uniform exit; with one split the workgroup still writes the zero output).
    if (a.nsplit > 1 && split >= used) return;
    const int t0 = start + split * chunk;
    const int t1 = min(end, t0 + chunk);
    const int last = end - 1;  // the token's own position (end > 0 whenever any work is done)

    const KT* kbase = (const KT*)a.kc + kvh * D + li * 8;
    const KT* vbase = (const KT*)a.vc + kvh * D + li * 8;
    // QK mode with new K/V: the token's own position is not read from the cache (its row is
    // written below); the split holding it folds it in after the loop.
    const bool own = QK && a.qk_k != nullptr;
    const int tc = own ? min(t1, last) : t1;
    // Each lane group takes U positions per step (t, t + SLOTS, ...), all 2U row loads issued
    // before any math, then folds them into its online softmax state in position order. A
    // position past the range loads the range's last row instead (in bounds, no per-lane
    // branch) and is not folded. The first step's rows are requested here, before the query
    // is (QK mode) normalised and rotated, which does not need them.
    constexpr int U = 4;
    const int nstep = t0 < tc ? (tc - t0 + U * SLOTS - 1) / (U * SLOTS) : 0;  // uniform
    float k[U][8], v[U][8];
    // The first step's loads and the own-row loads below are issued on every path (no load
    // under a branch): the compiler counts outstanding loads per path, and where paths with
    // fewer loads join, its waits for the earlier loads (the query) become waits for all of
    // them. With nothing to fold (nstep 0) the first step still loads, from row 0 of the
    // sequence (or, for an invalid position, whose rows may lie outside the cache, from a
    // zero row of this library): in bounds and never folded.
    const bool rows_ok = end > 0;  // uniform
    const KT* qsafe = (const KT*)g_attn_pad_row + li * 8;
    auto load_into = [&](float (&kk)[U][8], float (&vv)[U][8], int t) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int tu = max(min(t + u * SLOTS, tc - 1), 0);
            load8<KT>(rows_ok ? kbase + (rb + tu) * a.row_stride : qsafe, kk[u]);
            load8<KT>(rows_ok ? vbase + (rb + tu) * a.row_stride : qsafe, vv[u]);
        }
    };
    load_into(k, v, t0 + slot);
    // QK mode: the split holding the token's own position requests the raw K / V rows that
    // position is formed from (and the K norm factors) now, used after the loop; in the
    // other splits the same loads read an empty range (zeros, no memory access).
    const bool own_here = own && t0 <= last && last < t1;  // block-uniform
    f32x4 rk0{}, rk1{}, rv0{}, rv1{}, wk0{}, wk1{};
    if constexpr (QK) {
        const uint32_t rowb = own_here ? (uint32_t)D * 4u : 0u;
        const int64_t ro = ((int64_t)b * a.nkv + kvh) * D;
        const auto rs_k = buf_rsrc(own_here ? a.qk_k + ro : a.q, rowb);
        const auto rs_v = buf_rsrc(own_here ? a.qk_v + ro : a.q, rowb);
        const auto rs_w = buf_rsrc(a.qk_wk ? a.qk_wk : a.q, a.qk_wk ? rowb : 0u);
        const uint32_t o = (uint32_t)li * 32u;
        rk0 = bldf4(rs_k, o);
        rk1 = bldf4(rs_k, o + 16u);
        rv0 = bldf4(rs_v, o);
        rv1 = bldf4(rs_v, o + 16u);
        wk0 = bldf4(rs_w, o);
        wk1 = bldf4(rs_w, o + 16u);
    }

    if constexpr (QK) {
        // cos / sin of the token's position for the rotary pairs, while the loads fly
        if (a.qk_half > 0 && tid < a.qk_half && end > 0) {
            const float theta = ((float)last * a.qk_freq_scale) / rope_denom(tid, 2 * a.qk_half, a.qk_log2_base);
            rope_sincos(theta, &s_sin[tid], &s_cos[tid]);
        }
        __syncthreads();  // the cos / sin table
        const float wv[8] = {wq0.x, wq0.y, wq0.z, wq0.w, wq1.x, wq1.y, wq1.z, wq1.w};
        float fq[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) fq[e] = a.qk_uo ? 1.0f + wv[e] : wv[e];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (a.qk_wq) qk_norm8<LT>(q[g], D, a.qk_eps, fq);
            if (a.qk_half > 0) qk_rope8(q[g], li, a.qk_half, s_cos, s_sin);
        }
    }
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
    }
    // Online softmax step of one position for this lane group (k, v: its 8-element slices).
    auto fold = [&](const float* k, const float* v, bool take) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s = fmaf(q[g][e], k[e], s);
            s = group_sum<LT>(s) * a.scale;
            if (a.softcap > 0.0f) s = a.softcap * tanh_fast(div_by_uniform(s, a.softcap, a.inv_cap));
            if (take) {
                const float mn = fmaxf(m[g], s);
                const float c = exp2f((m[g] - mn) * kLog2e);
                const float p = exp2f((s - mn) * kLog2e);
                l[g] = l[g] * c + p;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] = fmaf(p, v[e], acc[g][e] * c);
                m[g] = mn;
            }
        }
    };

    auto fold_step = [&](const float (&kk)[U][8], const float (&vv)[U][8], int t) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (t + u * SLOTS >= tc) break;  // uniform within a lane group
            fold(kk[u], vv[u], true);
        }
    };
    if constexpr (DB) {
        // Two register sets in turn: the next step's rows are requested before the current
        // step is folded, so each step's round trip overlaps the previous step's arithmetic
        // (a step past the range loads the range's last row again and is not folded).
        float k2[U][8], v2[U][8];
        for (int st = 0; st < nstep; st += 2) {
            const int t = t0 + slot + st * U * SLOTS;
            load_into(k2, v2, t + U * SLOTS);
            fold_step(k, v, t);
            if (st + 1 >= nstep) break;  // uniform
            load_into(k, v, t + 2 * U * SLOTS);
            fold_step(k2, v2, t + U * SLOTS);
        }
    } else {
        for (int st = 0; st < nstep; ++st) {
            const int t = t0 + slot + st * U * SLOTS;
            if (st > 0) load_into(k, v, t);
            fold_step(k, v, t);
        }
    }
    if constexpr (QK) {
        if (own_here) {  // block-uniform: the split holding the token
            // Every lane group forms the row (uniform code); slot 0 folds it in and, in the
            // first head group's workgroup, writes it to the cache.
            float kn[8] = {rk0.x, rk0.y, rk0.z, rk0.w, rk1.x, rk1.y, rk1.z, rk1.w};
            float vn[8] = {rv0.x, rv0.y, rv0.z, rv0.w, rv1.x, rv1.y, rv1.z, rv1.w};
            const float wv[8] = {wk0.x, wk0.y, wk0.z, wk0.w, wk1.x, wk1.y, wk1.z, wk1.w};
            float fk[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) fk[e] = a.qk_uo ? 1.0f + wv[e] : wv[e];
            if (a.qk_wk) qk_norm8<LT>(kn, D, a.qk_eps, fk);
            if (a.qk_vnorm) {
                float one[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) one[e] = 1.0f;
                qk_norm8<LT>(vn, D, a.qk_eps, one);
            }
            if (a.qk_half > 0) qk_rope8(kn, li, a.qk_half, s_cos, s_sin);
            // attention uses the row as the cache holds it (bf16 caches: rounded), as it would
            // read it back
            u32x4 kp{}, vp{};
            if constexpr (sizeof(KT) == 2) {
                kp = Chunk<uint16_t>::pack(kn);
                vp = Chunk<uint16_t>::pack(vn);
                Chunk<uint16_t>::unpack(kp, kn);
                Chunk<uint16_t>::unpack(vp, vn);
            }
            fold(kn, vn, slot == 0);
            if (hgi == 0 && slot == 0) {
                KT* kd = (KT*)a.kc + (rb + last) * a.row_stride + kvh * D + li * 8;
                KT* vd = (KT*)a.vc + (rb + last) * a.row_stride + kvh * D + li * 8;
                if constexpr (sizeof(KT) == 4) {
                    *reinterpret_cast<f32x4*>(kd) = f32x4{kn[0], kn[1], kn[2], kn[3]};
                    *reinterpret_cast<f32x4*>(kd + 4) = f32x4{kn[4], kn[5], kn[6], kn[7]};
                    *reinterpret_cast<f32x4*>(vd) = f32x4{vn[0], vn[1], vn[2], vn[3]};
                    *reinterpret_cast<f32x4*>(vd + 4) = f32x4{vn[4], vn[5], vn[6], vn[7]};
                } else {
                    *reinterpret_cast<u32x4*>(kd) = kp;
                    *reinterpret_cast<u32x4*>(vd) = vp;
                }
            }
        }
    }

    // Merge the SLOTS states: every slot stores its state, then thread i merges element
    // (g, e) = i over the slots in slot order, rescaling each by exp(m_slot - max).
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += GM) {
        if (g0 > 0) __syncthreads();  // the previous pass has read the buffers
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            if (li == 0) {
                s_m[slot][g] = m[g0 + g];
                s_l[slot][g] = l[g0 + g];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) s_a[slot][g][li * 8 + e] = acc[g0 + g][e];
        }
        __syncthreads();
        for (int i = tid; i < GM * D; i += kAttnThreads) {
            const int g = i / D, e = i % D;
            float M = -INFINITY;
            for (int s = 0; s < SLOTS; ++s) M = fmaxf(M, s_m[s][g]);
            float L = 0.0f, A = 0.0f;
            if (M != -INFINITY) {
                for (int s = 0; s < SLOTS; ++s) {
                    const float c = exp2f((s_m[s][g] - M) * kLog2e);
                    L = fmaf(s_l[s][g], c, L);
                    A = fmaf(s_a[s][g][e], c, A);
                }
            }
            const int h = h0 + g0 + g;
            if (a.nsplit == 1) {
                a.out[((int64_t)b * a.nh + h) * D + e] = L > 0.0f ? A / L : 0.0f;
            } else {
                float* w = a.ws + (((int64_t)b * a.nh + h) * a.nsplit + split) * (D + 2);
                w[2 + e] = A;
                if (e == 0) {
                    w[0] = M;
                    w[1] = L;
                }
            }
        }
    }
}

// Merge the splits of (token b, head h) over columns [64 y, 64 y + 64): one workgroup per
// (b, h, y), over the sequence's non-empty splits. Every (m, l) pair and the first kMergePre
// partials of each lane's column are loaded at once through range-checked loads, with the
// position read (one memory round trip before the first reduction); the per-split factors
// exp(m_s - M) and the total L are formed in LDS, lane i of wave w sums column 64 y + i over
// splits w, w + 4, ... in split order, and the four waves' sums are added in wave order.
constexpr int kMaxSplit = 1024;
constexpr int kMergeCols = kWave;
#ifndef ZL_ATTN_MERGE_PRE
#define ZL_ATTN_MERGE_PRE 16
#endif
constexpr int kMergePre = ZL_ATTN_MERGE_PRE;
__device__ __forceinline__ float bldf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__global__ __launch_bounds__(kMergeThreads) void k_attn_merge(AttnArgs a) {
    constexpr int NW = kMergeThreads / kWave;
    constexpr int PER = kMaxSplit / kMergeThreads;  // (m, l) pairs per thread
    __shared__ float s_c[kMaxSplit];
    __shared__ float s_red[NW];
    __shared__ float s_part[NW][kMergeCols];
    const int bh = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid % kWave, wv = tid / kWave;
    const int e = blockIdx.y * kMergeCols + lane;
    // The loads go out before the position is read: over all nsplit splits of the workspace
    // (reads past the last split give 0), the splits at or past `used` dropped below. Those
    // slots hold whatever an earlier call left (the no-allocation scratch is never cleared):
    // the `< used` masks on mv / lv / pre below are what keep such contents, NaN included,
    // out of the result.
    const float* w = a.ws + (int64_t)bh * a.nsplit * (a.D + 2);
    const uint32_t rowb = (uint32_t)(a.D + 2) * 4u;
    const auto rs = buf_rsrc(w, (uint32_t)a.nsplit * rowb);
    float mv[PER], lv[PER], pre[kMergePre];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t o = (uint32_t)(tid + k * kMergeThreads) * rowb;
        mv[k] = bldf(rs, o);
        lv[k] = bldf(rs, o + 4u);
    }
#pragma unroll
    for (int k = 0; k < kMergePre; ++k) pre[k] = bldf(rs, (uint32_t)(wv + k * NW) * rowb + 8u + 4u * (uint32_t)e);
    int start, end, used;
    int64_t rb;
    attn_range(a, bh / a.nh, start, end, rb);
    split_chunk(a, end - start, used);
    float* out = a.out + (int64_t)bh * a.D;
    if (used == 0) {
        if (wv == 0) out[e] = 0.0f;
        return;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (tid + k * kMergeThreads < used) mx = fmaxf(mx, mv[k]);
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) s_red[wv] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    float lsum = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int sp = tid + k * kMergeThreads;
        if (sp < used) {
            const float c = M == -INFINITY ? 0.0f : exp2f((mv[k] - M) * kLog2e);
            s_c[sp] = c;
            lsum = fmaf(lv[k], c, lsum);
        }
    }
    lsum = group_sum<kWave>(lsum);
    if (lane == 0) s_red[wv] = lsum;
    __syncthreads();
    const float L = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    float A = 0.0f;
#pragma unroll
    for (int k = 0; k < kMergePre; ++k)
        if (wv + k * NW < used) A = fmaf(pre[k], s_c[wv + k * NW], A);
#pragma unroll 8
    for (int sp = wv + kMergePre * NW; sp < used; sp += NW) A = fmaf(w[(int64_t)sp * (a.D + 2) + 2 + e], s_c[sp], A);
    s_part[wv][lane] = A;
    __syncthreads();
    if (wv == 0) {
        const float t = (s_part[0][lane] + s_part[1][lane]) + (s_part[2][lane] + s_part[3][lane]);
        out[e] = L > 0.0f ? t / L : 0.0f;
    }
}

template <typename KT, int D, bool QK, bool DB>
static void launch_gq(const AttnArgs& a, hipStream_t s) {
    const unsigned grid = (unsigned)((int64_t)a.batch * a.nkv * a.hg * a.nsplit);
    switch (a.gq / a.hg) {
        case 1: k_attn<KT, D, 1, QK, DB><<<grid, kAttnThreads, 0, s>>>(a); break;
        case 2: k_attn<KT, D, 2, QK, DB><<<grid, kAttnThreads, 0, s>>>(a); break;
        case 4: k_attn<KT, D, 4, QK, DB><<<grid, kAttnThreads, 0, s>>>(a); break;
        default: k_attn<KT, D, 8, QK, DB><<<grid, kAttnThreads, 0, s>>>(a); break;
    }
}
// Double-buffered K/V steps where a split can exceed ZL_ATTN_DB_MIN positions (long steps
// chains; its extra registers cost more than it saves on short splits). Measured (us, Gemma-4B
// heads, f32 caches, positions ~U[0, 32767]): B = 256 5638 -> 5397, B = 64 1638 -> 1606, B = 8
// 253 -> 249; at B = 1 (256-position splits) 53.3 -> 55.9 and in the 4B decode step (short
// splits) 1451 -> 1482 us per token, so those keep one set.
#ifndef ZL_ATTN_DB_MIN
#define ZL_ATTN_DB_MIN 512
#endif
template <typename KT, int D>
static void launch_g(const AttnArgs& a, bool qk, hipStream_t s) {
    const int len = a.window > 0 ? std::min(a.window, a.max_len) : a.max_len;
    const bool db = cdiv((int64_t)len, (int64_t)a.nsplit) > ZL_ATTN_DB_MIN;
    if (qk) {
        if (db) launch_gq<KT, D, true, true>(a, s);
        else launch_gq<KT, D, true, false>(a, s);
    } else {
        if (db) launch_gq<KT, D, false, true>(a, s);
        else launch_gq<KT, D, false, false>(a, s);
    }
}

// Query heads per workgroup. Each workgroup loads its positions' K/V rows once for all the
// heads it takes, so with many (token, kv head) groups every workgroup takes all gq heads
// of its kv head (fewest K/V reads); with few groups (single-token decode over a few kv
// heads) every workgroup takes one head: the heads re-read the same rows (from L2 at
// decode sizes) but each workgroup's serial chain is gq times shorter. Measured on MI355X,
// one token at position 1234 (us per call, with the merge; 1 / 2 / 4 / 8 heads per
// workgroup): 8/1 heads x 256, window 512: 7.4 / 8.8 / 11.7 / 18.1; 8/1 x 512, full
// context: 16.7 / 18.2 / 24.2 / 35.8; 8/4 x 256: 7.4 / 8.8 (2 heads = all).
#ifndef ZL_ATTN_GW
#define ZL_ATTN_GW 0
#endif
// Only while the K/V rows the call can touch stay cache-resident (<= 32 MB: a 4096-position
// f32 cache of 8 heads x 256, say); longer contexts re-read them from HBM per head group, so
// every workgroup takes all heads (Gemma-4B heads at a position ~U[0, 32767], B = 1: 49.7 us
// with all heads, 70.4 us with one head per workgroup, before the per-sequence split).
constexpr int64_t kFewGroups = 16;
constexpr double kKvResidentBytes = 32.0 * (1 << 20);
static void choose_heads(AttnArgs& a, int es) {
    a.gq = a.nh / a.nkv;
    const int len = a.window > 0 ? std::min(a.window, a.max_len) : a.max_len;
    const double kv = (double)a.batch * len * a.nkv * a.D * 2.0 * es;
    int gw = a.gq;
    if (ZL_ATTN_GW > 0) gw = std::min(a.gq, ZL_ATTN_GW);
    else if ((int64_t)a.batch * a.nkv < kFewGroups && kv <= kKvResidentBytes) gw = 1;
    a.hg = a.gq / gw;
}

// Splits per sequence: enough that batch * n_kv_heads * head groups * splits reaches
// ZL_ATTN_TARGET_WG workgroups and no split exceeds 1024 positions of the longest possible
// sequence (sequences of a batch differ in length: short splits keep the long ones from
// leaving a tail), at most one per chunk_min positions, at most kMaxSplit. The actual lengths
// are on the device: each sequence cuts its own length into that many chunks (split_chunk).
// A decode workgroup is latency-bound (its K/V rows arrive at the rate one CU sustains with
// 4 waves), and every split adds to the merge. Measured on MI355X with K/V cold (caches
// rotated past the Infinity Cache), Gemma-4B heads (8/4 x 256), one token, us per call with
// the merge: f32 cache of 4096 rows, QK-fused call, positions 200 / 1250 / 4000: 2048
// workgroups with a 32-position floor 10.8 / 14.1 / 18.0; 512 and 16: 9.9 / 13.0 / 14.7; 512
// and 8: 9.0 / 13.0 / 14.7; 1024 and 16: 11.7 / 14.4 / 17.8. 32768-row cache, positions
// ~U[0, 32767]: 60.8 us with 2048 workgroups, 53.5 with 512.
#ifndef ZL_ATTN_SPLIT_MAX
#define ZL_ATTN_SPLIT_MAX 1024
#endif
#ifndef ZL_ATTN_TARGET_WG
#define ZL_ATTN_TARGET_WG 512
#endif
static void choose_split(AttnArgs& a, size_t ws_bytes) {
    const int len = a.window > 0 ? std::min(a.window, a.max_len) : a.max_len;
    const int64_t groups = (int64_t)a.batch * a.nkv * a.hg;
    const int64_t want = std::max<int64_t>(cdiv(ZL_ATTN_TARGET_WG, groups), cdiv(len, ZL_ATTN_SPLIT_MAX));
    // shortest split: 8 positions in caches of up to 4096 rows, growing to 32 from 16384 rows
    a.chunk_min = (int)std::min<int64_t>(std::max<int64_t>(len / 512, ZL_ATTN_CHUNK_MIN), 32);
    int nsplit = (int)std::max<int64_t>(1, std::min<int64_t>({cdiv(len, a.chunk_min), want, (int64_t)kMaxSplit}));
    const size_t need = (size_t)a.batch * a.nh * nsplit * (a.D + 2) * sizeof(float);
    if (!a.ws || need > ws_bytes) nsplit = 1;
    a.nsplit = nsplit;
}

static void launch_attn(int kv_dtype, AttnArgs& a, size_t ws_bytes, hipStream_t s, bool qk = false) {
    if (a.batch <= 0 || a.nh <= 0) return;
    const int G = a.nkv > 0 ? a.nh / a.nkv : 0;
    if (!a.q || !a.kc || !a.vc || !a.out || a.nkv <= 0 || a.nh % a.nkv != 0 || a.max_len <= 0) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    const bool shapes = (a.D == 64 || a.D == 128 || a.D == 256 || a.D == 512) &&
                        (G == 1 || G == 2 || G == 4 || G == 8) && (int64_t)a.nkv * a.D <= a.row_stride;
    const int es = kv_dtype == HIP_BRIDGE_BF16 ? 2 : 4;
    const bool aligned = aligned16(a.q) && aligned16(a.kc) && aligned16(a.vc) && (a.row_stride * es) % 16 == 0;
    if ((kv_dtype != HIP_BRIDGE_F32 && kv_dtype != HIP_BRIDGE_BF16) || !shapes || !aligned) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    a.inv_cap = a.softcap > 0.0f ? 1.0f / a.softcap : 0.0f;
    choose_heads(a, kv_dtype == HIP_BRIDGE_BF16 ? 2 : 4);
    choose_split(a, ws_bytes);
    if ((int64_t)a.batch * a.nkv * a.hg * a.nsplit > INT32_MAX) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    if (qk) {
        // QK mode: the rotary pairs must be whole 8-element lane slices a power-of-two number
        // of lanes apart; aligned raw K / V rows and norm weights
        const int hl = a.qk_half / 8;
        const bool rope_ok = a.qk_half == 0 || (a.qk_half % 8 == 0 && (hl & (hl - 1)) == 0 && 2 * a.qk_half <= a.D);
        const bool qk_ok = rope_ok && aligned16(a.qk_k) && aligned16(a.qk_v) && aligned16(a.qk_wq) &&
                           aligned16(a.qk_wk) && (!a.qk_k) == (!a.qk_v);
        if (!qk_ok) {
            set_error(HIP_BRIDGE_EUNSUPPORTED);
            return;
        }
    }
    if (kv_dtype == HIP_BRIDGE_F32) {
        if (a.D == 64) launch_g<float, 64>(a, qk, s);
        else if (a.D == 128) launch_g<float, 128>(a, qk, s);
        else if (a.D == 256) launch_g<float, 256>(a, qk, s);
        else launch_g<float, 512>(a, qk, s);
    } else {
        if (a.D == 64) launch_g<uint16_t, 64>(a, qk, s);
        else if (a.D == 128) launch_g<uint16_t, 128>(a, qk, s);
        else if (a.D == 256) launch_g<uint16_t, 256>(a, qk, s);
        else launch_g<uint16_t, 512>(a, qk, s);
    }
    if (a.nsplit > 1)
        k_attn_merge<<<dim3((unsigned)((int64_t)a.batch * a.nh), (unsigned)(a.D / kMergeCols)), kMergeThreads, 0, s>>>(a);
    check_launch();
}

static AttnArgs base_attn(const float* q, const void* kc, const void* vc, float* out, int n_heads,
                          int n_kv_heads, int head_dim, float scale, float softcap, int window) {
    AttnArgs a{};
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.out = out;
    a.nh = n_heads;
    a.nkv = n_kv_heads;
    a.D = head_dim;
    a.scale = scale;
    a.softcap = softcap;
    a.window = window;
    return a;
}

// ---- the no-allocation variant's scratch -------------------------------------------------
// hip_attention_decode_noalloc keeps its split partials in this file-scope device array
// instead of a caller workspace. Each GPU the library runs on holds its own copy, at its own
// address, until the process ends. Host code never passes the array's name to a kernel (in
// host code that name is a host-side stand-in, not a device address): the device address is
// looked up once per device, with that device current, and cached.
constexpr size_t kScratchBytes = size_t(32) << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchDevices];

// The current device's copy of `scratch`, or null (error recorded).
static void* scratch_on_current_device() {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error((int)e);
        return nullptr;
    }
    if (dev < 0 || dev >= kScratchDevices) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error(e != hipSuccess ? (int)e : HIP_BRIDGE_EINVAL);
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace zl

using namespace zl;

extern "C" {

size_t hip_attention_workspace_bytes(int batch, int n_heads, int n_kv_heads, int head_dim, int max_len,
                                     int sliding_window) {
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_len <= 0) return 0;
    AttnArgs a{};
    a.batch = batch;
    a.nh = n_heads;
    a.nkv = n_kv_heads;
    a.D = head_dim;
    a.max_len = max_len;
    a.window = sliding_window;
    a.ws = reinterpret_cast<float*>(16);  // any non-null pointer: size for the unconstrained split
    if (n_heads % n_kv_heads != 0) return 0;
    size_t need = 0;
    for (int es : {2, 4}) {  // the head grouping (and so the split) depends on the cache type
        choose_heads(a, es);
        choose_split(a, SIZE_MAX);
        if (a.nsplit > 1) need = std::max(need, (size_t)batch * n_heads * a.nsplit * (head_dim + 2) * sizeof(float));
    }
    return need;
}

void hip_attention_decode(int kv_dtype, const float* q, const void* k_cache, const void* v_cache, float* out,
                          int64_t cache_rows, int64_t row_stride, const int64_t* d_row_base, int64_t row_base,
                          const int32_t* d_pos, int pos_base, int max_len, int batch, int n_heads,
                          int n_kv_heads, int head_dim, float attn_scale, float softcap, int sliding_window,
                          void* workspace, size_t workspace_bytes, HipStream_t stream) {
    AttnArgs a = base_attn(q, k_cache, v_cache, out, n_heads, n_kv_heads, head_dim, attn_scale, softcap,
                           sliding_window);
    a.ws = (float*)workspace;
    a.cache_rows = cache_rows;
    a.row_stride = row_stride;
    a.row_base = d_row_base;
    a.row0 = row_base;
    a.pos = d_pos;
    a.pos_base = pos_base;
    a.max_len = max_len;
    a.batch = batch;
    if (!aligned16(workspace)) a.ws = nullptr;
    launch_attn(kv_dtype, a, workspace_bytes, stream_of(stream));
}

void hip_attention_decode_noalloc(int kv_dtype, const float* q, const void* k_cache, const void* v_cache,
                                  float* out, int64_t cache_rows, int64_t row_stride, const int64_t* d_row_base,
                                  int64_t row_base, const int32_t* d_pos, int pos_base, int max_len, int batch,
                                  int n_heads, int n_kv_heads, int head_dim, float attn_scale, float softcap,
                                  int sliding_window, HipStream_t stream) {
    // the split partials the workspace variant would ask for must fit the static scratch
    const size_t need = hip_attention_workspace_bytes(batch, n_heads, n_kv_heads, head_dim, max_len,
                                                      sliding_window);
    if (need > kScratchBytes) {
        set_error(HIP_BRIDGE_ESCRATCH);
        return;
    }
    void* ws = need > 0 ? scratch_on_current_device() : nullptr;
    if (need > 0 && !ws) return;  // error recorded
    hip_attention_decode(kv_dtype, q, k_cache, v_cache, out, cache_rows, row_stride, d_row_base, row_base, d_pos,
                         pos_base, max_len, batch, n_heads, n_kv_heads, head_dim, attn_scale, softcap,
                         sliding_window, ws, ws ? kScratchBytes : 0, stream);
}

void hip_attention_decode_qk(int kv_dtype, const float* q, const float* k, const float* v,
                             const float* q_norm_w, const float* k_norm_w, int v_norm, void* k_cache,
                             void* v_cache, float* out, int64_t cache_rows, int64_t row_stride,
                             const int64_t* d_row_base, int64_t row_base, const int32_t* d_pos, int pos_base,
                             int max_len, int batch, int n_heads, int n_kv_heads, int head_dim, int rotary_dim,
                             float freq_base, float freq_scale, float eps, int use_unit_offset, float attn_scale,
                             float softcap, int sliding_window, void* workspace, size_t workspace_bytes,
                             HipStream_t stream) {
    AttnArgs a = base_attn(q, k_cache, v_cache, out, n_heads, n_kv_heads, head_dim, attn_scale, softcap,
                           sliding_window);
    a.ws = aligned16(workspace) ? (float*)workspace : nullptr;
    a.cache_rows = cache_rows;
    a.row_stride = row_stride;
    a.row_base = d_row_base;
    a.row0 = row_base;
    a.pos = d_pos;
    a.pos_base = pos_base;
    a.max_len = max_len;
    a.batch = batch;
    a.qk_k = k;
    a.qk_v = v;
    a.qk_wq = q_norm_w;
    a.qk_wk = k_norm_w;
    a.qk_vnorm = v_norm;
    a.qk_uo = use_unit_offset;
    const int eff = (rotary_dim <= 0 || rotary_dim > head_dim) ? head_dim : rotary_dim;
    a.qk_half = eff / 2;
    a.qk_eps = eps;
    a.qk_freq_scale = freq_scale;
    a.qk_log2_base = log2((double)freq_base);
    launch_attn(kv_dtype, a, workspace_bytes, stream_of(stream), true);
}

void hip_attention_forward(const float* q, const float* k_cache, const float* v_cache, float* out,
                           int donor_layer, int pos, int max_seq, int n_heads, int n_kv_heads, int head_dim,
                           int max_kv_dim, float attn_scale, float softcap, int sliding_window,
                           HipStream_t stream) {
    hip_attention_batched(q, k_cache, v_cache, out, donor_layer, pos, 1, max_seq, n_heads, n_kv_heads,
                          head_dim, max_kv_dim, attn_scale, softcap, sliding_window, stream);
}

void hip_attention_forward_ind(const float* q, const float* k_cache, const float* v_cache, float* out,
                               int donor_layer, const int* d_pos, int max_seq, int n_heads, int n_kv_heads,
                               int head_dim, int max_kv_dim, float attn_scale, float softcap,
                               int sliding_window, HipStream_t stream) {
    if (!d_pos) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    AttnArgs a = base_attn(q, k_cache, v_cache, out, n_heads, n_kv_heads, head_dim, attn_scale, softcap,
                           sliding_window);
    a.row0 = (int64_t)donor_layer * max_seq;
    a.row_stride = max_kv_dim;
    a.pos = d_pos;
    a.max_len = max_seq;
    a.batch = 1;
    launch_attn(HIP_BRIDGE_F32, a, 0, stream_of(stream));
}

void hip_attention_batched(const float* q, const float* k_cache, const float* v_cache, float* out,
                           int donor_layer, int pos, int batch_size, int max_seq, int n_heads, int n_kv_heads,
                           int head_dim, int max_kv_dim, float attn_scale, float softcap, int sliding_window,
                           HipStream_t stream) {
    if (batch_size <= 0) return;
    AttnArgs a = base_attn(q, k_cache, v_cache, out, n_heads, n_kv_heads, head_dim, attn_scale, softcap,
                           sliding_window);
    a.row0 = (int64_t)donor_layer * max_seq;
    a.row_stride = max_kv_dim;
    a.pos_base = pos;
    a.max_len = max_seq;
    a.batch = batch_size;
    launch_attn(HIP_BRIDGE_F32, a, 0, stream_of(stream));
}

}  // extern "C"
