// RMSNorm family (replaces cuda_bridge.cu:1451-1553, 1942-2068) with ziglm's CPU numerics
// (math.zig:850-988): sum of squares in f32, mean = sum/n (IEEE divide), inv = 1/sqrt(mean +
// eps), out = (x*inv)*(1+w) | (x*inv)*w | x*inv (weight NULL). The register-row kernels take
// 1/sqrt from the hardware reciprocal square root (within 1 ulp of the reference's IEEE sqrt
// and divide; 2048 x 2560 bf16: input norm 4.28 -> 4.19 us, norm + add + norm 8.15 -> 7.92);
// the generic kernel keeps the IEEE form.
//
// Modes (one kernel family):
//   NORM           out = norm(x)                                   (rmsNorm, rmsNormBatched)
//   ADD_NORM       s = x + r; x = s; out = norm(s)                 (addRmsNorm, model.zig:714-723)
//   NORM_ADD       x = x + norm(r)                                 (rmsnormAdd, model.zig:748-755)
//   NORM_ADD_NORM  s = x + norm(r; w1); x = s; out = norm(s; w2)   (post-attn norm + add +
//                  pre-FFN norm, cuda_model.zig:930-942; post-FFN norm + add + next input norm)
// The whole row lives in registers: W = 1, 2 or 4 waves per row (wave reductions by
// DPP/permlane, then a W-float LDS exchange); a lane owns chunks g, g+64W, ... so x and r
// are read from HBM once and x/out written once, with every load of the row issued before
// the first use. The weights (f32,
// shared by all rows, L2-resident) are loaded as 128-bit vectors up front and turned into
// per-element factors (1+w), w or 1. Rows that are not 16-byte aligned, or longer than 16
// chunks per lane (f32 > 16384, bf16 > 32768 elements), use a block-per-row kernel that
// re-reads the row from L2. Launches of many rounds of 4-wave rows (prefill at 8192 tokens)
// run persistent workgroups that walk the rows with the next row's loads in flight
// (k_norm_pipe; k_norm_pipe_nan for NORM_ADD_NORM), with the same arithmetic.
// Aliasing: out may alias r (the reference calls addRmsNorm(x, xb, w, out=xb)) or x in
// NORM mode; every lane reads its chunks before writing the same chunks.
#include "zl_common.h"
#include "zl_host.h"

#include <algorithm>
#include <type_traits>

namespace zl {

enum NormMode { M_NORM = 0, M_ADD_NORM = 1, M_NORM_ADD = 2, M_NORM_ADD_NORM = 3 };

struct NormArgs {
    void* x;          // NORM: input (read only); otherwise the residual stream (updated)
    const void* r;    // ADD_NORM: residual; NORM_ADD: input to normalise; NORM_ADD_NORM: xb
    const float* w1;  // weight of the first norm (NULL: no scale)
    const float* w2;  // weight of the second norm (NORM_ADD_NORM only)
    void* out;
    int64_t rows;
    int n;
    float eps;
    int uo;           // use_unit_offset: scale by (1 + w)
};

// (v * inv) * wf with wf = 1 + w, w, or absent.
__device__ __forceinline__ float apply_w(float v, float inv, const float* w, int i, int uo, bool has_w) {
    const float y = v * inv;
    if (!has_w) return y;
    const float wi = w[i];
    return uo ? y * (1.0f + wi) : y * wi;
}

// Sum over the W waves of a row: wave reduction, then (W > 1) the W partials through LDS,
// added in wave order. Each reduction of a kernel uses its own LDS slot, so one barrier per
// reduction suffices (no slot is rewritten while another wave may still read it).
template <int W>
__device__ __forceinline__ float row_sum(float v, float* slot) {
    v = group_sum<kWave>(v);
    if constexpr (W == 1) {
        return v;
    } else {
        const int wave = (threadIdx.x >> 6) % W;
        if ((threadIdx.x & 63) == 0) slot[wave] = v;
        __syncthreads();
        float t = slot[0];
#pragma unroll
        for (int i = 1; i < W; ++i) t += slot[i];
        return t;
    }
}

// row_sum of R rows at once: slots[r] is row r's slot set; one barrier for all of them.
template <int W, int R>
__device__ __forceinline__ void row_sums(float (&v)[R], float* const (&slots)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = group_sum<kWave>(v[r]);
    if constexpr (W > 1) {
        const int wave = (threadIdx.x >> 6) % W;
        if ((threadIdx.x & 63) == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) slots[r][wave] = v[r];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float t = slots[r][0];
#pragma unroll
            for (int i = 1; i < W; ++i) t += slots[r][i];
            v[r] = t;
        }
    }
}

// W waves per row group (W in {1, 2, 4}), 256 threads per block, 4/W row groups per block,
// R consecutive rows per group (R in {1, 2}). Lane g of a group (g in [0, 64W)) owns chunks
// g, g + 64W, ... (NC of them at most) of each of its R rows, so it loads the weights of
// those chunks once for R rows: the weights are f32 while bf16 rows are 2 bytes an element,
// and at one row per lane their reads through the L1/L2 path cost up to 14% of the kernel
// (8192 x 5376 bf16, measured). All rows' HBM loads are issued first; row r+1's loads are
// in flight while row r is reduced and stored.
#ifndef ZL_NORM_GROUPS_PER_BLOCK
#define ZL_NORM_GROUPS_PER_BLOCK 0
#endif
template <int W>
__host__ __device__ constexpr int norm_gpb() {
    return ZL_NORM_GROUPS_PER_BLOCK ? ZL_NORM_GROUPS_PER_BLOCK : 4 / W;
}

// Cache policy of the row loads and stores (zl_common.h POL_*; tuning builds set others).
#ifndef ZL_NORM_LP
#define ZL_NORM_LP POL_NT
#endif
#ifndef ZL_NORM_SP
#define ZL_NORM_SP POL_NT
#endif

#ifndef ZL_NORM_STAGED
#define ZL_NORM_STAGED 1
#endif
// NORM_ADD_NORM with late weights: the second norm's weights are requested after the first
// reduction, not with the first norm's (2048 x 2560 bf16, four runs: 8.43 -> 8.29 us; 8192 x
// 5376 unchanged). ZL_NORM_W2_LATE=0 loads both together.
#ifndef ZL_NORM_W2_LATE
#define ZL_NORM_W2_LATE 1
#endif
template <typename T, int NC, int MODE, int W, int R, bool WL>
__global__ __launch_bounds__(256) void k_norm_rows(NormArgs a) {
    using C = Chunk<T>;
    constexpr int E = C::E;
    // Rows reduced stage by stage (one barrier per reduction for all R rows instead of one
    // per row and reduction), for the two-input modes at 4 waves per row: 8192 x 5376 bf16
    // norm + add + norm 62.3 -> 61.2 us, add + norm 61.5 -> 60.9 us; slower at 2 waves per
    // row (2048 x 2560: 8.32 -> 8.63 us, 7.55 -> 7.68 us) and for the plain norm (31.9 ->
    // 32.3 us), which keep the row-by-row order. ZL_NORM_STAGED=0 turns it off.
    constexpr bool STAGED = ZL_NORM_STAGED && W == 4 && R > 1 && MODE != M_NORM;
    constexpr int LP = ZL_NORM_LP, SP = ZL_NORM_SP;
    constexpr int GPB = norm_gpb<W>();  // row groups per block
    constexpr int STRIDE = kWave * W;
    // one slot set per (row, reduction): no slot is rewritten while a wave may still read it
    __shared__ float s_red[2 * R][W * GPB];
    const int rib = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) / W);  // group within block (wave-uniform)
    const int g = threadIdx.x - rib * STRIDE;
    const int64_t row0 = ((int64_t)blockIdx.x * GPB + rib) * R;
    const int n = a.n;
    const int nch = n / E;
    const bool has_w1 = a.w1 != nullptr;
    const bool has_w2 = a.w2 != nullptr;

    // Issue every HBM load of the group's rows, then the (L2-resident) weights, all through
    // range-checked buffer loads (bld16): chunks past a row's end, and rows past the
    // tensor's, read as zeros with no branch, so every load is in flight before the first
    // wait. Their slots are never used.
    u32x4 rx[R][NC], rr[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = row0 + r;
        const uint32_t bytes = row < a.rows ? (uint32_t)n * sizeof(T) : 0u;
        const auto rsx = buf_rsrc((const T*)a.x + row * n, bytes);
        const auto rsr = buf_rsrc((const T*)a.r + row * n, MODE != M_NORM ? bytes : 0u);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint32_t off = (uint32_t)(g + c * STRIDE) * 16u;
            rx[r][c] = bldp<LP>(rsx, off);
            if constexpr (MODE != M_NORM) rr[r][c] = bldp<LP>(rsr, off);
        }
    }
    // Weights: with the activations (WL false: latency-bound launches, one round trip in
    // all) or once the first row's activations have arrived (WL true: launches with every
    // row resident at once, where thousands of waves asking for the same weight lines in the
    // same instant queue behind each other; measured on 2048 x 2560 bf16 rows, input norm
    // 5.84 -> 4.62 us).
    float f1[NC][E];
    float f2[MODE == M_NORM_ADD_NORM ? NC : 1][E];
    constexpr bool W2L = ZL_NORM_W2_LATE && WL && MODE == M_NORM_ADD_NORM;
    auto load_w2 = [&]() {
        if constexpr (MODE == M_NORM_ADD_NORM) {
            const auto rsw2 = buf_rsrc(a.w2, has_w2 ? (uint32_t)n * 4u : 0u);
#pragma unroll
            for (int c = 0; c < NC; ++c) load_wb<E>(rsw2, (uint32_t)(g + c * STRIDE) * E * 4u, f2[c]);
        }
    };
    auto load_weights = [&]() {
        const uint32_t wbytes = (uint32_t)n * 4u;
        const auto rsw1 = buf_rsrc(a.w1, has_w1 ? wbytes : 0u);
#pragma unroll
        for (int c = 0; c < NC; ++c) load_wb<E>(rsw1, (uint32_t)(g + c * STRIDE) * E * 4u, f1[c]);
        if constexpr (!W2L) load_w2();
    };
    if constexpr (!WL) load_weights();

    if constexpr (STAGED) {
        // Stage by stage over the R rows: every row's first sums, one barrier for all of
        // them; (NORM_ADD_NORM) every row's second sums, one barrier; then the stores.
        float v[R][NC][E];
        float ss[R];
        float* s1[R];
        float* s2[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool row_ok = row0 + r < a.rows;
            s1[r] = s_red[2 * r] + rib * W;
            s2[r] = s_red[2 * r + 1] + rib * W;
            ss[r] = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (row_ok && idx < nch) {
                    if constexpr (MODE == M_NORM) {
                        C::unpack(rx[r][c], v[r][c]);
                    } else if constexpr (MODE == M_ADD_NORM) {
                        float xv[E], rv[E];
                        C::unpack(rx[r][c], xv);
                        C::unpack(rr[r][c], rv);
#pragma unroll
                        for (int j = 0; j < E; ++j) v[r][c][j] = xv[j] + rv[j];
                    } else {
                        C::unpack(rr[r][c], v[r][c]);
                    }
#pragma unroll
                    for (int j = 0; j < E; ++j) ss[r] = fmaf(v[r][c][j], v[r][c][j], ss[r]);
                }
            }
            if constexpr (WL) {
                if (r == 0) load_weights();
            }
        }
        row_sums<W, R>(ss, s1);
        if constexpr (W2L) load_w2();
        float inv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) inv[r] = rms_inv_hw(ss[r], n, a.eps);
        if constexpr (MODE == M_NORM_ADD_NORM) {
            float ss2[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const bool row_ok = row0 + r < a.rows;
                ss2[r] = 0.0f;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const int idx = g + c * STRIDE;
                    if (row_ok && idx < nch) {
                        float xv[E];
                        C::unpack(rx[r][c], xv);
#pragma unroll
                        for (int j = 0; j < E; ++j) {
                            v[r][c][j] = xv[j] + (v[r][c][j] * inv[r]) * w_factor(f1[c][j], has_w1, a.uo);
                            ss2[r] = fmaf(v[r][c][j], v[r][c][j], ss2[r]);
                        }
                    }
                }
            }
            row_sums<W, R>(ss2, s2);
#pragma unroll
            for (int r = 0; r < R; ++r) inv[r] = rms_inv_hw(ss2[r], n, a.eps);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = row0 + r;
            const bool row_ok = row < a.rows;
            const uint32_t row_bytes = row_ok ? (uint32_t)n * sizeof(T) : 0u;
            T* const xrow = (T*)a.x + row * n;
            T* const orow = (T*)a.out + row * n;
            const auto wsx = buf_rsrc(xrow, MODE != M_NORM ? row_bytes : 0u);
            const auto wso = buf_rsrc(orow, MODE != M_NORM_ADD ? row_bytes : 0u);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (!(row_ok && idx < nch)) continue;
                if constexpr (MODE == M_NORM_ADD) {
                    float xv[E];
                    C::unpack(rx[r][c], xv);
#pragma unroll
                    for (int j = 0; j < E; ++j) xv[j] = xv[j] + (v[r][c][j] * inv[r]) * w_factor(f1[c][j], has_w1, a.uo);
                    strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(xv));
                } else {
                    float y[E];
                    if constexpr (MODE == M_NORM_ADD_NORM) {
#pragma unroll
                        for (int j = 0; j < E; ++j) y[j] = (v[r][c][j] * inv[r]) * w_factor(f2[c][j], has_w2, a.uo);
                    } else {
#pragma unroll
                        for (int j = 0; j < E; ++j) y[j] = (v[r][c][j] * inv[r]) * w_factor(f1[c][j], has_w1, a.uo);
                    }
                    if constexpr (MODE != M_NORM) strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(v[r][c]));
                    strow16<SP>(orow, wso, (uint32_t)idx * 16u, C::pack(y));
                }
            }
        }
        return;
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = row0 + r;
        const bool row_ok = row < a.rows;
        const uint32_t row_bytes = row_ok ? (uint32_t)n * sizeof(T) : 0u;
        T* const xrow = (T*)a.x + row * n;
        T* const orow = (T*)a.out + row * n;
        const auto wsx = buf_rsrc(xrow, MODE != M_NORM ? row_bytes : 0u);
        const auto wso = buf_rsrc(orow, MODE != M_NORM_ADD ? row_bytes : 0u);
        float* slot1 = s_red[2 * r] + rib * W;
        float* slot2 = s_red[2 * r + 1] + rib * W;

        // v: the vector normalised first.
        float v[NC][E];
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int idx = g + c * STRIDE;
            if (row_ok && idx < nch) {
                if constexpr (MODE == M_NORM) {
                    C::unpack(rx[r][c], v[c]);
                } else if constexpr (MODE == M_ADD_NORM) {
                    float xv[E], rv[E];
                    C::unpack(rx[r][c], xv);
                    C::unpack(rr[r][c], rv);
#pragma unroll
                    for (int j = 0; j < E; ++j) v[c][j] = xv[j] + rv[j];
                } else {
                    C::unpack(rr[r][c], v[c]);
                }
#pragma unroll
                for (int j = 0; j < E; ++j) ss = fmaf(v[c][j], v[c][j], ss);
            }
        }
        if constexpr (WL) {
            if (r == 0) load_weights();
        }
        ss = row_sum<W>(ss, slot1);
        if constexpr (W2L) {
            if (r == 0) load_w2();
        }
        const float inv = rms_inv_hw(ss, n, a.eps);

        if constexpr (MODE == M_NORM || MODE == M_ADD_NORM) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (row_ok && idx < nch) {
                    float y[E];
#pragma unroll
                    for (int j = 0; j < E; ++j) y[j] = (v[c][j] * inv) * w_factor(f1[c][j], has_w1, a.uo);
                    if constexpr (MODE == M_ADD_NORM) strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(v[c]));
                    strow16<SP>(orow, wso, (uint32_t)idx * 16u, C::pack(y));
                }
            }
        } else if constexpr (MODE == M_NORM_ADD) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (row_ok && idx < nch) {
                    float xv[E];
                    C::unpack(rx[r][c], xv);
#pragma unroll
                    for (int j = 0; j < E; ++j) xv[j] = xv[j] + (v[c][j] * inv) * w_factor(f1[c][j], has_w1, a.uo);
                    strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(xv));
                }
            }
        } else {  // M_NORM_ADD_NORM
            float ss2 = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (row_ok && idx < nch) {
                    float xv[E];
                    C::unpack(rx[r][c], xv);
#pragma unroll
                    for (int j = 0; j < E; ++j) {
                        v[c][j] = xv[j] + (v[c][j] * inv) * w_factor(f1[c][j], has_w1, a.uo);
                        ss2 = fmaf(v[c][j], v[c][j], ss2);
                    }
                }
            }
            ss2 = row_sum<W>(ss2, slot2);
            const float inv2 = rms_inv_hw(ss2, n, a.eps);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (row_ok && idx < nch) {
                    float y[E];
#pragma unroll
                    for (int j = 0; j < E; ++j) y[j] = (v[c][j] * inv2) * w_factor(f2[c][j], has_w2, a.uo);
                    strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(v[c]));
                    strow16<SP>(orow, wso, (uint32_t)idx * 16u, C::pack(y));
                }
            }
        }
    }
}

// Persistent, software-pipelined form for launches of several rounds of 4-wave rows: as many
// workgroups as stay resident, each walking rows blockIdx.x, blockIdx.x + gridDim.x, ...,
// with the next row's loads issued before the current row is reduced and stored, so a
// workgroup keeps a row in flight from its first load to its last store instead of
// alternating between a load phase and a reduce / store phase; the norm factors are loaded
// once per workgroup. Same arithmetic, in the same order, as k_norm_rows at 4 waves per row.
// The loop is unrolled by two so that both register buffers have compile-time indices; the
// reduction slots alternate with them (a wave that runs ahead into the next row writes the
// other slot set, and cannot reach the row after it before every wave has passed the next
// row's barrier). Rows go round-robin over the workgroups, so the rows in flight at any time
// are neighbours. Measured at 8192 x 5376 bf16 and not taken (us, input norm / add + norm /
// norm + add, against 29.7 / 58.5 / 42.9): a contiguous range of rows per workgroup 35.5 /
// 67.3 / 50.3; default-policy loads 31.7 / 62.4 / 49.8; three row buffers (two rows in
// flight) at the same workgroup counts 31.6 / 59.2 / 45.3, at one workgroup per CU 31.7 /
// 59.6 / 42.8; two rows per step reduced stage by stage (one barrier per reduction for both)
// 30.1 / 59.8 / 43.3 at the best of 1, 2 and the default workgroups per CU.
template <typename T, int NC, int MODE>
__global__ __launch_bounds__(256) void k_norm_pipe(NormArgs a) {
    using C = Chunk<T>;
    constexpr int E = C::E;
    constexpr int W = 4;
    constexpr int STRIDE = kWave * W;
    constexpr int LP = ZL_NORM_LP, SP = ZL_NORM_SP;
    __shared__ float s_red[2][2][W];  // [buffer][reduction][wave]
    const int g = threadIdx.x;
    const int n = a.n;
    const int nch = n / E;
    const uint32_t row_bytes = (uint32_t)n * sizeof(T);
    const bool has_w1 = a.w1 != nullptr;
    const bool has_w2 = a.w2 != nullptr;
    const int64_t end = a.rows;
    const int64_t step = gridDim.x;

    u32x4 bx[2][NC], br[2][NC];
    // every load of a row through range-checked resources (rows past the tensor read zeros)
    auto issue = [&](auto B, int64_t row) {
        constexpr int b = decltype(B)::value;
        const bool ok = row < end;
        const int64_t rr = ok ? row : 0;
        const auto rsx = buf_rsrc((const T*)a.x + rr * n, ok ? row_bytes : 0u);
        const auto rsr = buf_rsrc((const T*)a.r + rr * n, ok && MODE != M_NORM ? row_bytes : 0u);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint32_t off = (uint32_t)(g + c * STRIDE) * 16u;
            bx[b][c] = bldp<LP>(rsx, off);
            if constexpr (MODE != M_NORM) br[b][c] = bldp<LP>(rsr, off);
        }
    };
    float f1[NC][E];
    float f2[MODE == M_NORM_ADD_NORM ? NC : 1][E];

    // one row (row < a.rows, block-uniform) from buffer B
    auto process = [&](auto B, int64_t row) {
        constexpr int b = decltype(B)::value;
        T* const xrow = (T*)a.x + row * n;
        T* const orow = (T*)a.out + row * n;
        const auto wsx = buf_rsrc(xrow, MODE != M_NORM ? row_bytes : 0u);
        const auto wso = buf_rsrc(orow, MODE != M_NORM_ADD ? row_bytes : 0u);
        float v[NC][E];
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (g + c * STRIDE < nch) {
                if constexpr (MODE == M_NORM) {
                    C::unpack(bx[b][c], v[c]);
                } else if constexpr (MODE == M_ADD_NORM) {
                    float xv[E], rv[E];
                    C::unpack(bx[b][c], xv);
                    C::unpack(br[b][c], rv);
#pragma unroll
                    for (int j = 0; j < E; ++j) v[c][j] = xv[j] + rv[j];
                } else {
                    C::unpack(br[b][c], v[c]);
                }
#pragma unroll
                for (int j = 0; j < E; ++j) ss = fmaf(v[c][j], v[c][j], ss);
            }
        }
        ss = row_sum<W>(ss, s_red[b][0]);
        const float inv = rms_inv_hw(ss, n, a.eps);
        if constexpr (MODE == M_NORM || MODE == M_ADD_NORM) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (idx < nch) {
                    float y[E];
#pragma unroll
                    for (int j = 0; j < E; ++j) y[j] = (v[c][j] * inv) * w_factor(f1[c][j], has_w1, a.uo);
                    if constexpr (MODE == M_ADD_NORM) strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(v[c]));
                    strow16<SP>(orow, wso, (uint32_t)idx * 16u, C::pack(y));
                }
            }
        } else if constexpr (MODE == M_NORM_ADD) {
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (idx < nch) {
                    float xv[E];
                    C::unpack(bx[b][c], xv);
#pragma unroll
                    for (int j = 0; j < E; ++j) xv[j] = xv[j] + (v[c][j] * inv) * w_factor(f1[c][j], has_w1, a.uo);
                    strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(xv));
                }
            }
        } else {  // M_NORM_ADD_NORM
            float ss2 = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                if (g + c * STRIDE < nch) {
                    float xv[E];
                    C::unpack(bx[b][c], xv);
#pragma unroll
                    for (int j = 0; j < E; ++j) {
                        v[c][j] = xv[j] + (v[c][j] * inv) * w_factor(f1[c][j], has_w1, a.uo);
                        ss2 = fmaf(v[c][j], v[c][j], ss2);
                    }
                }
            }
            ss2 = row_sum<W>(ss2, s_red[b][1]);
            const float inv2 = rms_inv_hw(ss2, n, a.eps);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int idx = g + c * STRIDE;
                if (idx < nch) {
                    float y[E];
#pragma unroll
                    for (int j = 0; j < E; ++j) y[j] = (v[c][j] * inv2) * w_factor(f2[c][j], has_w2, a.uo);
                    strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(v[c]));
                    strow16<SP>(orow, wso, (uint32_t)idx * 16u, C::pack(y));
                }
            }
        }
    };

    constexpr std::integral_constant<int, 0> B0{};
    constexpr std::integral_constant<int, 1> B1{};
    int64_t row = blockIdx.x;
    issue(B0, row);
    // the weights once, behind the first row's loads
    {
        const auto rsw1 = buf_rsrc(a.w1, has_w1 ? (uint32_t)n * 4u : 0u);
#pragma unroll
        for (int c = 0; c < NC; ++c) load_wb<E>(rsw1, (uint32_t)(g + c * STRIDE) * E * 4u, f1[c]);
        if constexpr (MODE == M_NORM_ADD_NORM) {
            const auto rsw2 = buf_rsrc(a.w2, has_w2 ? (uint32_t)n * 4u : 0u);
#pragma unroll
            for (int c = 0; c < NC; ++c) load_wb<E>(rsw2, (uint32_t)(g + c * STRIDE) * E * 4u, f2[c]);
        }
    }
    // one row in flight while another is reduced and stored
    while (row < end) {
        issue(B1, row + step);
        process(B0, row);
        row += step;
        if (row >= end) break;
        issue(B0, row + step);
        process(B1, row);
        row += step;
    }
}

// NORM_ADD_NORM in the persistent, pipelined form with one barrier per row: row q's first
// statistic and the pending row p's second statistic (p the row before q in this
// workgroup's walk) are exchanged behind the same barrier, then p is stored and q's sum s =
// x + norm1(r) formed, whose second statistic waits for the next row. Same arithmetic, in
// the same order, as k_norm_rows.
template <typename T, int NC>
__global__ __launch_bounds__(256) void k_norm_pipe_nan(NormArgs a) {
    using C = Chunk<T>;
    constexpr int E = C::E;
    constexpr int W = 4;
    constexpr int STRIDE = kWave * W;
    constexpr int LP = ZL_NORM_LP, SP = ZL_NORM_SP;
    __shared__ float s_red[2][2][W];  // [parity][row p / row q][wave]
    const int g = threadIdx.x;
    const int n = a.n;
    const int nch = n / E;
    const uint32_t row_bytes = (uint32_t)n * sizeof(T);
    const bool has_w1 = a.w1 != nullptr;
    const bool has_w2 = a.w2 != nullptr;
    const int64_t end = a.rows;
    const int64_t step = gridDim.x;

    u32x4 bx[2][NC], br[2][NC];
    auto issue = [&](auto B, int64_t row) {
        constexpr int b = decltype(B)::value;
        const bool ok = row < end;
        const int64_t rr = ok ? row : 0;
        const auto rsx = buf_rsrc((const T*)a.x + rr * n, ok ? row_bytes : 0u);
        const auto rsr = buf_rsrc((const T*)a.r + rr * n, ok ? row_bytes : 0u);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint32_t off = (uint32_t)(g + c * STRIDE) * 16u;
            bx[b][c] = bldp<LP>(rsx, off);
            br[b][c] = bldp<LP>(rsr, off);
        }
    };
    float f1[NC][E], f2[NC][E];
    float sv[NC][E];  // s = x + norm1(r) of the pending row
    float ss2 = 0.0f;  // its second statistic, this lane's part
    // this lane's part of row q's first statistic (buffer B)
    auto first_sum = [&](auto B) -> float {
        constexpr int b = decltype(B)::value;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (g + c * STRIDE < nch) {
                float v[E];
                C::unpack(br[b][c], v);
#pragma unroll
                for (int j = 0; j < E; ++j) ss = fmaf(v[j], v[j], ss);
            }
        }
        return ss;
    };
    // s of row q (buffer B) with inv1, and this lane's part of its second statistic
    auto form_s = [&](auto B, float inv) {
        constexpr int b = decltype(B)::value;
        ss2 = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (g + c * STRIDE < nch) {
                float xv[E], v[E];
                C::unpack(bx[b][c], xv);
                C::unpack(br[b][c], v);
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    sv[c][j] = xv[j] + (v[j] * inv) * w_factor(f1[c][j], has_w1, a.uo);
                    ss2 = fmaf(sv[c][j], sv[c][j], ss2);
                }
            }
        }
    };
    auto store_p = [&](int64_t row, float inv2) {
        T* const xrow = (T*)a.x + row * n;
        T* const orow = (T*)a.out + row * n;
        const auto wsx = buf_rsrc(xrow, row_bytes);
        const auto wso = buf_rsrc(orow, row_bytes);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int idx = g + c * STRIDE;
            if (idx < nch) {
                float y[E];
#pragma unroll
                for (int j = 0; j < E; ++j) y[j] = (sv[c][j] * inv2) * w_factor(f2[c][j], has_w2, a.uo);
                strow16<SP>(xrow, wsx, (uint32_t)idx * 16u, C::pack(sv[c]));
                strow16<SP>(orow, wso, (uint32_t)idx * 16u, C::pack(y));
            }
        }
    };
    // one iteration: pending row p (sv, ss2), row q = p + step in buffer B, the other
    // buffer free; slots of parity P
    auto iter = [&](auto B, auto Bo, int64_t p, int P) {
        constexpr int b = decltype(B)::value;
        const int64_t q = p + step;
        issue(Bo, q + step);
        float two[2] = {ss2, first_sum(B)};
        float* const slots[2] = {s_red[P][0], s_red[P][1]};
        row_sums<W, 2>(two, slots);
        const float inv2 = rms_inv_hw(two[0], n, a.eps);
        const float inv1 = rms_inv_hw(two[1], n, a.eps);
        store_p(p, inv2);
        form_s(B, inv1);
        (void)b;
    };

    constexpr std::integral_constant<int, 0> B0{};
    constexpr std::integral_constant<int, 1> B1{};
    int64_t p = blockIdx.x;
    if (p >= end) return;  // block-uniform
    issue(B0, p);
    {
        const auto rsw1 = buf_rsrc(a.w1, has_w1 ? (uint32_t)n * 4u : 0u);
        const auto rsw2 = buf_rsrc(a.w2, has_w2 ? (uint32_t)n * 4u : 0u);
#pragma unroll
        for (int c = 0; c < NC; ++c) load_wb<E>(rsw1, (uint32_t)(g + c * STRIDE) * E * 4u, f1[c]);
#pragma unroll
        for (int c = 0; c < NC; ++c) load_wb<E>(rsw2, (uint32_t)(g + c * STRIDE) * E * 4u, f2[c]);
    }
    issue(B1, p + step);
    // the first row's first statistic alone
    {
        float one = first_sum(B0);
        one = row_sum<W>(one, s_red[1][0]);
        form_s(B0, rms_inv_hw(one, n, a.eps));
    }
    // pending p; row p + step in B1, B0 free
    int P = 0;
    while (true) {
        if (p + step >= end) break;
        iter(B1, B0, p, P);
        p += step;
        P ^= 1;
        if (p + step >= end) break;
        iter(B0, B1, p, P);
        p += step;
        P ^= 1;
    }
    // the last pending row's second statistic alone
    const float last = row_sum<W>(ss2, s_red[P][0]);
    store_p(p, rms_inv_hw(last, n, a.eps));
}

// ---- block-per-row fallback: any n, any alignment ------------------------------------------

template <typename T>
__device__ __forceinline__ float ld1(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld1<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ld1<uint16_t>(const uint16_t* p, int64_t i) { return bf16_lo(p[i]); }

template <typename T>
__device__ __forceinline__ void st1(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st1<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void st1<uint16_t>(uint16_t* p, int64_t i, float v) {
    p[i] = (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu);
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = group_sum<kWave>(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    const float t = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return t;
}

template <typename T, int MODE>
__global__ __launch_bounds__(256) void k_norm_rows_generic(NormArgs a) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int n = a.n;
    T* xrow = (T*)a.x + row * n;
    const T* rrow = (const T*)a.r + row * n;
    T* orow = (T*)a.out + row * n;
    const bool has_w1 = a.w1 != nullptr;
    const bool has_w2 = a.w2 != nullptr;

    auto first = [&](int i) -> float {
        if constexpr (MODE == M_NORM) return ld1(xrow, i);
        else if constexpr (MODE == M_ADD_NORM) return ld1(xrow, i) + ld1(rrow, i);
        else return ld1(rrow, i);
    };
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = first(i);
        ss = fmaf(v, v, ss);
    }
    const float inv = rms_inv(block_sum256(ss, red), n, a.eps);

    if constexpr (MODE == M_NORM || MODE == M_ADD_NORM) {
        for (int i = threadIdx.x; i < n; i += 256) {
            const float v = first(i);
            const float y = apply_w(v, inv, a.w1, i, a.uo, has_w1);
            if constexpr (MODE == M_ADD_NORM) st1(xrow, i, v);
            st1(orow, i, y);
        }
    } else if constexpr (MODE == M_NORM_ADD) {
        for (int i = threadIdx.x; i < n; i += 256) {
            const float v = first(i);
            st1(xrow, i, ld1(xrow, i) + apply_w(v, inv, a.w1, i, a.uo, has_w1));
        }
    } else {
        // Pass 2 computes s = x + norm1(xb) for the second statistic; pass 3 recomputes s
        // with the same f32 operations (x is only overwritten in pass 3).
        float ss2 = 0.0f;
        for (int i = threadIdx.x; i < n; i += 256) {
            const float s = ld1(xrow, i) + apply_w(first(i), inv, a.w1, i, a.uo, has_w1);
            ss2 = fmaf(s, s, ss2);
        }
        const float inv2 = rms_inv(block_sum256(ss2, red), n, a.eps);
        for (int i = threadIdx.x; i < n; i += 256) {
            const float s = ld1(xrow, i) + apply_w(first(i), inv, a.w1, i, a.uo, has_w1);
            st1(xrow, i, s);
            st1(orow, i, apply_w(s, inv2, a.w2, i, a.uo, has_w2));
        }
    }
}

template <typename T, int MODE, int W, bool WL>
static void launch_w(const NormArgs& a, int per_lane, int R, hipStream_t s) {
    constexpr int GPB = norm_gpb<W>();
    constexpr int NT = 64 * W * GPB;
    const unsigned grid = (unsigned)cdiv(a.rows, (int64_t)GPB * R);
    // NC = chunks per lane, fitted to the row (the register footprint, and so the occupancy,
    // grows with NC); two rows per lane group up to 4 chunks per lane
    if (R == 2 && per_lane <= 4) {
        if (per_lane <= 1) k_norm_rows<T, 1, MODE, W, 2, WL><<<grid, NT, 0, s>>>(a);
        else if (per_lane <= 2) k_norm_rows<T, 2, MODE, W, 2, WL><<<grid, NT, 0, s>>>(a);
        else if (per_lane <= 3) k_norm_rows<T, 3, MODE, W, 2, WL><<<grid, NT, 0, s>>>(a);
        else k_norm_rows<T, 4, MODE, W, 2, WL><<<grid, NT, 0, s>>>(a);
        return;
    }
    const unsigned grid1 = (unsigned)cdiv(a.rows, GPB);
    if (per_lane <= 1) k_norm_rows<T, 1, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
    else if (per_lane <= 2) k_norm_rows<T, 2, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
    else if (per_lane <= 3) k_norm_rows<T, 3, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
    else if (per_lane <= 4) k_norm_rows<T, 4, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
    else if (per_lane <= 5 && MODE == M_NORM_ADD) k_norm_rows<T, 5, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
    else if (per_lane <= 6) k_norm_rows<T, 6, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
    else if (per_lane <= 8) k_norm_rows<T, 8, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
    else if constexpr (W == 4) k_norm_rows<T, 16, MODE, W, 1, WL><<<grid1, NT, 0, s>>>(a);
}
// Launches of at least this many waves (rows x waves per row, at 4 waves per row) take
// k_norm_pipe (0: never) with pipe_wgs_per_cu<MODE>() workgroups per CU. Measured on MI355X
// at 8192 x 5376 bf16 (us; k_norm_rows with two rows per group and 4096 workgroups, then
// k_norm_pipe at 1 / 2 / 3 / 4 workgroups per CU and at its occupancy limit of 4-7, two
// runs each, within 0.3%):
//   input norm         31.6 -> 37.3 / 30.5 / 29.7 / 30.8 / 31.7
//   add + norm         60.9 -> 58.4 / 60.3 / 63.5 / 64.0 / 63.3
//   norm + add         44.9 -> 45.1 / 42.9 / 45.4 / 45.8 / 45.8
//   norm + add + norm  61.3 -> 65.0 / 61.9 / 65.7 / 65.5 / 65.1 (two barriers per row; with
//                      two rows per step reduced stage by stage, 61.9 / 64.5 at 1 / 2);
//                      k_norm_pipe_nan (one barrier per row) 61.1-61.4 -> 59.9-60.2 / 63.1-63.7
//                      at 1 / 2, so one workgroup per CU
// Each mode has its own best count of rows in flight per CU; more or fewer are slower.
#ifndef ZL_NORM_PIPE_WAVES
#define ZL_NORM_PIPE_WAVES 16384
#endif
// Nonzero: workgroups per CU of every mode's k_norm_pipe launch (tuning builds).
#ifndef ZL_NORM_PIPE_WG
#define ZL_NORM_PIPE_WG 0
#endif
#ifndef ZL_NORM_PIPE_NAN_WG
#define ZL_NORM_PIPE_NAN_WG 1
#endif
template <int MODE>
constexpr int pipe_wgs_per_cu() {
    return ZL_NORM_PIPE_WG ? ZL_NORM_PIPE_WG
           : MODE == M_NORM ? 3
           : MODE == M_ADD_NORM ? 1
           : MODE == M_NORM_ADD ? 2
                                : ZL_NORM_PIPE_NAN_WG;
}
// false: this mode keeps k_norm_rows
template <typename T, int MODE>
static bool launch_pipe(const NormArgs& a, int per_lane, hipStream_t s) {
    constexpr int wg = pipe_wgs_per_cu<MODE>();
    if constexpr (wg == 0) {
        return false;
    } else {
        const unsigned grid = (unsigned)std::min<int64_t>(a.rows, (int64_t)device_cus() * wg);
        if constexpr (MODE == M_NORM_ADD_NORM) {
            if (per_lane <= 1) k_norm_pipe_nan<T, 1><<<grid, 256, 0, s>>>(a);
            else if (per_lane <= 2) k_norm_pipe_nan<T, 2><<<grid, 256, 0, s>>>(a);
            else if (per_lane <= 3) k_norm_pipe_nan<T, 3><<<grid, 256, 0, s>>>(a);
            else k_norm_pipe_nan<T, 4><<<grid, 256, 0, s>>>(a);
            return true;
        }
        if (per_lane <= 1) k_norm_pipe<T, 1, MODE><<<grid, 256, 0, s>>>(a);
        else if (per_lane <= 2) k_norm_pipe<T, 2, MODE><<<grid, 256, 0, s>>>(a);
        else if (per_lane <= 3) k_norm_pipe<T, 3, MODE><<<grid, 256, 0, s>>>(a);
        else k_norm_pipe<T, 4, MODE><<<grid, 256, 0, s>>>(a);
        return true;
    }
}

template <typename T, int MODE, int W>
static void launch_wl(const NormArgs& a, int per_lane, int R, bool late, hipStream_t s) {
    if (late) launch_w<T, MODE, W, true>(a, per_lane, R, s);
    else launch_w<T, MODE, W, false>(a, per_lane, R, s);
}

// Waves per row: the fewest (1, 2 or 4) that keep a row within 4 chunks (128-bit loads)
// per lane (3 for NORM_ADD_NORM, which also holds the second weight vector; for NORM_ADD one
// wave per row up to 6 chunks, which skips the cross-wave reduction: 2048 x 2560 bf16 6.57 ->
// 6.26 us, with exactly 5 chunks per lane there 6.49 -> 6.32 us against 6; past one wave it
// takes 4 chunks too, so 8192 x 5376 runs 4 waves of 3 chunks and two rows stage by stage
// instead of 2 waves of 6: 45.7 -> 44.8 us), so a row lives in registers with few
// cross-wave reductions and every row of a 2048-token prefill is resident at once; rows
// longer than that at 4 waves take up to 16 chunks per lane.
// ZL_NORM_WAVES_PER_ROW, ZL_NORM_ROWS_PER_GROUP and ZL_NORM_LATE (0 / 1) force values.
#ifndef ZL_NORM_WAVES_PER_ROW
#define ZL_NORM_WAVES_PER_ROW 0
#endif
#ifndef ZL_NORM_ROWS_PER_GROUP
#define ZL_NORM_ROWS_PER_GROUP 0
#endif
#ifndef ZL_NORM_FIT_ADD
#define ZL_NORM_FIT_ADD 6
#endif
#ifndef ZL_NORM_FIT_NAN
#define ZL_NORM_FIT_NAN 3
#endif
#ifndef ZL_NORM_LATE
#define ZL_NORM_LATE -1
#endif
template <typename T, int MODE>
static void launch_t(const NormArgs& a, hipStream_t s) {
    constexpr int E = Chunk<T>::E;
    const int nch = a.n / E;
    int W = ZL_NORM_WAVES_PER_ROW;
    if (W == 0) {
        const int fit = MODE == M_NORM_ADD_NORM ? ZL_NORM_FIT_NAN : 4;
        const int fit1 = MODE == M_NORM_ADD ? ZL_NORM_FIT_ADD : fit;  // one wave per row
        W = nch <= fit1 * kWave ? 1 : nch <= 2 * fit * kWave ? 2 : 4;
    }
    const int per_lane = (int)cdiv(nch, kWave * W);
    // Two rows per lane group (the second row's loads in flight while the first is reduced
    // and stored) once the launch has several rounds of waves (8192 x 5376 bf16, 4 waves per
    // row: 5-8% faster for every mode), and from 2048 waves for the modes with two input
    // streams (2048 x 2560 bf16, 2 waves per row: residual add + norm 7.9 -> 7.2 us); the
    // plain norm keeps one row each there (4.6 against 5.0 us).
    const int64_t waves = a.rows * W;
    const int R = ZL_NORM_ROWS_PER_GROUP ? ZL_NORM_ROWS_PER_GROUP
                  : waves >= 8192 || (MODE != M_NORM && waves >= 2048) ? 2 : 1;
    // weights after the first row's activations (k_norm_rows; NORM_ADD at 2048 x 2560 bf16,
    // interleaved in-process rounds: 6.68 against 6.77 us with the activations)
    const bool late = ZL_NORM_LATE >= 0 ? ZL_NORM_LATE != 0 : waves >= 1024;
    const bool vec = a.n % E == 0 && aligned16(a.x) && (MODE == M_NORM || aligned16(a.r)) &&
                     (MODE == M_NORM_ADD || aligned16(a.out)) && aligned16(a.w1) &&
                     (MODE != M_NORM_ADD_NORM || aligned16(a.w2)) && per_lane <= (W == 4 ? 16 : 8);
    const bool pipe = vec && W == 4 && per_lane <= 4 && ZL_NORM_PIPE_WAVES > 0 && waves >= ZL_NORM_PIPE_WAVES;
    if (pipe && launch_pipe<T, MODE>(a, per_lane, s)) {
        // launched: persistent, pipelined rows
    } else if (vec) {
        if (W == 4) launch_wl<T, MODE, 4>(a, per_lane, R, late, s);
        else if (W == 2) launch_wl<T, MODE, 2>(a, per_lane, R, late, s);
        else launch_wl<T, MODE, 1>(a, per_lane, R, late, s);
    } else {
        k_norm_rows_generic<T, MODE><<<(unsigned)a.rows, 256, 0, s>>>(a);
    }
    check_launch();
}

template <int MODE>
static void launch_norm(int dtype, const NormArgs& a, hipStream_t s) {
    if (a.rows <= 0 || a.n <= 0) return;
    if (!a.x || (MODE != M_NORM && !a.r) || (MODE != M_NORM_ADD && !a.out)) {
        set_error(HIP_BRIDGE_EINVAL);
        return;
    }
    if (a.rows > 0x7fffffffLL) {
        set_error(HIP_BRIDGE_EUNSUPPORTED);
        return;
    }
    if (dtype == HIP_BRIDGE_F32) launch_t<float, MODE>(a, s);
    else if (dtype == HIP_BRIDGE_BF16) launch_t<uint16_t, MODE>(a, s);
    else set_error(HIP_BRIDGE_EUNSUPPORTED);
}

}  // namespace zl

using namespace zl;

extern "C" {

void hip_rmsnorm_rows(int dtype, const void* x, const float* weight, void* out, int64_t rows,
                      int n, float eps, int use_unit_offset, HipStream_t stream) {
    NormArgs a{const_cast<void*>(x), nullptr, weight, nullptr, out, rows, n, eps, use_unit_offset};
    launch_norm<M_NORM>(dtype, a, stream_of(stream));
}

void hip_add_rmsnorm_rows(int dtype, void* x, const void* residual, const float* weight,
                          void* out, int64_t rows, int n, float eps, int use_unit_offset,
                          HipStream_t stream) {
    NormArgs a{x, residual, weight, nullptr, out, rows, n, eps, use_unit_offset};
    launch_norm<M_ADD_NORM>(dtype, a, stream_of(stream));
}

void hip_rmsnorm_add_rows(int dtype, void* x, const void* in, const float* weight, int64_t rows,
                          int n, float eps, int use_unit_offset, HipStream_t stream) {
    NormArgs a{x, in, weight, nullptr, nullptr, rows, n, eps, use_unit_offset};
    launch_norm<M_NORM_ADD>(dtype, a, stream_of(stream));
}

void hip_rmsnorm_add_rmsnorm(int dtype, void* x, const void* xb, const float* w1,
                             const float* w2, void* out, int64_t rows, int n, float eps,
                             int use_unit_offset, HipStream_t stream) {
    NormArgs a{x, xb, w1, w2, out, rows, n, eps, use_unit_offset};
    launch_norm<M_NORM_ADD_NORM>(dtype, a, stream_of(stream));
}

// ---- reference-ABI f32 entry points -------------------------------------------------------

void hip_rmsnorm(const float* x, const float* weight, float* out, int n, float eps,
                 int use_unit_offset, HipStream_t stream) {
    hip_rmsnorm_rows(HIP_BRIDGE_F32, x, weight, out, 1, n, eps, use_unit_offset, stream);
}

void hip_rmsnorm_batched(float* x, const float* weight, float* out, int head_dim, int count,
                         float eps, int use_unit_offset, HipStream_t stream) {
    hip_rmsnorm_rows(HIP_BRIDGE_F32, x, weight, out, count, head_dim, eps, use_unit_offset, stream);
}

void hip_add_rmsnorm(float* x, const float* residual, const float* weight, float* out, int n,
                     float eps, int use_unit_offset, HipStream_t stream) {
    hip_add_rmsnorm_rows(HIP_BRIDGE_F32, x, residual, weight, out, 1, n, eps, use_unit_offset, stream);
}

void hip_add_rmsnorm_batched(float* x, const float* residual, const float* weight, float* out,
                             int n, int batch_size, float eps, int use_unit_offset,
                             HipStream_t stream) {
    hip_add_rmsnorm_rows(HIP_BRIDGE_F32, x, residual, weight, out, batch_size, n, eps,
                         use_unit_offset, stream);
}

void hip_rmsnorm_add(float* x, const float* in, const float* weight, int n, float eps,
                     int use_unit_offset, HipStream_t stream) {
    hip_rmsnorm_add_rows(HIP_BRIDGE_F32, x, in, weight, 1, n, eps, use_unit_offset, stream);
}

}  // extern "C"
