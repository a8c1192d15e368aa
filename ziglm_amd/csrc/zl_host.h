// Host-side helpers shared by the hip_bridge translation units: error recording, launch
// checks, grid sizing. Not part of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/hip_bridge.h"

namespace zl {

// Record an op error for hip_bridge_last_error() (thread-local, first error wins until read).
void set_error(int code);

// After a launch: record hipGetLastError() if the launch failed.
inline void check_launch() {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) set_error((int)e);
}

inline hipStream_t stream_of(HipStream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device, looked up once (the persistent kernels size their
// grids by it); 256 if the query fails.
inline int device_cus() {
    static std::atomic<int> cus{0};
    int c = cus.load(std::memory_order_relaxed);
    if (c == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) {
            (void)hipGetLastError();  // the failed query's error is not an op's
            c = 256;
        }
        cus.store(c, std::memory_order_relaxed);
    }
    return c;
}

// Matrix-core GEMM (gemm.hip) for batches of at least gemm_mfma_min_batch(qtype, rows, cols) tokens:
// launches and returns true when the type, shape (cols % 32 == 0, K-quants % 256) and
// alignment suit it, else launches nothing and returns false (the caller takes the vector
// path).
// Split K in the matrix-core kernel (gemm.hip launch_qt): products at least this deep with
// f32 output run each tile as two K halves when their tiles number fewer than two rounds.
#ifndef ZL_GEMM_SPLITK
#define ZL_GEMM_SPLITK 1
#endif
#ifndef ZL_GEMM_SPLITK_MIN_COLS
#define ZL_GEMM_SPLITK_MIN_COLS 4096
#endif
// The matrix-core kernel's smallest workgroup tile is 64 tokens x 64 rows, so below a few
// hundred tiles it leaves most of the chip idle (2560 x 10240 at up to 128 tokens: 40-80
// workgroups; split in two K halves ~130 us for Q4_0 whatever the batch), while the vector
// kernels' time grows with the batch. The batch from which it wins, measured per type on
// 10240 x 2560 (160 row tiles: "wide") and 2560 x 10240 (40, deep enough to split) products:
// Q4_0 / Q8_0 96 / 64, Q4_K 128 / 96 (against the small-batch kernel: 44 / 86 us at 64 tokens,
// the matrix cores 73 / 136), Q6_K 64 / 96 (small-batch kernel at 48 tokens 73 / 80 us, matrix
// cores 86 / 173); narrow products too shallow to split keep the unsplit crossovers (128, 96,
// 96).
// y[0, n) = 0 (a kernel, not hipMemsetAsync, so that graph captures of the products that
// add into y replay correctly)
void launch_zero_f32(float* y, int64_t n, hipStream_t s);
#ifndef ZL_GEMM_MIN_BATCH
#define ZL_GEMM_MIN_BATCH 0
#endif
inline int gemm_mfma_min_batch(int qtype, int rows, int cols) {
    if (ZL_GEMM_MIN_BATCH) return ZL_GEMM_MIN_BATCH;
    const bool wide = rows >= 128 * 64;  // enough row tiles to fill half the chip's workgroup slots
    const bool deep = ZL_GEMM_SPLITK && cols >= ZL_GEMM_SPLITK_MIN_COLS;
    if (qtype == HIP_BRIDGE_Q4_K) return wide ? 128 : 96;
    if (qtype == HIP_BRIDGE_Q6_K) return wide ? 64 : 96;
    return wide ? 96 : deep ? 64 : 128;
}
bool launch_gemm_mfma(int qtype, const void* w, int64_t row_bytes, const float* x, float* y, int rows, int cols,
                      int batch, hipStream_t s);
// The same for any batch with f32 or bf16 activations and output and an optional up matrix
// (y = gelu(W x) * (U x)); returns 0 when launched, else a HIP_BRIDGE_* code (nothing launched).
int launch_gemm_mfma_ex(int qtype, const void* w, const void* wu, int64_t row_bytes, int x_dtype, const void* x,
                        int y_dtype, void* y, int rows, int cols, int batch, hipStream_t s);

}  // namespace zl
