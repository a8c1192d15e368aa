// Host-side helpers shared by the hip_bridge translation units: error recording, launch
// checks, grid sizing. Not part of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Matrix-core GEMM (gemm.hip) for batches of at least kGemmMfmaMinBatch tokens: launches and
// returns true when the type, shape (cols % 32 == 0) and alignment suit it, else launches
// nothing and returns false (the caller takes the vector path).
constexpr int kGemmMfmaMinBatch = 32;
bool launch_gemm_mfma(int qtype, const void* w, int64_t row_bytes, const float* x, float* y, int rows, int cols,
                      int batch, hipStream_t s);
// The same for any batch with f32 or bf16 activations and output and an optional up matrix
// (y = gelu(W x) * (U x)); returns 0 when launched, else a HIP_BRIDGE_* code (nothing launched).
int launch_gemm_mfma_ex(int qtype, const void* w, const void* wu, int64_t row_bytes, int x_dtype, const void* x,
                        int y_dtype, void* y, int rows, int cols, int batch, hipStream_t s);

}  // namespace zl
