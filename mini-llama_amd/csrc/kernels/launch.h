// Internal launchers (C++ linkage, library-private). The C ABI in capi.cpp
// validates arguments and then calls these; they only configure and launch.
#pragma once

#include <hip/hip_runtime.h>

#include "../mlq_layout.h"

namespace mlq {

// repack.hip
hipError_t launch_repack(int type, const void* aos, int n, int k,
                         const mlq_weight& w, hipStream_t stream);
hipError_t launch_dequant(const mlq_weight& w, int row0, int rows, float* out,
                          hipStream_t stream);
hipError_t launch_bias(float* y, const float* bias, int m, int n,
                       hipStream_t stream);

// gemv.hip: m in 1..8 rows of x.
constexpr int kGemvMaxRows = 8;
// Returns hipErrorInvalidValue when the activation staging does not fit LDS.
hipError_t launch_gemv(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream);
// Largest k the GEMV accepts for m rows (LDS-bound).
int gemv_max_k(int type, int m);
// Split override (0 = automatic); validated by the caller.
void set_gemv_split(int split);

// gemm_mfma.hip: any m >= 1. The _ws form converts x to fp16 into `ws`
// first when ws_bytes >= gemm_workspace_bytes(m, k) (else reads fp32 x).
hipError_t launch_gemm(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream);
hipError_t launch_gemm_ws(const mlq_weight& w, const float* x, float* y, int m,
                          void* ws, size_t ws_bytes, hipStream_t stream);
size_t gemm_workspace_bytes(int m, int k);

}  // namespace mlq
