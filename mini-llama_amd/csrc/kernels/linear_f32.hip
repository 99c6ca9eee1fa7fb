// F32 Linear: y[r][row] = sum_k x[r][k] * W[row][k] + epilogue, W fp32
// [n][k] row-major (cudaLinearDeviceInput, src/cuda_matmul.cc:205-241, which
// calls cuBLAS Sgemm; also the F32 arm of forwardLinearDevice,
// src/forward.cc:206-209). The reference's F32 weights are the unquantized
// model's projections and the tied lm_head.
//
// HBM-streaming GEMV: one workgroup (4 waves) per 16-row tile, 4 rows per
// wave; lanes stride K with float4 loads, so every W element is read once per
// launch (non-temporal: W is streamed, x stays cached). Up to 8 activation
// rows share each W pass; more rows run as further passes. Under the SwiGLU
// epilogue a wave takes two gate rows and their two up rows (rows 16t+j and
// 16t+8+j of the interleaved tile), so both operands of an output meet in one
// wave.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"

namespace mlq {
namespace {

constexpr int kF32MaxRows = 8;

struct F32Args {
  const float* w;
  const float* x;
  float* y;
  int n, k, ny;
  Epilogue epi;
};

template <int MR, bool VEC>
__global__ __launch_bounds__(256) void linear_f32_kernel(F32Args a) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const bool glu = a.epi.act == kEpiSwiGLU;
  int rows[4];
  const float* wr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int off = glu ? (i < 2 ? 2 * wave + i : 8 + 2 * wave + (i - 2)) : 4 * wave + i;
    rows[i] = 16 * (int)blockIdx.x + off;
    wr[i] = a.w + (size_t)min(rows[i], a.n - 1) * a.k;
  }
  float acc[4][MR];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[i][r] = 0.0f;

  if constexpr (VEC) {
#pragma unroll 2
    for (int kk = lane * 4; kk < a.k; kk += 256) {
      f4_t wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[i] = __builtin_nontemporal_load((const f4_t*)(wr[i] + kk));
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        const f4_t xv = *(const f4_t*)(a.x + (size_t)r * a.k + kk);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[i][r] += wv[i].x * xv.x;
          acc[i][r] += wv[i].y * xv.y;
          acc[i][r] += wv[i].z * xv.z;
          acc[i][r] += wv[i].w * xv.w;
        }
      }
    }
  } else {
    for (int kk = lane; kk < a.k; kk += 64) {
      float wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) wv[i] = wr[i][kk];
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        const float xv = a.x[(size_t)r * a.k + kk];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][r] += wv[i] * xv;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[i][r] = wave_sum(acc[i][r]);
  if (lane != 0) return;
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    float* yr = a.y + (size_t)r * a.ny;
    if (glu) {
      // n % 16 == 0 under SwiGLU, so every row of the tile exists
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float g = add_bias(a.epi, acc[i][r], rows[i]);
        const float u = add_bias(a.epi, acc[i + 2][r], rows[i + 2]);
        yr[glu_col(rows[i])] = silu_f(g) * u;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (rows[i] < a.n) yr[rows[i]] = add_bias(a.epi, acc[i][r], rows[i]);
    }
  }
}

template <bool VEC>
void launch_rows(const F32Args& a, int mr, hipStream_t s) {
  const dim3 grid((a.n + 15) / 16), block(256);
  switch (mr) {
    case 1: hipLaunchKernelGGL((linear_f32_kernel<1, VEC>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((linear_f32_kernel<2, VEC>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((linear_f32_kernel<3, VEC>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((linear_f32_kernel<4, VEC>), grid, block, 0, s, a); break;
    case 5: hipLaunchKernelGGL((linear_f32_kernel<5, VEC>), grid, block, 0, s, a); break;
    case 6: hipLaunchKernelGGL((linear_f32_kernel<6, VEC>), grid, block, 0, s, a); break;
    case 7: hipLaunchKernelGGL((linear_f32_kernel<7, VEC>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((linear_f32_kernel<8, VEC>), grid, block, 0, s, a); break;
  }
}

}  // namespace

hipError_t launch_linear_f32(const float* w, int n, int k, const float* x, float* y, int m,
                             hipStream_t stream, const Epilogue& epi) {
  F32Args a;
  a.w = w;
  a.n = n;
  a.k = k;
  a.ny = epi.act == kEpiSwiGLU ? n / 2 : n;
  a.epi = epi;
  const bool vec = k % 4 == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0;
  for (int r0 = 0; r0 < m; r0 += kF32MaxRows) {
    const int mr = m - r0 < kF32MaxRows ? m - r0 : kF32MaxRows;
    a.x = x + (size_t)r0 * k;
    a.y = y + (size_t)r0 * a.ny;
    if (vec) launch_rows<true>(a, mr, stream);
    else launch_rows<false>(a, mr, stream);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mlq
