// The fp16 copy of an activation matrix that the skinny and prefill GEMMs
// read (library-private, included by skinny.hip and gemm_mfma.hip).
//
// Row r of x fp32 [m][k] is stored as fp16 of x[r] * 2^e_r, with e_r =
// pow2_scale_exp(max_c |x[r][c]|) written to rexp[r]: any finite fp32 row
// fits fp16 without overflow, and its subnormal floor sits 2^-39 below the
// row's largest element; the GEMMs scale row r's fp32 results by 2^-e_r.
// Columns k <= c < kp are zero; with the fragment layout, rows m <= r <
// 16 * mbt are zero too (exponent 0).
//
// One workgroup per row: every thread loads its chunks of 8 elements into
// registers, the row maximum is reduced (DPP and scalar within a wave, LDS
// across waves), then the scaled chunks are stored: one memory round trip.
// Rows longer than the register budget take two passes (the second read
// hits the caches).
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"

namespace mlq {

constexpr int kCopyThreads = 512;
constexpr int kCopyMaxChunks = 8;  // 8 * 8 * 512 = 32768 elements in registers
enum { kCopyRowMajor = 0, kCopyFragments = 1 };

struct RowCopyArgs {
  const float* x;
  _Float16* dst;
  int* rexp;
  int m, k, kp;
  int mbt;  // fragment layout: 16-row blocks
};

// Destination of the 8 halves starting at column c0 of row r. Fragment
// layout (skinny GEMM): element (r, c) of row block mb = r/16, 128-k group
// j = c/128, 32-k block b = c%128/32 sits at lane r%16 + 16*(c%32/8),
// position c%8 of run ((j*mbt + mb)*4 + b).
template <int LAYOUT>
__device__ __forceinline__ _Float16* copy_dst(const RowCopyArgs& a, int r, int c0) {
  if constexpr (LAYOUT == kCopyRowMajor) {
    return a.dst + (size_t)r * a.kp + c0;
  } else {
    const int j = c0 / 128, b = (c0 % 128) / 32, kq = (c0 % 32) / 8;
    const int mb = r / 16, lane = r % 16 + 16 * kq;
    return a.dst + ((((size_t)j * a.mbt + mb) * 4 + b) * 64 + lane) * 8;
  }
}

__device__ __forceinline__ void load8(const float* xr, int k, int c0, bool live, float (&v)[8]) {
  if (live && (k & 3) == 0 && c0 + 8 <= k) {
    const float4 lo = *(const float4*)(xr + c0);
    const float4 hi = *(const float4*)(xr + c0 + 4);
    v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
    v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = (live && c0 + t < k) ? xr[c0 + t] : 0.0f;
  }
}

__device__ __forceinline__ uint4 pack8(const float (&v)[8], int e) {
  uint4 o;
  o.x = pack_h2(ldexp_f(v[0], e), ldexp_f(v[1], e));
  o.y = pack_h2(ldexp_f(v[2], e), ldexp_f(v[3], e));
  o.z = pack_h2(ldexp_f(v[4], e), ldexp_f(v[5], e));
  o.w = pack_h2(ldexp_f(v[6], e), ldexp_f(v[7], e));
  return o;
}

// CH > 0: each thread holds CH chunks (8 * kCopyThreads * CH >= kp);
// CH == 0: two passes over the row.
template <int LAYOUT, int CH>
__global__ __launch_bounds__(kCopyThreads) void row_copy_kernel(RowCopyArgs a) {
  __shared__ int pmax[kCopyThreads / 64];
  const int r = blockIdx.x, tid = threadIdx.x;
  const bool live = r < a.m;
  const float* xr = a.x + (size_t)(live ? r : 0) * a.k;
  constexpr int NV = CH > 0 ? CH : 1;
  float v[NV][8];
  float mx = 0.0f;
  if constexpr (CH > 0) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      load8(xr, a.k, 8 * (tid + kCopyThreads * j), live, v[j]);
#pragma unroll
      for (int t = 0; t < 8; ++t) mx = fmaxf(mx, fabsf(v[j][t]));
    }
  } else {
    for (int c0 = 8 * tid; c0 < a.k; c0 += 8 * kCopyThreads) {
      load8(xr, a.k, c0, live, v[0]);
#pragma unroll
      for (int t = 0; t < 8; ++t) mx = fmaxf(mx, fabsf(v[0][t]));
    }
  }
  const float wm = wave_max_nonneg(mx);
  if ((tid & 63) == 0) pmax[tid >> 6] = __builtin_bit_cast(int, wm);
  __syncthreads();
  int best = pmax[0];
#pragma unroll
  for (int i = 1; i < kCopyThreads / 64; ++i) best = max(best, pmax[i]);
  const int e = pow2_scale_exp(__builtin_bit_cast(float, best));
  if (tid == 0) a.rexp[r] = e;
  if constexpr (CH > 0) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c0 = 8 * (tid + kCopyThreads * j);
      if (c0 < a.kp) *(uint4*)copy_dst<LAYOUT>(a, r, c0) = pack8(v[j], e);
    }
  } else {
    for (int c0 = 8 * tid; c0 < a.kp; c0 += 8 * kCopyThreads) {
      load8(xr, a.k, c0, live, v[0]);
      *(uint4*)copy_dst<LAYOUT>(a, r, c0) = pack8(v[0], e);
    }
  }
}

// Launches one workgroup per destination row (rows: m, or 16 * mbt for the
// fragment layout).
template <int LAYOUT>
inline hipError_t launch_row_copy(const RowCopyArgs& a, int rows, hipStream_t stream) {
  const int per = (a.kp / 8 + kCopyThreads - 1) / kCopyThreads;  // chunks per thread
  const dim3 grid(rows), block(kCopyThreads);
  if (per <= 1) row_copy_kernel<LAYOUT, 1><<<grid, block, 0, stream>>>(a);
  else if (per <= 2) row_copy_kernel<LAYOUT, 2><<<grid, block, 0, stream>>>(a);
  else if (per <= 4) row_copy_kernel<LAYOUT, 4><<<grid, block, 0, stream>>>(a);
  else if (per <= kCopyMaxChunks) row_copy_kernel<LAYOUT, kCopyMaxChunks><<<grid, block, 0, stream>>>(a);
  else row_copy_kernel<LAYOUT, 0><<<grid, block, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace mlq
