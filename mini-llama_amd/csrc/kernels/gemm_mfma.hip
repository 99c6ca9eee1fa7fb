// Prefill / batched GEMM on gfx950 MFMA: y[m, n] = sum_k W[n, k] x[m, k].
//
// The reference never issues m > 1 on the GPU (src/batch.cc:32-55 loops
// tokens); its kernels (src/cuda_quant.cu:78-182) re-stream W once per row
// of x (grid.y = rows). This kernel is a dense contraction instead:
//  - Workgroup tile 128 (m) x 128 (n), four waves in a 2x2 grid, each wave
//    64 x 64 = 4 x 4 tiles of v_mfma_f32_16x16x32_f16 (fp32 accumulate).
//  - K advances one 128-k block group per step; MFMA step j covers block
//    4g+j. Activations are converted fp32 -> fp16 into LDS; weights are read
//    as contiguous 1 KiB (q4) / 2 KiB (q8) lines per 16-row tile (the tiled
//    layout puts each MFMA B fragment in one lane's 16 B) and dequantized
//    once per workgroup to fp16 d*(q-8) / d*q+m / d*q (exact code decode,
//    one fp16 rounding) into LDS. Both LDS slabs are stored in MFMA operand
//    order (16 B per lane per operand): fragment reads are ds_read_b128.
//  - Per k step: 16 fragment reads and 64 MFMAs per wave.
// The scale is applied before the MFMA (per weight), so no per-block fixup
// of the accumulators is needed; that is what keeps VALU work independent of
// m (an int8 MFMA variant would need a per-(m, n, block) fp32 fixup).
#include <hip/hip_runtime.h>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kBM = 128;  // x rows per workgroup
constexpr int kBN = 128;  // W rows per workgroup
constexpr int kATiles = kBM / 16;
constexpr int kBTiles = kBN / 16;
constexpr int kThreads = 256;

struct GemmArgs {
  const uint8_t* qs;
  const uint16_t* d;
  const uint16_t* mn;
  const float* x;
  float* y;
  int m, n, k, g, nt;
};

// Dequantize one 32-bit word of codes into 8 (q4) or 4 (q8) pre-scaled fp16
// values.
__device__ __forceinline__ uint4 deq_q4_0(uint32_t v, h2_t d2) {
  const Q4Pairs p = q4_pairs(v);
  const h2_t b1024 = {(_Float16)1032.0f, (_Float16)1032.0f};
  const h2_t b64 = {(_Float16)72.0f, (_Float16)72.0f};
  uint4 o;
  o.x = as_u32((as_h2(p.p0) - b1024) * d2);
  o.y = as_u32((as_h2(p.p1) - b64) * d2);
  o.z = as_u32((as_h2(p.p2) - b1024) * d2);
  o.w = as_u32((as_h2(p.p3) - b64) * d2);
  return o;
}

__device__ __forceinline__ uint4 deq_q4_1(uint32_t v, h2_t d2, h2_t m2) {
  const Q4Pairs p = q4_pairs(v);
  const h2_t b1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const h2_t b64 = {(_Float16)64.0f, (_Float16)64.0f};
  uint4 o;
  o.x = as_u32(__builtin_elementwise_fma(as_h2(p.p0) - b1024, d2, m2));
  o.y = as_u32(__builtin_elementwise_fma(as_h2(p.p1) - b64, d2, m2));
  o.z = as_u32(__builtin_elementwise_fma(as_h2(p.p2) - b1024, d2, m2));
  o.w = as_u32(__builtin_elementwise_fma(as_h2(p.p3) - b64, d2, m2));
  return o;
}

__device__ __forceinline__ uint2 deq_q8_0(uint32_t v, h2_t d2) {
  uint32_t p0, p1;
  q8_pairs(v, p0, p1);
  const h2_t b = {(_Float16)1152.0f, (_Float16)1152.0f};
  uint2 o;
  o.x = as_u32((as_h2(p0) - b) * d2);
  o.y = as_u32((as_h2(p1) - b) * d2);
  return o;
}

template <int QT>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmArgs a) {
  // LDS slabs in MFMA operand order: [tile][t][lane] x 16 B.
  __shared__ __align__(16) uint4 as[kATiles * 4 * 64];
  __shared__ __align__(16) uint4 bs[kBTiles * 4 * 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * kBM;
  const int tile0 = blockIdx.x * kBTiles;  // first W row tile
  const bool vec_ok = (a.k & 3) == 0;

  f4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) acc[i][jj] = (f4_t){0.f, 0.f, 0.f, 0.f};

  for (int g = 0; g < a.g; ++g) {
    // ---- activations: 128 rows x 128 k, 8 floats per item ---------------
#pragma unroll
    for (int it = 0; it < (kBM * 16) / kThreads; ++it) {
      const int id = tid + it * kThreads;
      const int ml = id >> 4, sg = id & 15;
      const int mrow = m0 + ml;
      const int k0 = g * kGroupK + sg * 8;
      float v[8];
      const float* xr = a.x + (size_t)mrow * a.k;
      if (mrow < a.m && vec_ok && k0 + 8 <= a.k) {
        const float4 lo = *(const float4*)(xr + k0);
        const float4 hi = *(const float4*)(xr + k0 + 4);
        v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
        v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[e] = (mrow < a.m && k0 + e < a.k) ? xr[k0 + e] : 0.0f;
      }
      uint4 h;
      h.x = pack_h2(v[0], v[1]);
      h.y = pack_h2(v[2], v[3]);
      h.z = pack_h2(v[4], v[5]);
      h.w = pack_h2(v[6], v[7]);
      // k-in-group = 32*j + 8*kq: MFMA step j (block), lane = i + 16*kq
      const int j = sg >> 2, kq = sg & 3;
      as[((ml >> 4) * 4 + j) * 64 + (ml & 15) + 16 * kq] = h;
    }

    // ---- weights: dequantize the group's lines of 8 row tiles ------------
    // chunk lane L = n + 16*kq holds quarter kq of blocks 4g..4g+3 of row n;
    // word j (block 4g+j) becomes the B fragment of MFMA step j.
    if (QT == MLQ_Q8_0) {
#pragma unroll
      for (int it = 0; it < (kBTiles * 128) / kThreads; ++it) {
        const int id = tid + it * kThreads;
        const int wt = id >> 7, hh = (id >> 6) & 1, ln = id & 63;
        const int tile = tile0 + wt;
        uint4 o0 = {0, 0, 0, 0}, o1 = {0, 0, 0, 0};
        if (tile < a.nt) {
          const size_t unit = (size_t)tile * a.g + g;
          const uint4 q = *(const uint4*)(a.qs + ((unit * 2 + hh) * 64 + ln) * 16);
          const uint2 ds = *(const uint2*)(a.d + (unit * 16 + (ln & 15)) * 4);
          const uint32_t dw = hh ? ds.y : ds.x;  // scales of blocks 2hh, 2hh+1
          const _Float16 d0 = __builtin_bit_cast(_Float16, (uint16_t)(dw & 0xffffu));
          const _Float16 d1 = __builtin_bit_cast(_Float16, (uint16_t)(dw >> 16));
          const uint2 w0 = deq_q8_0(q.x, (h2_t){d0, d0});
          const uint2 w1 = deq_q8_0(q.y, (h2_t){d0, d0});
          const uint2 w2 = deq_q8_0(q.z, (h2_t){d1, d1});
          const uint2 w3 = deq_q8_0(q.w, (h2_t){d1, d1});
          o0 = (uint4){w0.x, w0.y, w1.x, w1.y};
          o1 = (uint4){w2.x, w2.y, w3.x, w3.y};
        }
        bs[(wt * 4 + 2 * hh) * 64 + ln] = o0;
        bs[(wt * 4 + 2 * hh + 1) * 64 + ln] = o1;
      }
    } else {
#pragma unroll
      for (int it = 0; it < (kBTiles * 64) / kThreads; ++it) {
        const int id = tid + it * kThreads;
        const int wt = id >> 6, ln = id & 63;
        const int tile = tile0 + wt;
        uint4 o[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
        if (tile < a.nt) {
          const size_t unit = (size_t)tile * a.g + g;
          const uint4 q = *(const uint4*)(a.qs + (unit * 64 + ln) * 16);
          const size_t si = (unit * 16 + (ln & 15)) * 4;
          const uint2 ds = *(const uint2*)(a.d + si);
          const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
          const uint16_t dbits[4] = {(uint16_t)(ds.x & 0xffffu), (uint16_t)(ds.x >> 16),
                                     (uint16_t)(ds.y & 0xffffu), (uint16_t)(ds.y >> 16)};
          if (QT == MLQ_Q4_0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const _Float16 dh = __builtin_bit_cast(_Float16, dbits[j]);
              o[j] = deq_q4_0(qw[j], (h2_t){dh, dh});
            }
          } else {
            const uint2 ms = *(const uint2*)(a.mn + si);
            const uint16_t mbits[4] = {(uint16_t)(ms.x & 0xffffu), (uint16_t)(ms.x >> 16),
                                       (uint16_t)(ms.y & 0xffffu), (uint16_t)(ms.y >> 16)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const _Float16 dh = __builtin_bit_cast(_Float16, dbits[j]);
              const _Float16 mh = __builtin_bit_cast(_Float16, mbits[j]);
              o[j] = deq_q4_1(qw[j], (h2_t){dh, dh}, (h2_t){mh, mh});
            }
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) bs[(wt * 4 + j) * 64 + ln] = o[j];
      }
    }
    __syncthreads();

    // ---- MFMA: wave (wm, wn) -> A tiles 4wm..4wm+3, B tiles 4wn..4wn+3 ----
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      h8_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = __builtin_bit_cast(h8_t, as[((4 * wm + i) * 4 + t) * 64 + lane]);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        bf[jj] = __builtin_bit_cast(h8_t, bs[((4 * wn + jj) * 4 + t) * 64 + lane]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[jj],
                                                             acc[i][jj], 0, 0, 0);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds D[4*(lane/16) + r][lane%16] of each tile -------
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int ncol = (tile0 + 4 * wn + jj) * 16 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int mrow = m0 + (4 * wm + i) * 16 + 4 * (lane >> 4) + r;
        if (mrow < a.m && ncol < a.n) a.y[(size_t)mrow * a.n + ncol] = acc[i][jj][r];
      }
    }
  }
}

}  // namespace

hipError_t launch_gemm(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream) {
  const Geometry geo = geometry(w.n, w.k);
  GemmArgs a;
  a.qs = (const uint8_t*)w.base + w.qs_off;
  a.d = (const uint16_t*)((const uint8_t*)w.base + w.d_off);
  a.mn = w.type == MLQ_Q4_1
             ? (const uint16_t*)((const uint8_t*)w.base + w.m_off)
             : nullptr;
  a.x = x;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.k = w.k;
  a.g = geo.g;
  a.nt = geo.nt;
  const dim3 grid((unsigned)((geo.nt + kBTiles - 1) / kBTiles),
                  (unsigned)((m + kBM - 1) / kBM));
  switch (w.type) {
    case MLQ_Q8_0: gemm_kernel<MLQ_Q8_0><<<grid, kThreads, 0, stream>>>(a); break;
    case MLQ_Q4_0: gemm_kernel<MLQ_Q4_0><<<grid, kThreads, 0, stream>>>(a); break;
    default: gemm_kernel<MLQ_Q4_1><<<grid, kThreads, 0, stream>>>(a); break;
  }
  return hipGetLastError();
}

}  // namespace mlq
