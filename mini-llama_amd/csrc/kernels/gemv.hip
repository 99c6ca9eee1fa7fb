// Decode GEMV / skinny GEMM for gfx950: y[m, n] = sum_k W[n, k] x[m, k] for
// m = 1..8 activation rows.
//
// Replaces q80LinearKernel / q40LinearKernel / q41LinearKernel
// (src/cuda_quant.cu:78-182) for decode-sized m. Design (HBM-bound):
//  - A workgroup owns one 16-row tile at a time; its waves split K into
//    contiguous ranges of 128-k groups. Per group a wave reads one contiguous
//    1 KiB (q4) / 2 KiB (q8) line with one dwordx4 per lane plus an 8-byte
//    scale load; every weight byte is read from HBM exactly once.
//  - Lane L = n + 16*kq holds quarter kq of the group's 4 blocks of row n,
//    which is the B operand of v_mfma_f32_16x16x32_f16 for one block. Codes
//    are decoded EXACTLY to fp16 (q-8, q, or q): one AND-OR places a code in
//    the mantissa of 1024 (or 64), one packed fp16 subtract removes the bias.
//  - Activations are staged once per workgroup in LDS as an fp16 hi/lo pair
//    (x = hi + lo to ~2^-22); MFMA row 2r is hi, row 2r+1 is lo of activation
//    row r, so up to 8 activation rows ride in one MFMA at no extra cost.
//  - Per block: acc += d * (D[hi] + D[lo]) in fp32 (+ m * sum(x) for q4_1),
//    so the result is fp32-class accurate (products are exact in fp32).
//  - Waves combine their partial sums through LDS in a fixed order.
// Activations must be finite and |x| < 65504 (the fp16 range of the hi part).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kMaxWaves = 16;

// Largest dynamic LDS allocation a workgroup may use on the current device
// (160 KiB on gfx950), read once.
size_t lds_limit() {
  static const size_t limit = [] {
    int dev = 0, bytes = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock,
                              dev) != hipSuccess ||
        bytes <= 0)
      return (size_t)64 * 1024;
    return (size_t)bytes;
  }();
  return limit;
}
constexpr int kRowPadHalves = 32;  // 64 B: consecutive LDS rows hit other banks

// Groups per wave whose loads are issued together (8 KiB of quants in flight
// per wave for every type; q8_0 lines are twice as long).
template <int QT>
constexpr int unroll_for() {
  return QT == MLQ_Q8_0 ? 4 : 8;
}
constexpr int kMaxUnroll = 8;

struct GemvArgs {
  const uint8_t* qs;
  const uint16_t* d;
  const uint16_t* mn;
  const float* x;
  float* y;
  int m, n, k, g, nt;
  int gw;               // 128-k groups per wave
  int tiles_per_block;  // row tiles handled by one workgroup, in sequence
  int xstride;          // fp16 elements per staged activation row
};

template <int QT>
struct Chunk {
  uint4 q[kMaxUnroll];
  uint4 q2[kMaxUnroll];  // second 16-byte line (q8_0)
  uint2 d[kMaxUnroll];   // four fp16 scales of the group's blocks
  uint2 m[kMaxUnroll];   // four fp16 mins (q4_1)
};

template <int QT>
__device__ __forceinline__ void issue_loads(const GemvArgs& a, Chunk<QT>& c,
                                            int tile, int gc, int g1,
                                            int lane) {
  const int n = lane & 15;
#pragma unroll
  for (int u = 0; u < unroll_for<QT>(); ++u) {
    const int g = gc + u;
    if (g < g1) {
      const size_t unit = (size_t)tile * a.g + g;
      if (QT == MLQ_Q8_0) {
        c.q[u] = *(const uint4*)(a.qs + ((unit * 2) * kLanes + lane) * 16);
        c.q2[u] = *(const uint4*)(a.qs + ((unit * 2 + 1) * kLanes + lane) * 16);
      } else {
        c.q[u] = *(const uint4*)(a.qs + (unit * kLanes + lane) * 16);
      }
      c.d[u] = *(const uint2*)(a.d + (unit * kTileRows + n) * kGroupBlocks);
      if (QT == MLQ_Q4_1)
        c.m[u] = *(const uint2*)(a.mn + (unit * kTileRows + n) * kGroupBlocks);
    }
  }
}

// Exact fp16 decode of 8 codes of one quarter-block (MFMA B fragment).
template <int QT>
__device__ __forceinline__ h8_t decode8(uint32_t w0, uint32_t w1) {
  uint4 o;
  if (QT == MLQ_Q8_0) {
    const h2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    uint32_t p0, p1, p2, p3;
    q8_pairs(w0, p0, p1);
    q8_pairs(w1, p2, p3);
    o.x = as_u32(as_h2(p0) - bias);
    o.y = as_u32(as_h2(p1) - bias);
    o.z = as_u32(as_h2(p2) - bias);
    o.w = as_u32(as_h2(p3) - bias);
  } else {
    const float lo = QT == MLQ_Q4_0 ? 1032.0f : 1024.0f;
    const float hi = QT == MLQ_Q4_0 ? 72.0f : 64.0f;
    const h2_t blo = {(_Float16)lo, (_Float16)lo};
    const h2_t bhi = {(_Float16)hi, (_Float16)hi};
    const Q4Pairs p = q4_pairs(w0);
    o.x = as_u32(as_h2(p.p0) - blo);
    o.y = as_u32(as_h2(p.p1) - bhi);
    o.z = as_u32(as_h2(p.p2) - blo);
    o.w = as_u32(as_h2(p.p3) - bhi);
  }
  return __builtin_bit_cast(h8_t, o);
}

__device__ __forceinline__ float scale_at(uint2 s, int j) {
  const uint32_t w = (j & 2) ? s.y : s.x;
  return half_bits_to_float((uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu)));
}

// LDS layout (bytes):
//   xs:   2*m rows of xstride fp16 (row 2r = hi(x[r]), row 2r+1 = lo(x[r]))
//   xsum: m * blocks fp32 (q4_1: per-block sum of x, exact fp32 inputs)
//   part: waves * m * 16 fp32 (cross-wave partials)
template <int QT, int MR>
__global__ __launch_bounds__(1024) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int G = a.g;
  const int M = a.m;
  const int nblk = G * kGroupBlocks;
  _Float16* xs = (_Float16*)smem;
  float* xsum = (float*)(smem + (size_t)2 * M * a.xstride * 2);
  float* part = xsum + (QT == MLQ_Q4_1 ? M * nblk : 0);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int n = lane & 15;   // W row within the tile (and MFMA A row)
  const int kq = lane >> 4;  // quarter of each block (and D row group)
  const int g0 = wave * a.gw;
  const int g1 = min(G, g0 + a.gw);
  const int tile_begin = blockIdx.x * a.tiles_per_block;
  const int tile_end = min(a.nt, tile_begin + a.tiles_per_block);

  Chunk<QT> c;
  // Weight loads first: their HBM latency covers the activation staging.
  issue_loads<QT>(a, c, tile_begin, g0, g1, lane);

  // ---- stage activations: hi/lo fp16 rows (+ block sums for q4_1) --------
  {
    const int segs = G * (kGroupK / 8);  // 8-element segments per row
    const int items = M * segs;
    const bool vec_ok = (a.k & 3) == 0;
    for (int base = 0; base < items; base += blockDim.x) {
      const int i = base + tid;
      const bool act = i < items;
      const int r = act ? i / segs : 0;
      const int seg = act ? i % segs : 0;
      const int k0 = seg * 8;
      float v[8];
      const float* xr = a.x + (size_t)r * a.k;
      if (act && vec_ok && k0 + 8 <= a.k) {
        const float4 lo4 = *(const float4*)(xr + k0);
        const float4 hi4 = *(const float4*)(xr + k0 + 4);
        v[0] = lo4.x; v[1] = lo4.y; v[2] = lo4.z; v[3] = lo4.w;
        v[4] = hi4.x; v[5] = hi4.y; v[6] = hi4.z; v[7] = hi4.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (act && k0 + e < a.k) ? xr[k0 + e] : 0.0f;
      }
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const _Float16 h0 = (_Float16)v[2 * p], h1 = (_Float16)v[2 * p + 1];
        const _Float16 l0 = (_Float16)(v[2 * p] - (float)h0);
        const _Float16 l1 = (_Float16)(v[2 * p + 1] - (float)h1);
        hw[p] = as_u32((h2_t){h0, h1});
        lw[p] = as_u32((h2_t){l0, l1});
      }
      if (act) {
        *(uint4*)(xs + (size_t)(2 * r) * a.xstride + k0) =
            (uint4){hw[0], hw[1], hw[2], hw[3]};
        *(uint4*)(xs + (size_t)(2 * r + 1) * a.xstride + k0) =
            (uint4){lw[0], lw[1], lw[2], lw[3]};
      }
      if (QT == MLQ_Q4_1) {
        float sx = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sx += v[e];
        sx += __shfl_xor(sx, 1);
        sx += __shfl_xor(sx, 2);
        if (act && (seg & 3) == 0) xsum[r * nblk + (seg >> 2)] = sx;
      }
    }
  }
  __syncthreads();

  // MFMA A row `n` carries activation row n/2 (hi for even n, lo for odd n).
  const bool a_live = n < 2 * M;
  const _Float16* arow = xs + (size_t)(a_live ? n : 0) * a.xstride + 8 * kq;
  const int r0 = 2 * kq, r1 = 2 * kq + 1;  // activation rows of this lane's D

  bool first = true;
  for (int tile = tile_begin; tile < tile_end; ++tile) {
    float acc0 = 0.0f, acc1 = 0.0f;
    for (int gc = g0; gc < g1; gc += unroll_for<QT>()) {
      if (!first) issue_loads<QT>(a, c, tile, gc, g1, lane);
      first = false;
#pragma unroll
      for (int u = 0; u < unroll_for<QT>(); ++u) {
        const int g = gc + u;
        if (g < g1) {
#pragma unroll
          for (int j = 0; j < kGroupBlocks; ++j) {
            h8_t bfrag;
            if (QT == MLQ_Q8_0) {
              const uint4 q = (j < 2) ? c.q[u] : c.q2[u];
              const uint32_t w0 = (j & 1) ? q.z : q.x;
              const uint32_t w1 = (j & 1) ? q.w : q.y;
              bfrag = decode8<QT>(w0, w1);
            } else {
              const uint4 q = c.q[u];
              const uint32_t w0 = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
              bfrag = decode8<QT>(w0, 0);
            }
            uint4 av = {0, 0, 0, 0};
            if (a_live) av = *(const uint4*)(arow + g * kGroupK + j * kQK);
            const f4_t zero = {0.f, 0.f, 0.f, 0.f};
            const f4_t dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(h8_t, av), bfrag, zero, 0, 0, 0);
            const float df = scale_at(c.d[u], j);
            acc0 = fmaf(df, dd[0] + dd[1], acc0);
            if (MR > 1) acc1 = fmaf(df, dd[2] + dd[3], acc1);
            if (QT == MLQ_Q4_1) {
              const float mf = scale_at(c.m[u], j);
              const int b = g * kGroupBlocks + j;
              if (r0 < M) acc0 = fmaf(mf, xsum[r0 * nblk + b], acc0);
              if (MR > 1 && r1 < M) acc1 = fmaf(mf, xsum[r1 * nblk + b], acc1);
            }
          }
        }
      }
    }

    // ---- combine waves in a fixed order -----------------------------------
    if (r0 < M) part[(wave * M + r0) * kTileRows + n] = acc0;
    if (MR > 1 && r1 < M) part[(wave * M + r1) * kTileRows + n] = acc1;
    __syncthreads();
    // (a single-wave workgroup has fewer threads than m*16 outputs)
    for (int o = tid; o < M * kTileRows; o += blockDim.x) {
      const int r = o / kTileRows, nn = o % kTileRows;
      float s = 0.0f;
      for (int wv = 0; wv < nwaves; ++wv) s += part[(wv * M + r) * kTileRows + nn];
      const int row = tile * kTileRows + nn;
      if (row < a.n) a.y[(size_t)r * a.n + row] = s;
    }
    __syncthreads();
  }
}

size_t gemv_lds_bytes(int type, int m, int g, int nwaves) {
  const size_t xstride = (size_t)g * kGroupK + kRowPadHalves;
  return (size_t)2 * m * xstride * 2 +
         (type == MLQ_Q4_1 ? (size_t)m * g * kGroupBlocks * 4 : 0) +
         (size_t)nwaves * m * kTileRows * 4;
}

template <int QT, int MR>
hipError_t launch_typed(const GemvArgs& a, int nwaves, size_t lds,
                        hipStream_t stream) {
  // Opt in to more than the default 64 KiB of dynamic LDS when needed.
  static size_t configured = 64 * 1024;
  if (lds > configured) {
    hipError_t e = hipFuncSetAttribute((const void*)gemv_kernel<QT, MR>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    configured = lds;
  }
  const unsigned blocks =
      (unsigned)((a.nt + a.tiles_per_block - 1) / a.tiles_per_block);
  gemv_kernel<QT, MR><<<blocks, 64 * nwaves, lds, stream>>>(a);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_rows(const GemvArgs& a, int nwaves, size_t lds,
                       hipStream_t stream) {
  if (a.m == 1) return launch_typed<QT, 1>(a, nwaves, lds, stream);
  return launch_typed<QT, kGemvMaxRows>(a, nwaves, lds, stream);
}

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

}  // namespace

int gemv_max_k(int type, int m) {
  if (m < 1 || m > kGemvMaxRows) return 0;
  int g = 0;
  while (gemv_lds_bytes(type, m, g + 1, kMaxWaves) <= lds_limit()) ++g;
  return g * kGroupK;
}

hipError_t launch_gemv(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream) {
  const Geometry geo = geometry(w.n, w.k);
  if (m < 1 || m > kGemvMaxRows || w.k > gemv_max_k(w.type, m))
    return hipErrorInvalidValue;
  GemvArgs a;
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
  a.xstride = geo.g * kGroupK + kRowPadHalves;
  // K split: about 8 KiB of quants per wave per round of loads.
  const int per_wave = w.type == MLQ_Q8_0 ? 4 : 8;
  int nwaves = std::min(kMaxWaves, std::max(1, (geo.g + per_wave - 1) / per_wave));
  a.gw = (geo.g + nwaves - 1) / nwaves;
  nwaves = (geo.g + a.gw - 1) / a.gw;
  // Tuning knob: row tiles per workgroup (activation staging is amortised
  // over them), default 1.
  static const int tiles_per_block =
      std::max(1, env_int("MLQ_GEMV_TILES_PER_BLOCK", 1));
  a.tiles_per_block = tiles_per_block;
  const size_t lds = gemv_lds_bytes(w.type, m, geo.g, nwaves);
  switch (w.type) {
    case MLQ_Q8_0: return launch_rows<MLQ_Q8_0>(a, nwaves, lds, stream);
    case MLQ_Q4_0: return launch_rows<MLQ_Q4_0>(a, nwaves, lds, stream);
    default: return launch_rows<MLQ_Q4_1>(a, nwaves, lds, stream);
  }
}

}  // namespace mlq
