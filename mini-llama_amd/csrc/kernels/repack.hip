// Weight-format kernels for gfx950:
//  - repack_kernel: GGUF AoS blocks (device) -> tiled layout (mlq_layout.h);
//    the device twin of the host repack used by the upload path.
//  - dequant_kernel: tiled layout -> fp32 rows, exactly d*q / d*(q-8) /
//    d*q+m, the reference's dequantizeFromQ* (src/quant.cc:192-392).
//  - bias_kernel: y[m, :] += bias (the reference adds it on the host,
//    src/cuda_quant.cu:229-235).
//  - act_q8_0_kernel: fp32 rows -> q8_0 blocks with the reference's
//    quantizeToQ80 rules (src/quant.cc:130-190), bit for bit.
// These are off the hot path (one-time or debug); they favour clarity.
#include <hip/hip_runtime.h>

#include "act_q8.h"

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

struct RepackArgs {
  const uint8_t* aos;  // GGUF blocks, row-major [n][nb]
  uint8_t* qs;
  uint16_t* d;
  uint16_t* m;
  Geometry geo;
  // alignment gaps between and after the regions ([begin, end) byte
  // offsets from the weight base): zeroed, like the host repack does
  uint8_t* base;
  uint64_t gap[3][2];
};

// One thread per padded (row, block); padding blocks decode to 0.
template <int QT>
__global__ void repack_kernel(RepackArgs a) {
  const int bpr = a.geo.g * kGroupBlocks;  // padded blocks per row
  const uint64_t total = (uint64_t)a.geo.nt * kTileRows * bpr;
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) {
    uint64_t g = idx - total;
    for (int i = 0; i < 3; ++i) {
      const uint64_t len = a.gap[i][1] - a.gap[i][0];
      if (g < len) {
        a.base[a.gap[i][0] + g] = 0;
        return;
      }
      g -= len;
    }
    return;
  }
  const int row = (int)(idx / bpr), b = (int)(idx % bpr);
  const bool real = row < a.geo.n && b < a.geo.nb;
  const int bytes = QT == MLQ_Q8_0 ? 34 : (QT == MLQ_Q4_0 ? 18 : 20);
  const uint8_t* src =
      real ? a.aos + ((uint64_t)row * a.geo.nb + b) * bytes : nullptr;
  repack_block(QT, a.geo, row, b, src, a.qs, a.d, a.m);
}

struct DequantArgs {
  const uint8_t* qs;
  const uint16_t* d;
  const uint16_t* m;
  float* out;
  Geometry geo;
  int row0, rows;
};

// One thread per output element of rows [row0, row0 + rows): exactly the
// reference's d*q, d*(q-8), d*q+m in fp32 (d*q is exact, so contraction of
// the q4_1 multiply-add cannot change the result).
template <int QT>
__global__ void dequant_kernel(DequantArgs a) {
  const int k = a.geo.k;
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (uint64_t)a.rows * k) return;
  const int row = a.row0 + (int)(idx / k);
  const int kk = (int)(idx % k);
  const int b = kk / kQK, e = kk % kQK;
  const uint64_t si = scale_index(a.geo, row, b);
  const float d = half_bits_to_float(a.d[si]);
  const int c = read_code(QT, a.geo, a.qs, row, b, e);
  float v;
  if (QT == MLQ_Q8_0) {
    v = d * (float)c;
  } else if (QT == MLQ_Q4_0) {
    v = d * (float)(c - 8);
  } else {
    v = d * (float)c + half_bits_to_float(a.m[si]);
  }
  a.out[idx] = v;
}

__global__ void bias_kernel(float* y, const float* bias, int m, int n) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (uint64_t)m * n) return;
  y[idx] += bias[idx % n];
}

}  // namespace

hipError_t launch_repack(int type, const void* aos, int n, int k,
                         const mlq_weight& w, hipStream_t stream) {
  const Geometry geo = geometry(n, k);
  RepackArgs a;
  a.aos = (const uint8_t*)aos;
  a.qs = (uint8_t*)w.base + w.qs_off;
  a.d = (uint16_t*)((uint8_t*)w.base + w.d_off);
  a.m = type == MLQ_Q4_1 ? (uint16_t*)((uint8_t*)w.base + w.m_off) : nullptr;
  a.geo = geo;
  a.base = (uint8_t*)w.base;
  const uint64_t qbytes = unit_count(geo) * kLanes * quant_bytes_per_lane(type);
  const uint64_t sbytes = scale_count(geo) * 2;
  const uint64_t d_end = w.d_off + sbytes;
  a.gap[0][0] = w.qs_off + qbytes;
  a.gap[0][1] = w.d_off;
  a.gap[1][0] = d_end;
  a.gap[1][1] = type == MLQ_Q4_1 ? w.m_off : w.bytes;
  a.gap[2][0] = type == MLQ_Q4_1 ? w.m_off + sbytes : w.bytes;
  a.gap[2][1] = w.bytes;
  const uint64_t gaps = (a.gap[0][1] - a.gap[0][0]) + (a.gap[1][1] - a.gap[1][0]) +
                        (a.gap[2][1] - a.gap[2][0]);
  const uint64_t total = (uint64_t)geo.nt * kTileRows * geo.g * kGroupBlocks;
  const unsigned threads = 256;
  const unsigned blocks = (unsigned)((total + gaps + threads - 1) / threads);
  switch (type) {
    case MLQ_Q8_0:
      repack_kernel<MLQ_Q8_0><<<blocks, threads, 0, stream>>>(a);
      break;
    case MLQ_Q4_0:
      repack_kernel<MLQ_Q4_0><<<blocks, threads, 0, stream>>>(a);
      break;
    default:
      repack_kernel<MLQ_Q4_1><<<blocks, threads, 0, stream>>>(a);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const mlq_weight& w, int row0, int rows, float* out,
                          hipStream_t stream) {
  const Geometry geo = geometry(w.n, w.k);
  DequantArgs a;
  a.qs = (const uint8_t*)w.base + w.qs_off;
  a.d = (const uint16_t*)((const uint8_t*)w.base + w.d_off);
  a.m = w.type == MLQ_Q4_1
            ? (const uint16_t*)((const uint8_t*)w.base + w.m_off)
            : nullptr;
  a.out = out;
  a.geo = geo;
  a.row0 = row0;
  a.rows = rows;
  const uint64_t total = (uint64_t)rows * w.k;
  const unsigned threads = 256;
  const unsigned blocks = (unsigned)((total + threads - 1) / threads);
  switch (w.type) {
    case MLQ_Q8_0:
      dequant_kernel<MLQ_Q8_0><<<blocks, threads, 0, stream>>>(a);
      break;
    case MLQ_Q4_0:
      dequant_kernel<MLQ_Q4_0><<<blocks, threads, 0, stream>>>(a);
      break;
    default:
      dequant_kernel<MLQ_Q4_1><<<blocks, threads, 0, stream>>>(a);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_bias(float* y, const float* bias, int m, int n,
                       hipStream_t stream) {
  const uint64_t total = (uint64_t)m * n;
  const unsigned threads = 256;
  const unsigned blocks = (unsigned)((total + threads - 1) / threads);
  bias_kernel<<<blocks, threads, 0, stream>>>(y, bias, m, n);
  return hipGetLastError();
}

namespace {

// Sixteen lanes per 32-element block (kActLanes), two elements each: block
// g of the [rows][nb] output is row g / nb, block g % nb of that row. Every
// store is one aligned 16-bit word per lane (34-byte blocks are only 2-byte
// aligned; lane 15 stores d, so no lane holds two adjacent words to merge).
__global__ __launch_bounds__(256) void act_q8_0_kernel(const float* __restrict__ x,
                                                       uint8_t* __restrict__ out,
                                                       int rows, int k, int nb) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t g = t / kActLanes;
  const int part = (int)(t % kActLanes);
  const bool live = g < (uint64_t)rows * nb;  // lanes past the end only shuffle
  const int row = live ? (int)(g / nb) : 0;
  const int blk = live ? (int)(g % nb) : 0;
  const int k0 = blk * 32 + part * 2;
  const float* xr = x + (size_t)row * k;
  // past the row: padding (quantizes to code 0)
  const float v0 = live && k0 < k ? xr[k0] : 0.0f;
  const float v1 = live && k0 + 1 < k ? xr[k0 + 1] : 0.0f;
  const Q8Codes c = q8_block_codes(v0, v1);
  if (!live) return;
  // block: fp16 d, then qs[32]
  uint16_t* ob = (uint16_t*)(out + g * 34);
  ob[1 + part] = (uint16_t)(((uint32_t)c.q0 & 0xffu) | (((uint32_t)c.q1 & 0xffu) << 8));
  if (part == kActLanes - 1) ob[0] = (uint16_t)c.dbits;
}

}  // namespace

hipError_t launch_quantize_act_q8_0(const float* x, int rows, int k, void* out,
                                    hipStream_t stream) {
  const int nb = (k + 31) / 32;
  const uint64_t threads = (uint64_t)rows * nb * kActLanes;
  const unsigned block = 256;
  act_q8_0_kernel<<<(unsigned)((threads + block - 1) / block), block, 0, stream>>>(
      x, (uint8_t*)out, rows, k, nb);
  return hipGetLastError();
}

}  // namespace mlq
