// GEMV on raw GGUF blocks (array of structs: the bytes of a GGUF tensor, as
// the reference uploads them): y[r][n] = sum_k W[n][k] x[r][k] for r < m <= 8,
// every weight byte read from HBM once, no repack. This is the raw-pointer
// meaning of the reference's cudaQ*LinearDeviceWeight / DeviceInput weight
// (src/cuda_quant.cu:300-361), behind mlq_linear_aos.
//  - A workgroup of 8 waves owns 8 output rows (one per wave) and stages x
//    [m][k] in LDS once (coalesced; 32 elements per block padded to 36
//    floats so lanes reading consecutive blocks hit different banks).
//  - A wave walks its row in chunks of 64 blocks. A chunk's bytes (64 x 34 /
//    18 / 20) are covered by 16-byte units loaded straight into the wave's
//    LDS area with buffer_load ... lds (no registers), the next chunk in
//    flight while the current one is used. The row's buffer range starts at
//    the 16-byte boundary below the row and ends at the 4-byte boundary past
//    it, so the loads stay inside the pages the row occupies and anything
//    past the row reads as zero.
//  - Lane l takes block l of the chunk: its scale(s) with 16-bit reads, its
//    codes with aligned 32-bit reads funnel-shifted by the block's 2-byte
//    offset (34- and 18-byte blocks alternate between 4-byte phases).
//  - Per element (d * q [+ m]) * x in fp32, the reference's per-element
//    dequant (src/quant.cc:477-503), accumulated per lane in block order;
//    the lanes' sums are added across the wave at the end.
#include <hip/hip_runtime.h>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kAosWaves = 8;
constexpr int kAosThreads = 64 * kAosWaves;
constexpr int kAosChunk = 64;                 // blocks per chunk (one per lane)
constexpr int kAosBuf = 3 * 1024;             // three 1 KiB DMA loads per chunk
constexpr int kXBlockFloats = 36;             // 32 elements + pad per block in LDS

struct AosArgs {
  const uint8_t* w;   // AoS blocks, row n at w + n * row_bytes
  const float* x;     // [m][k]
  float* y;           // [m][n]
  int n, k, nb, m;
  int row_bytes;
};

template <int QT>
constexpr int aos_block_bytes() {
  return QT == MLQ_Q8_0 ? 34 : QT == MLQ_Q4_0 ? 18 : 20;
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ float lds_f16(const uint8_t* p) {
  return half_bits_to_float(*(const uint16_t*)p);
}

// Four consecutive code words (16 bytes) starting at 2-byte aligned LDS
// offset `at`.
__device__ __forceinline__ void code_words(const uint8_t* buf, int at, uint32_t (&w)[8], int nw) {
  const int a0 = at & ~3;
  const uint32_t sh = (uint32_t)(at & 3) * 8;
  uint32_t prev = lds_u32(buf + a0);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < nw) {
      const uint32_t next = lds_u32(buf + a0 + 4 * (i + 1));
      w[i] = sh ? __builtin_amdgcn_alignbit(next, prev, sh) : prev;
      prev = next;
    }
  }
}

template <int QT, int MR>
__global__ __launch_bounds__(kAosThreads) void aos_gemv_kernel(AosArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int BS = aos_block_bytes<QT>();
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int xstride = a.nb * kXBlockFloats;  // floats per row of x in LDS
  float* xs = (float*)lds;
  uint8_t* wbuf = lds + (((size_t)MR * xstride * 4 + 255) & ~(size_t)255) +
                  (size_t)wave * 2 * kAosBuf;

  // x -> LDS, zero past k and for the rows past m up to MR
  const int kq = a.nb * 32;
  for (int i = tid; i < MR * kq; i += kAosThreads) {
    const int r = i / kq, c = i - r * kq;
    const float v = r < a.m && c < a.k ? a.x[(size_t)r * a.k + c] : 0.0f;
    xs[r * xstride + (c >> 5) * kXBlockFloats + (c & 31)] = v;
  }
  __syncthreads();

  const int row = blockIdx.x * kAosWaves + wave;
  if (row >= a.n) return;  // (no barrier below)
  const uint8_t* rowp = a.w + (size_t)row * a.row_bytes;
  const int lead = (int)((uintptr_t)rowp & 15);
  const rsrc_t rw = make_rsrc(rowp - lead, (uint32_t)((lead + a.row_bytes + 3) & ~3));
  const int chunks = (a.nb + kAosChunk - 1) / kAosChunk;

  // chunk c's 16-byte units [u0, u0 + 138) into buffer slot (c & 1); units
  // past the row read as zero
  auto fetch = [&](int c) __attribute__((always_inline)) {
    const int u0 = (lead + c * kAosChunk * BS) >> 4;
    uint8_t* dst = wbuf + (c & 1) * kAosBuf;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const uint32_t off = (uint32_t)((u0 + 64 * j + lane) * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rw, (__attribute__((address_space(3))) void*)(dst + 1024 * j), 16, off, 0, 0, 0);
    }
  };

  float acc[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) acc[r] = 0.0f;

  fetch(0);
  for (int c = 0; c < chunks; ++c) {
    if (c + 1 < chunks) {
      fetch(c + 1);
      __builtin_amdgcn_s_waitcnt(0x0F73);  // vmcnt(3): chunk c landed
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    __builtin_amdgcn_wave_barrier();
    const int b = c * kAosChunk + lane;
    if (b < a.nb) {
      const uint8_t* buf = wbuf + (c & 1) * kAosBuf;
      const int at = (lead + b * BS) - (((lead + c * kAosChunk * BS) >> 4) << 4);
      const float d = lds_f16(buf + at);
      const float* xb = xs + b * kXBlockFloats;
      if constexpr (QT == MLQ_Q8_0) {
        uint32_t w[8];
        code_words(buf, at + 2, w, 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float wv = d * (float)(int8_t)(w[i] >> (8 * j));
#pragma unroll
            for (int r = 0; r < MR; ++r) acc[r] = fmaf(wv, xb[r * xstride + 4 * i + j], acc[r]);
          }
        }
      } else {
        const float mn = QT == MLQ_Q4_1 ? lds_f16(buf + at + 2) : 0.0f;
        uint32_t w[8];
        code_words(buf, at + (QT == MLQ_Q4_1 ? 4 : 2), w, 4);
        // element e < 16: low nibble of byte e; e >= 16: high nibble of byte e - 16
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int q = (int)((w[i] >> (8 * j + 4 * half)) & 15);
              const float wv = QT == MLQ_Q4_0 ? d * (float)(q - 8) : d * (float)q + mn;
              const int e = 16 * half + 4 * i + j;
#pragma unroll
              for (int r = 0; r < MR; ++r) acc[r] = fmaf(wv, xb[r * xstride + e], acc[r]);
            }
          }
        }
      }
    }
    // this chunk's slot is refilled two chunks later: every lane is done
    // reading it before the next fetch (issued at the top of the loop)
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == 0 && r < a.m) a.y[(size_t)r * a.n + row] = s;
  }
}

// x rows the kernel holds for m activation rows (MR)
int aos_rows(int m) { return m == 1 ? 1 : m == 2 ? 2 : m <= 4 ? 4 : 8; }

size_t aos_lds_bytes(int m, int nb) {
  return (((size_t)aos_rows(m) * nb * kXBlockFloats * 4 + 255) & ~(size_t)255) +
         (size_t)kAosWaves * 2 * kAosBuf;
}

size_t aos_lds_limit() {
  static const size_t limit = [] {
    int dev = 0, bytes = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) !=
            hipSuccess ||
        bytes <= 0)
      return (size_t)64 * 1024;
    return (size_t)bytes;
  }();
  return limit;
}

template <int QT, int MR>
hipError_t launch_mr(const AosArgs& a, size_t lds, hipStream_t stream) {
  const hipError_t e = allow_dynamic_lds((const void*)aos_gemv_kernel<QT, MR>, lds);
  if (e != hipSuccess) return e;
  const unsigned grid = (unsigned)((a.n + kAosWaves - 1) / kAosWaves);
  aos_gemv_kernel<QT, MR><<<grid, kAosThreads, lds, stream>>>(a);
  return hipGetLastError();
}

template <int QT>
hipError_t launch_typed(const AosArgs& a, size_t lds, hipStream_t stream) {
  if (a.m == 1) return launch_mr<QT, 1>(a, lds, stream);
  if (a.m == 2) return launch_mr<QT, 2>(a, lds, stream);
  if (a.m <= 4) return launch_mr<QT, 4>(a, lds, stream);
  return launch_mr<QT, 8>(a, lds, stream);
}

}  // namespace

bool aos_gemv_supported(int type, int m, int n, int k) {
  if (m < 1 || m > 8 || n < 1 || k < 1) return false;
  if (type != MLQ_Q8_0 && type != MLQ_Q4_0 && type != MLQ_Q4_1) return false;
  const int nb = (k + kQK - 1) / kQK;
  return aos_lds_bytes(m, nb) <= aos_lds_limit();
}

hipError_t launch_aos_gemv(int type, const void* aos, int n, int k, const float* x, float* y,
                           int m, hipStream_t stream) {
  if (!aos_gemv_supported(type, m, n, k)) return hipErrorInvalidValue;
  AosArgs a;
  a.w = (const uint8_t*)aos;
  a.x = x;
  a.y = y;
  a.n = n;
  a.k = k;
  a.nb = (k + kQK - 1) / kQK;
  a.m = m;
  const int bs = type == MLQ_Q8_0 ? 34 : type == MLQ_Q4_0 ? 18 : 20;
  a.row_bytes = a.nb * bs;
  const size_t lds = aos_lds_bytes(m, a.nb);
  switch (type) {
    case MLQ_Q8_0: return launch_typed<MLQ_Q8_0>(a, lds, stream);
    case MLQ_Q4_0: return launch_typed<MLQ_Q4_0>(a, lds, stream);
    default: return launch_typed<MLQ_Q4_1>(a, lds, stream);
  }
}

}  // namespace mlq
