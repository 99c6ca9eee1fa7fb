// Decode GEMV / skinny GEMM for gfx950: y[m, n] = sum_k W[n, k] x[m, k] for
// m = 1..8 activation rows.
//
// Replaces q80LinearKernel / q40LinearKernel / q41LinearKernel
// (src/cuda_quant.cu:78-182) for decode-sized m. Design (HBM-bound):
//  - A workgroup owns one 16-row tile; its S waves (S = 1..16) split the
//    tile's K range into contiguous runs of 128-k groups, sized so that the
//    whole grid is resident at once (about 16 waves per CU). Per group a
//    wave reads one contiguous 1 KiB (q4) / 2 KiB (q8) line with a dwordx4
//    per lane plus an 8-byte scale load; every weight byte is read from HBM
//    exactly once. Up to D groups are loaded up front (a register ring for
//    longer runs), and each group is decoded as soon as its data lands.
//  - Lane L = n + 16*kq holds quarter kq of the group's 4 blocks of row n,
//    which is the B operand of v_mfma_f32_16x16x32_f16 for one block. Codes
//    are decoded EXACTLY to fp16 (q-8, q, or q): one AND-OR places a code in
//    the mantissa of 1024 (or 64), one packed fp16 subtract removes the bias.
//  - Each wave stages the activations of its own K range in a private LDS
//    slice as an fp16 hi/lo pair (x = hi + lo to ~2^-22); the activation
//    loads are issued before the weight loads, so staging never waits on
//    HBM and no workgroup barrier is needed before the math. MFMA row 2r is
//    hi, row 2r+1 is lo of activation row r: up to 8 rows in one MFMA.
//  - Per block: acc += d * (D[hi] + D[lo]) in fp32 (+ m * sum(x) for q4_1),
//    so the result is fp32-class accurate (products are exact in fp32).
//  - K-split waves combine partial sums through LDS in a fixed order.
// Activations must be finite and |x| < 65504 (the fp16 range of the hi part).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kMaxSplit = 16;       // waves per workgroup (one tile)
constexpr int kTargetWaves = 4096;  // ~16 resident waves per CU on 256 CUs
constexpr int kRowPadHalves = 32;   // 64 B: consecutive LDS rows hit other banks
constexpr int kMaxXRegs = 4;        // float4 activation loads held per lane

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

struct GemvArgs {
  const uint8_t* qs;
  const uint16_t* d;
  const uint16_t* mn;
  const float* x;
  float* y;
  int m, n, k, g, nt;
  int split;     // waves per workgroup = K slices of its tile
  int gw;        // groups per wave (last slice may be shorter)
  int xstride;   // fp16 elements per staged activation row
  int wave_lds;  // bytes of LDS per wave (activation slice + block sums)
};

template <int QT>
struct Slot {
  uint4 q;
  uint4 q2;  // second 16-byte line (q8_0)
  uint2 d;   // four fp16 scales of the group's blocks
  uint2 m;   // four fp16 mins (q4_1)
};

template <int QT>
__device__ __forceinline__ void load_slot(const GemvArgs& a, Slot<QT>& s,
                                          size_t unit, int lane) {
  const int n = lane & 15;
  if (QT == MLQ_Q8_0) {
    s.q = *(const uint4*)(a.qs + ((unit * 2) * kLanes + lane) * 16);
    s.q2 = *(const uint4*)(a.qs + ((unit * 2 + 1) * kLanes + lane) * 16);
  } else {
    s.q = *(const uint4*)(a.qs + (unit * kLanes + lane) * 16);
  }
  s.d = *(const uint2*)(a.d + (unit * kTileRows + n) * kGroupBlocks);
  if (QT == MLQ_Q4_1)
    s.m = *(const uint2*)(a.mn + (unit * kTileRows + n) * kGroupBlocks);
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

// Four consecutive activations x[row][k..k+3], zero past k (vec: k is a
// multiple of 4, so whole float4 loads stay in bounds and aligned).
__device__ __forceinline__ float4 load_x4(const float* xr, int k, int kmax,
                                          bool vec) {
  if (vec && k + 4 <= kmax) return *(const float4*)(xr + k);
  float4 v;
  v.x = k + 0 < kmax ? xr[k + 0] : 0.0f;
  v.y = k + 1 < kmax ? xr[k + 1] : 0.0f;
  v.z = k + 2 < kmax ? xr[k + 2] : 0.0f;
  v.w = k + 3 < kmax ? xr[k + 3] : 0.0f;
  return v;
}

// fp32 pair -> fp16 hi pair + fp16 lo pair with hi + lo = (a, b) to ~2^-22.
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi,
                                       uint32_t& lo) {
  const h2_t h = __builtin_convertvector((f2_t){a, b}, h2_t);
  const h2_t l = __builtin_convertvector(
      (f2_t){a - (float)h.x, b - (float)h.y}, h2_t);
  hi = as_u32(h);
  lo = as_u32(l);
}

// hi/lo fp16 split of four activations written at column kl of rows 2r and
// 2r+1 of the wave's slice; returns their exact fp32 sum (q4_1 block sums).
__device__ __forceinline__ float stage4(_Float16* xs, int xstride, int r,
                                        int kl, float4 v) {
  uint2 hi, lo;
  split2(v.x, v.y, hi.x, lo.x);
  split2(v.z, v.w, hi.y, lo.y);
  *(uint2*)(xs + (size_t)(2 * r) * xstride + kl) = hi;
  *(uint2*)(xs + (size_t)(2 * r + 1) * xstride + kl) = lo;
  return (v.x + v.y) + (v.z + v.w);
}

template <int QT, int MR, int D>
__global__ __launch_bounds__(1024) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int M = a.m;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int slice = wave;                       // K slice of this wave
  const int tile = blockIdx.x;
  const int g0 = slice * a.gw;
  const int g1 = min(a.g, g0 + a.gw);
  const int ng = g1 - g0;
  const int n = lane & 15;   // W row within the tile (and MFMA A row)
  const int kq = lane >> 4;  // quarter of each block (and D row group)

  unsigned char* wl = smem + (size_t)wave * a.wave_lds;
  _Float16* xs = (_Float16*)wl;
  float* xsum = (float*)(wl + (size_t)2 * M * a.xstride * 2);
  float* part = (float*)(smem + (size_t)a.split * a.wave_lds);

  // ---- activations of this wave's K range ---------------------------------
  // M == 1 and a short range: loads are issued before the weight loads and
  // held in registers, so converting them never waits on HBM.
  const int c4 = ng * (kGroupK / 4);  // float4 per activation row of the slice
  const int kbase = g0 * kGroupK;
  const bool vec = (a.k & 3) == 0;
  const bool x_in_regs = M == 1 && c4 <= kMaxXRegs * 64;
  float4 xr[kMaxXRegs];
  if (x_in_regs) {
#pragma unroll
    for (int i = 0; i < kMaxXRegs; ++i) {
      const int c = lane + 64 * i;
      xr[i] = c < c4 ? load_x4(a.x, kbase + 4 * c, a.k, vec) : make_float4(0, 0, 0, 0);
    }
  }

  // ---- weight prologue: D groups in flight -------------------------------
  const size_t unit0 = (size_t)tile * a.g + g0;
  Slot<QT> ring[D];
#pragma unroll
  for (int s = 0; s < D; ++s) load_slot<QT>(a, ring[s], unit0 + min(s, ng - 1), lane);

  // ---- stage hi/lo activations (+ q4_1 block sums: 8 float4 per block) ---
  const int nblk_w = ng * kGroupBlocks;
  if (x_in_regs) {
#pragma unroll
    for (int i = 0; i < kMaxXRegs; ++i) {
      if (64 * i < c4) {  // wave-uniform
        const int c = lane + 64 * i;
        float sx = 0.0f;
        if (c < c4) sx = stage4(xs, a.xstride, 0, 4 * c, xr[i]);
        if (QT == MLQ_Q4_1) {
          sx += __shfl_xor(sx, 1);
          sx += __shfl_xor(sx, 2);
          sx += __shfl_xor(sx, 4);
          if (c < c4 && (c & 7) == 0) xsum[c >> 3] = sx;
        }
      }
    }
  } else {
    for (int r = 0; r < M; ++r) {
      const float* xrow = a.x + (size_t)r * a.k;
      for (int c0 = 0; c0 < c4; c0 += 64) {
        const int c = c0 + lane;
        float sx = 0.0f;
        if (c < c4) sx = stage4(xs, a.xstride, r, 4 * c, load_x4(xrow, kbase + 4 * c, a.k, vec));
        if (QT == MLQ_Q4_1) {
          sx += __shfl_xor(sx, 1);
          sx += __shfl_xor(sx, 2);
          sx += __shfl_xor(sx, 4);
          if (c < c4 && (c & 7) == 0) xsum[r * nblk_w + (c >> 3)] = sx;
        }
      }
    }
  }
  // the slice is private to this wave: only LDS completion is needed
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();

  // MFMA A row `n` carries activation row n/2 (hi for even n, lo for odd n).
  // Rows past 2m read row 0 again: their D rows are never used, and an
  // unmasked read costs no VALU work.
  const _Float16* arow = xs + (size_t)(n < 2 * M ? n : 0) * a.xstride + 8 * kq;
  const int r0 = 2 * kq, r1 = 2 * kq + 1;  // activation rows of this lane's D
  float acc0 = 0.0f, acc1 = 0.0f;

  // One group: unpack the slot (B fragments, scales), optionally refill the
  // slot's registers with group `refill` (its old contents are dead by then),
  // then the four MFMAs and fp32 fixups.
  auto group = [&](Slot<QT>& slot, int gl, bool do_refill, size_t refill) {
    h8_t bfrag[kGroupBlocks];
    float df[kGroupBlocks], mf[kGroupBlocks];
#pragma unroll
    for (int j = 0; j < kGroupBlocks; ++j) {
      if (QT == MLQ_Q8_0) {
        const uint4 q = (j < 2) ? slot.q : slot.q2;
        bfrag[j] = decode8<QT>((j & 1) ? q.z : q.x, (j & 1) ? q.w : q.y);
      } else {
        const uint32_t w0 = j == 0 ? slot.q.x : j == 1 ? slot.q.y
                          : j == 2 ? slot.q.z : slot.q.w;
        bfrag[j] = decode8<QT>(w0, 0);
      }
      df[j] = scale_at(slot.d, j);
      mf[j] = QT == MLQ_Q4_1 ? scale_at(slot.m, j) : 0.0f;
    }
    if (do_refill) load_slot<QT>(a, slot, refill, lane);
#pragma unroll
    for (int j = 0; j < kGroupBlocks; ++j) {
      const uint4 av = *(const uint4*)(arow + gl * kGroupK + j * kQK);
      const f4_t zero = {0.f, 0.f, 0.f, 0.f};
      const f4_t dd = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(h8_t, av), bfrag[j], zero, 0, 0, 0);
      acc0 = fmaf(df[j], dd[0] + dd[1], acc0);
      if (MR > 1) acc1 = fmaf(df[j], dd[2] + dd[3], acc1);
      if (QT == MLQ_Q4_1) {
        const int b = gl * kGroupBlocks + j;
        if (r0 < M) acc0 = fmaf(mf[j], xsum[r0 * ng * kGroupBlocks + b], acc0);
        if (MR > 1 && r1 < M) acc1 = fmaf(mf[j], xsum[r1 * ng * kGroupBlocks + b], acc1);
      }
    }
  };

  // Full chunks of D groups: every slot is consumed and refilled D groups
  // ahead (refills past the range repeat the last group and are never used).
  int gb = 0;
  for (; gb + D <= ng; gb += D) {
#pragma unroll
    for (int s = 0; s < D; ++s)
      group(ring[s], gb + s, true, unit0 + min(gb + s + D, ng - 1));
  }
  // Tail: the remaining groups are already in the ring; no more loads.
#pragma unroll
  for (int s = 0; s < D; ++s)
    if (gb + s < ng) group(ring[s], gb + s, false, 0);

  // ---- output ------------------------------------------------------------
  if (a.split == 1) {
    const int row = tile * kTileRows + n;
    if (row < a.n) {
      if (r0 < M) a.y[(size_t)r0 * a.n + row] = acc0;
      if (MR > 1 && r1 < M) a.y[(size_t)r1 * a.n + row] = acc1;
    }
    return;
  }
  // K slices combine in slice order (deterministic)
  if (r0 < M) part[(wave * M + r0) * kTileRows + n] = acc0;
  if (MR > 1 && r1 < M) part[(wave * M + r1) * kTileRows + n] = acc1;
  __syncthreads();
  for (int o = tid; o < M * kTileRows; o += blockDim.x) {
    const int r = o / kTileRows, nn = o % kTileRows;
    float s = 0.0f;
    for (int w = 0; w < a.split; ++w) s += part[(w * M + r) * kTileRows + nn];
    const int row = tile * kTileRows + nn;
    if (row < a.n) a.y[(size_t)r * a.n + row] = s;
  }
}

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

// Plan override: set through mlq_set_gemv_plan, initialised from the
// MLQ_GEMV_SPLIT / MLQ_GEMV_DEPTH environment variables (0 = automatic).
int g_split_override = -1;
int g_depth_override = -1;

int split_override() {
  if (g_split_override < 0) g_split_override = env_int("MLQ_GEMV_SPLIT", 0);
  return g_split_override;
}
int depth_override() {
  if (g_depth_override < 0) g_depth_override = env_int("MLQ_GEMV_DEPTH", 0);
  return g_depth_override;
}

struct Plan {
  int split, gw, depth;
  size_t wave_lds, lds;
};

size_t wave_lds_bytes(int type, int m, int gw) {
  const size_t xstride = (size_t)gw * kGroupK + kRowPadHalves;
  size_t b = (size_t)2 * m * xstride * 2;
  if (type == MLQ_Q4_1) b += (size_t)m * gw * kGroupBlocks * 4;
  return (b + 15) / 16 * 16;
}

Plan make_plan(int type, int m, const Geometry& geo) {
  Plan p;
  const int env_split = split_override();
  const int env_depth = depth_override();
  int depth = env_depth;
  if (depth != 2 && depth != 4 && depth != 8) depth = 8;
  p.depth = depth;
  // Default split: enough waves for the whole grid to be resident at about
  // 16 waves per CU, but at least two groups per wave.
  int split = 1;
  if (env_split >= 1 && env_split <= kMaxSplit && (env_split & (env_split - 1)) == 0) {
    split = env_split;
  } else {
    while (split < kMaxSplit && geo.nt * split < kTargetWaves &&
           (geo.g + 2 * split - 1) / (2 * split) >= 2)
      split *= 2;
  }
  split = std::min(split, std::max(1, geo.g));
  // Each wave stages its own K slice: widen the split until they fit in LDS.
  for (;;) {
    p.split = split;
    p.gw = (geo.g + split - 1) / split;
    p.wave_lds = wave_lds_bytes(type, m, p.gw);
    p.lds = p.wave_lds * split +
            (split > 1 ? (size_t)split * m * kTileRows * 4 : 0);
    if (p.lds <= lds_limit() || split >= kMaxSplit) break;
    split *= 2;
  }
  // every wave of the workgroup must own at least one group
  p.split = (geo.g + p.gw - 1) / p.gw;
  p.lds = p.wave_lds * p.split +
          (p.split > 1 ? (size_t)p.split * m * kTileRows * 4 : 0);
  return p;
}

template <int QT, int MR, int D>
hipError_t launch_typed(const GemvArgs& a, size_t lds, hipStream_t stream) {
  // Opt in to more than the default 64 KiB of dynamic LDS when needed.
  static size_t configured = 64 * 1024;
  if (lds > configured) {
    hipError_t e = hipFuncSetAttribute((const void*)gemv_kernel<QT, MR, D>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    configured = lds;
  }
  gemv_kernel<QT, MR, D><<<a.nt, 64 * a.split, lds, stream>>>(a);
  return hipGetLastError();
}

template <int QT, int MR>
hipError_t launch_depth(const GemvArgs& a, int depth, size_t lds,
                        hipStream_t stream) {
  switch (depth) {
    case 2: return launch_typed<QT, MR, 2>(a, lds, stream);
    case 4: return launch_typed<QT, MR, 4>(a, lds, stream);
    default: return launch_typed<QT, MR, 8>(a, lds, stream);
  }
}

template <int QT>
hipError_t launch_rows(const GemvArgs& a, int depth, size_t lds,
                       hipStream_t stream) {
  if (a.m == 1) return launch_depth<QT, 1>(a, depth, lds, stream);
  return launch_depth<QT, kGemvMaxRows>(a, depth, lds, stream);
}

}  // namespace

void set_gemv_plan(int split, int depth) {
  g_split_override = split;
  g_depth_override = depth;
}

int gemv_max_k(int type, int m) {
  if (m < 1 || m > kGemvMaxRows) return 0;
  // the largest K whose default plan fits the LDS budget
  int best = 0;
  for (int g = 1; g <= 4096; ++g) {
    const Geometry geo = geometry(kTileRows, g * kGroupK);
    if (make_plan(type, m, geo).lds > lds_limit()) break;
    best = g * kGroupK;
  }
  return best;
}

hipError_t launch_gemv(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream) {
  const Geometry geo = geometry(w.n, w.k);
  if (m < 1 || m > kGemvMaxRows) return hipErrorInvalidValue;
  const Plan p = make_plan(w.type, m, geo);
  if (p.lds > lds_limit()) return hipErrorInvalidValue;
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
  a.split = p.split;
  a.gw = p.gw;
  a.xstride = p.gw * kGroupK + kRowPadHalves;
  a.wave_lds = (int)p.wave_lds;
  switch (w.type) {
    case MLQ_Q8_0: return launch_rows<MLQ_Q8_0>(a, p.depth, p.lds, stream);
    case MLQ_Q4_0: return launch_rows<MLQ_Q4_0>(a, p.depth, p.lds, stream);
    default: return launch_rows<MLQ_Q4_1>(a, p.depth, p.lds, stream);
  }
}

}  // namespace mlq
