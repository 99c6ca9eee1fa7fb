// Int8-MFMA GEMM for q8_0 weights times q8_0-quantized activations, the
// int8 alternative to the fp16 prefill GEMM (gemm_mfma.hip):
//   y[m, n] = sum_b dx[m, b] * dw[n, b] * sum_{k in b} qx[m, k] * qw[n, k]
// with qx, dx the activations quantized by quantizeToQ80's rules
// (src/quant.cc:130-190) and qw, dw the weight's own codes and scales. The
// reference computes y = W x on fp32 x (src/quant.cc:505-628 on the CPU,
// src/cuda_quant.cu:78-128 on the GPU); this variant adds the activation
// quantization error (|x| / 254 per element at most) in exchange for an
// integer contraction.
//
//  - act_frag_kernel quantizes x into the workspace in MFMA fragment order:
//    codes [mtp][nbp][64 lanes][16 B] (32-row m tile, block, lane: row
//    32 mt + L % 32, elements 16 (L / 32) .. +15 of the block, each 4-byte
//    word in the weight layout's byte order: element 4w + i at byte
//    4w + i/2 + 2 (i%2)), scales [mtp][G][32 rows][4 blocks] fp16, zero for
//    rows past m and blocks past ceil(k/32). The contraction is over the same
//    permutation of k in both operands, so it is the plain dot product.
//  - gemm_i8_kernel: workgroup tile 128 (m) x 256 (n); eight waves in
//    2 (m) x 4 (n), each 64 x 64 = 2 x 2 32x32 tiles (WMT = 2), two waves
//    per SIMD; K in stages of two blocks. Four waves of 128 x 64 (WMT = 4)
//    measured 2x slower: the accumulators fill the VGPRs, so every MFMA
//    result went through AGPRs and back (one extra VALU copy per output). Weights come straight from the tiled layout (the q8 chunks of a
//    stage give each lane 16 codes of a block for two blocks; codes are
//    stored as q + 128, one XOR makes them signed); activations straight
//    from the workspace (every wave of a workgroup reads the same fragments,
//    which the L1 serves). Per (tile, block): one v_mfma_i32_32x32x32_i8
//    (k = 32 = one block) gives the block's integer dot products I; one
//    v_mfma_f32_32x32x16_f16 with the two fp16 scales in k slot 0 (every
//    other slot zero) gives S = dx * dw exactly in fp32 in the same lane
//    layout (a single fp16 product is exact, subnormal scales included);
//    then acc = fma(S, float(I), acc), two VALU instructions per output and
//    block (a convert and an FMA; float(I) is exact, |I| < 2^24), no weight
//    decode. A variant that seeded the int accumulator with 1.5 * 2^23 (so
//    the raw bits read as the float M + I, one VALU per output) and
//    subtracted M * sum_b S_b at the end was rejected: the MFMA's sum of
//    sixteen scale products of very different magnitudes is not rounded
//    like sequential fp32 adds, and M = 1.26e7 turned that into errors of
//    ~5 % on a block with a 144x larger scale than its neighbours.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../mlq_layout.h"
#include "act_q8.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;                  // x rows per workgroup
constexpr int kBN = 256;                  // W rows per workgroup
constexpr int kTiles = kBN / kTileRows;   // 16 weight row tiles
constexpr int kThreads = 256;
constexpr int kXcds = 8;
constexpr int kFragBytes = 1024;          // one (m tile, block) A fragment
constexpr uint32_t kOutOfRange = 0x80000000u;  // buffer offset that reads 0

struct I8Args {
  const uint8_t* qs;   // weight codes (tiled q8 layout)
  const uint8_t* d;    // weight scales (tiled)
  const uint8_t* xq;   // activation codes (fragment order)
  const uint8_t* xs;   // activation scales [mtp][g][32][4] fp16
  float* y;
  int m, n, g, nt;     // rows of x, rows of W, 128-k groups, W row tiles
  int nbp, mtp;        // blocks per row padded to groups (4g), 32-row m tiles
  int mtiles, ntiles;  // workgroup tiles
};

// x [m][k] fp32 -> fragment-order q8_0 codes and scales (layout above).
// Sixteen lanes per block (q8_block_codes); block-groups numbered
// ((mt * nbp + b) * 32 + row % 32), so a wave writes four rows of one block.
__global__ __launch_bounds__(256) void act_frag_kernel(const float* __restrict__ x,
                                                       uint8_t* __restrict__ xq,
                                                       uint16_t* __restrict__ xs, int m,
                                                       int k, int nb, int nbp, int g, int mtp) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t gid = t / kActLanes;
  const int part = (int)(t % kActLanes);
  const bool live = gid < (uint64_t)mtp * nbp * 32;
  const int rr = (int)(gid % 32);
  const uint64_t mb = gid / 32;
  const int b = live ? (int)(mb % nbp) : 0;
  const int mt = live ? (int)(mb / nbp) : 0;
  const int row = 32 * mt + rr;
  const bool real = live && row < m && b < nb;
  const int k0 = 32 * b + 2 * part;
  const float* xr = x + (size_t)row * k;
  const float v0 = real && k0 < k ? xr[k0] : 0.0f;
  const float v1 = real && k0 + 1 < k ? xr[k0 + 1] : 0.0f;
  const Q8Codes c = q8_block_codes(v0, v1);
  // elements 2p, 2p+1 (p = part) sit in word (2p % 16) / 4 of half 2p / 16;
  // as i = 0, 1 of the word they go to bytes 0, 2, as i = 2, 3 to bytes 1, 3
  const int sh = (part & 1) ? 8 : 0;
  uint32_t word = (((uint32_t)c.q0 & 0xffu) << sh) | (((uint32_t)c.q1 & 0xffu) << (sh + 16));
  word |= (uint32_t)__shfl_xor((int)word, 1, kActLanes);
  if (!live) return;
  const int half = part >> 3, w = (part & 7) >> 1;
  if ((part & 1) == 0) {
    const size_t off = (((size_t)mt * nbp + b) * 64 + rr + 32 * half) * 16 + 4 * w;
    *(uint32_t*)(xq + off) = word;
  }
  if (part == 0) xs[(((size_t)mt * g + b / 4) * 32 + rr) * 4 + (b & 3)] = (uint16_t)c.dbits;
}

// Operands of one stage (two blocks) held by one lane of a wave covering
// WMT 32-row m tiles.
template <int WMT>
struct Stage {
  uint4 c[2][2];     // weight chunks: column block j, quarter pair half ci
  uint32_t dw[2];    // weight scales of the two blocks (lanes 0..31; else 0)
  uint4 af[WMT][2];  // activation fragments: m tile i, block u
  uint32_t dx[WMT];  // activation scales of the two blocks (lanes 0..31)
};

__device__ __forceinline__ h8_t scale_operand(uint32_t pair, int u) {
  const uint32_t v = u ? (pair >> 16) : (pair & 0xffffu);
  return __builtin_bit_cast(h8_t, make_uint4(v, 0u, 0u, 0u));
}

// WMT: 32-row m tiles per wave. 4: four waves, each 128 x 64 of the
// workgroup tile; 2: eight waves in 2 (m) x 4 (n), each 64 x 64 (half the
// accumulator and operand registers, two waves per SIMD).
template <int WMT>
__global__ __launch_bounds__(kThreads * 4 / WMT, 1) void gemm_i8_kernel(I8Args a) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wn = (tid >> 6) & 3;            // wave's 64-column quarter
  const int im0 = (tid >> 8) * WMT;         // wave's first m tile (of 4)
  const int fr = lane & 31, o = lane >> 5, nr = lane & 15;

  // XCD-major numbering (hardware sends workgroup b to XCD b % 8): each XCD
  // gets a contiguous run of logical ids, m fastest, so the m tiles of one
  // weight column block share an L2
  const int nwg = a.mtiles * a.ntiles;
  const int bid = blockIdx.x;
  const int full = nwg / kXcds * kXcds;
  const int id = bid < full ? (bid % kXcds) * (full / kXcds) + bid / kXcds : bid;
  const int mt = id % a.mtiles, ntile = id / a.mtiles;
  const int mt32 = mt * (kBM / 32);
  const int tile0 = ntile * kTiles;

  // buffer ranges: m tiles past mtp and weight tiles past nt read as zero
  const int m32 = min(kBM / 32, a.mtp - mt32);
  const rsrc_t rx = make_rsrc(a.xq + (size_t)mt32 * a.nbp * kFragBytes,
                              (uint32_t)((size_t)m32 * a.nbp * kFragBytes));
  const rsrc_t rxs = make_rsrc(a.xs + (size_t)mt32 * a.g * 256, (uint32_t)(m32 * a.g * 256));
  const int tiles = min(kTiles, a.nt - tile0);
  const rsrc_t rq = make_rsrc(a.qs + (size_t)tile0 * a.g * 2048, (uint32_t)(tiles * a.g * 2048));
  const rsrc_t rd = make_rsrc(a.d + (size_t)tile0 * a.g * 128, (uint32_t)(tiles * a.g * 128));

  // this lane's weight row tile of column block j (relative to tile0)
  int trel[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) trel[j] = 4 * wn + 2 * j + ((lane >> 4) & 1);

  auto load = [&](Stage<WMT>& st, int s) {
    const int gi = s >> 1, h = s & 1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t unit = (uint32_t)(trel[j] * a.g + gi);
#pragma unroll
      for (int ci = 0; ci < 2; ++ci)
        st.c[j][ci] = buf_load16(rq, ((unit * 2 + h) * 64 + nr + 16 * (2 * o + ci)) * 16, 0);
      st.dw[j] = buf_load4(rd, o == 0 ? ((unit * kTileRows + nr) * 4 + 2 * h) * 2 : kOutOfRange, 0);
    }
#pragma unroll
    for (int i = 0; i < WMT; ++i) {
      const int im = im0 + i;
#pragma unroll
      for (int u = 0; u < 2; ++u)
        st.af[i][u] = buf_load16(rx, (uint32_t)(((im * a.nbp + 2 * s + u) * 64 + lane) * 16), 0);
      st.dx[i] = buf_load4(rxs, o == 0 ? (((im * a.g + gi) * 32 + fr) * 4 + 2 * h) * 2 : kOutOfRange,
                           0);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the loads where they are issued
  };

  f32x16_t acc[WMT][2];
#pragma unroll
  for (int i = 0; i < WMT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  const i32x16_t izero = {};
  const f32x16_t zero = {};

  auto compute = [&](const Stage<WMT>& st) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      i32x4_t bq[2];
      h8_t bs[2], as[WMT];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint4 c0 = st.c[j][0], c1 = st.c[j][1];
        bq[j] = (i32x4_t){(int)((u ? c0.z : c0.x) ^ 0x80808080u), (int)((u ? c0.w : c0.y) ^ 0x80808080u),
                          (int)((u ? c1.z : c1.x) ^ 0x80808080u), (int)((u ? c1.w : c1.y) ^ 0x80808080u)};
        bs[j] = scale_operand(st.dw[j], u);
      }
#pragma unroll
      for (int i = 0; i < WMT; ++i) as[i] = scale_operand(st.dx[i], u);
#pragma unroll
      for (int i = 0; i < WMT; ++i) {
        const i32x4_t aq = __builtin_bit_cast(i32x4_t, st.af[i][u]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const i32x16_t d = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq[j], izero, 0, 0, 0);
          const f32x16_t f = __builtin_convertvector(d, f32x16_t);
          const f32x16_t sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(as[i], bs[j], zero, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(sc[r], f[r], acc[i][j][r]);
        }
      }
    }
  };

  const int stages = 2 * a.g;  // even
  Stage<WMT> st0, st1;
  load(st0, 0);
  for (int s = 0; s < stages; s += 2) {
    load(st1, s + 1);
    compute(st0);
    load(st0, min(s + 2, stages - 1));  // past the end: re-reads the last stage
    compute(st1);
  }

  // output: lane holds D[8 (r/4) + 4 o + r%4][fr] of each 32x32 tile
  const int m0 = mt * kBM;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ncol = tile0 * kTileRows + 64 * wn + 32 * j + fr;
    if (ncol >= a.n) continue;
#pragma unroll
    for (int i = 0; i < WMT; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int mrow = m0 + 32 * (im0 + i) + 8 * (r >> 2) + 4 * o + (r & 3);
        if (mrow < a.m)
          a.y[(size_t)mrow * a.n + ncol] = acc[i][j][r];
      }
    }
  }
}

struct I8Geometry {
  int nb, g, nbp, mtp;
  size_t codes, scales_off, bytes;
};

I8Geometry i8_geometry(const mlq_weight& w, int m) {
  I8Geometry q;
  const Geometry geo = geometry(w.n, w.k);
  q.nb = geo.nb;
  q.g = geo.g;
  q.nbp = 4 * geo.g;
  q.mtp = (m + 31) / 32;
  q.codes = (size_t)q.mtp * q.nbp * kFragBytes;
  q.scales_off = (size_t)align_up(q.codes, kRegionAlign);
  q.bytes = q.scales_off + (size_t)q.mtp * q.g * 256;
  return q;
}

}  // namespace

size_t gemm_i8_workspace_bytes(const mlq_weight& w, int m) {
  return i8_geometry(w, m).bytes;
}

hipError_t launch_gemm_i8(const mlq_weight& w, const float* x, float* y, int m,
                          void* workspace, hipStream_t stream) {
  const I8Geometry q = i8_geometry(w, m);
  uint8_t* ws = (uint8_t*)workspace;
  {
    const uint64_t threads = (uint64_t)q.mtp * q.nbp * 32 * kActLanes;
    const unsigned block = 256;
    act_frag_kernel<<<(unsigned)((threads + block - 1) / block), block, 0, stream>>>(
        x, ws, (uint16_t*)(ws + q.scales_off), m, w.k, q.nb, q.nbp, q.g, q.mtp);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const Geometry geo = geometry(w.n, w.k);
  I8Args a;
  const uint8_t* base = (const uint8_t*)w.base;
  a.qs = base + w.qs_off;
  a.d = base + w.d_off;
  a.xq = ws;
  a.xs = ws + q.scales_off;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.g = q.g;
  a.nt = geo.nt;
  a.nbp = q.nbp;
  a.mtp = q.mtp;
  a.mtiles = (m + kBM - 1) / kBM;
  a.ntiles = (geo.nt + kTiles - 1) / kTiles;
  constexpr int kWmt = 2;
  gemm_i8_kernel<kWmt><<<a.mtiles * a.ntiles, kThreads * 4 / kWmt, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace mlq
