// Skinny GEMM for gfx950: y[m, n] = sum_k W[n, k] x[m, k] for m = 9..64
// (batched decode, SURVEY config c3).
//
// Between the decode GEMV (m <= 8) and the prefill GEMM (128-row tiles)
// neither fits: a 128-row activation tile wastes most of its MFMA rows and,
// with N = 4096, gives only 32 workgroups. This kernel keeps the GEMV's
// grid (one workgroup per 16-row weight tile, its waves splitting K, so the
// weights stream from HBM once with 256+ workgroups in flight) and runs the
// rows of x through v_mfma_f32_16x16x32_f16 in blocks of 16:
//  - x comes from the fp16 copy that mlq_linear_ws makes first (rows of kp
//    halves, zero past k). An MFMA A fragment is 16 contiguous bytes of one
//    row, so waves load fragments straight from that copy (L2-resident)
//    instead of staging x in LDS.
//  - Weights: one 1 KiB (q4) / 2 KiB (q8) line per (tile, 128-k group) as in
//    the GEMV; codes are decoded exactly and scaled by d in fp16 (one
//    rounding, the prefill GEMM's numerics), so the MFMA accumulates across
//    blocks with no per-block fixup.
//  - Group g+1's weight line and x fragments are requested before group g's
//    MFMAs run. K slices combine through LDS in slice order.
#include <hip/hip_runtime.h>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kWaves = 8;  // K slices per workgroup
constexpr int kThreads = 64 * kWaves;

struct SkinnyArgs {
  const uint8_t* qs;
  const uint8_t* d;
  const uint8_t* mn;
  const _Float16* xh;  // [m][kp] fp16, zero past k
  float* y;
  int m, n, g, kp;
  int gw;  // groups per wave
};

template <int QT, int MB>
struct Group {
  uint4 q, q2;   // weight line chunk(s)
  uint2 d, mm;   // four fp16 scales / mins
  uint4 a[MB][4];  // x fragments: m block, weight block
};

template <int QT, int MB>
__device__ __forceinline__ void load_group(const SkinnyArgs& a, Group<QT, MB>& gr,
                                           rsrc_t rq, rsrc_t rd, rsrc_t rm,
                                           rsrc_t rx, int j, int lane) {
  const uint32_t unit = (uint32_t)j;  // relative to the wave's first unit
  if (QT == MLQ_Q8_0) {
    gr.q = buf_load16_stream(rq, ((unit * 2) * 64 + lane) * 16, 0);
    gr.q2 = buf_load16_stream(rq, ((unit * 2 + 1) * 64 + lane) * 16, 0);
  } else {
    gr.q = buf_load16_stream(rq, (unit * 64 + lane) * 16, 0);
  }
  const uint32_t soff = (unit * kTileRows + (lane & 15)) * 8;
  gr.d = buf_load8(rd, soff, 0);
  if (QT == MLQ_Q4_1) gr.mm = buf_load8(rm, soff, 0);
  // A fragment of block b, m block mb: row 16mb + lane%16, k 32b + 8(lane/16)
  const int r = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      gr.a[mb][b] = buf_load16(
          rx, (uint32_t)(((16 * mb + r) * a.kp + j * kGroupK + 32 * b + 8 * kq) * 2), 0);
}

__device__ __forceinline__ h2_t splat(uint2 s, int b) {
  const uint32_t w = (b & 2) ? s.y : s.x;
  const _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)((b & 1) ? (w >> 16) : (w & 0xffffu)));
  return (h2_t){v, v};
}

// B fragment of block b: 8 codes of quarter lane/16 of row lane%16, decoded
// exactly and scaled in fp16.
template <int QT, int MB>
__device__ __forceinline__ h8_t decode(const Group<QT, MB>& gr, int b) {
  const h2_t d2 = splat(gr.d, b);
  uint4 o;
  if (QT == MLQ_Q8_0) {
    const uint4 q = b < 2 ? gr.q : gr.q2;
    const uint32_t w0 = (b & 1) ? q.z : q.x, w1 = (b & 1) ? q.w : q.y;
    const h2_t bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    uint32_t p0, p1, p2, p3;
    q8_pairs(w0, p0, p1);
    q8_pairs(w1, p2, p3);
    o.x = as_u32((as_h2(p0) - bias) * d2);
    o.y = as_u32((as_h2(p1) - bias) * d2);
    o.z = as_u32((as_h2(p2) - bias) * d2);
    o.w = as_u32((as_h2(p3) - bias) * d2);
  } else {
    const uint32_t w = b == 0 ? gr.q.x : b == 1 ? gr.q.y : b == 2 ? gr.q.z : gr.q.w;
    const float lo = QT == MLQ_Q4_0 ? 1032.0f : 1024.0f;
    const float hi = QT == MLQ_Q4_0 ? 72.0f : 64.0f;
    const h2_t blo = {(_Float16)lo, (_Float16)lo};
    const h2_t bhi = {(_Float16)hi, (_Float16)hi};
    const Q4Pairs p = q4_pairs(w);
    if (QT == MLQ_Q4_0) {
      o.x = as_u32((as_h2(p.p0) - blo) * d2);
      o.y = as_u32((as_h2(p.p1) - bhi) * d2);
      o.z = as_u32((as_h2(p.p2) - blo) * d2);
      o.w = as_u32((as_h2(p.p3) - bhi) * d2);
    } else {
      const h2_t m2 = splat(gr.mm, b);
      o.x = as_u32(__builtin_elementwise_fma(as_h2(p.p0) - blo, d2, m2));
      o.y = as_u32(__builtin_elementwise_fma(as_h2(p.p1) - bhi, d2, m2));
      o.z = as_u32(__builtin_elementwise_fma(as_h2(p.p2) - blo, d2, m2));
      o.w = as_u32(__builtin_elementwise_fma(as_h2(p.p3) - bhi, d2, m2));
    }
  }
  return __builtin_bit_cast(h8_t, o);
}

template <int QT, int MB>
__global__ __launch_bounds__(kThreads) void skinny_kernel(SkinnyArgs a) {
  __shared__ float part[kWaves * 64 * 16];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = blockIdx.x;
  const int g0 = wave * a.gw;
  const int ng = max(0, min(a.gw, a.g - g0));

  constexpr uint32_t QB = QT == MLQ_Q8_0 ? 2048u : 1024u;
  const size_t unit0 = (size_t)tile * a.g + g0;
  const rsrc_t rq = make_rsrc(a.qs + unit0 * QB, (uint32_t)ng * QB);
  const rsrc_t rd = make_rsrc(a.d + unit0 * 128, (uint32_t)ng * 128u);
  const rsrc_t rm = QT == MLQ_Q4_1 ? make_rsrc(a.mn + unit0 * 128, (uint32_t)ng * 128u) : rd;
  // x fragments of this wave's k range; rows past m read as zero
  const rsrc_t rx = make_rsrc(a.xh + (size_t)g0 * kGroupK,
                              (uint32_t)(((size_t)(a.m - 1) * a.kp + (size_t)ng * kGroupK) * 2));

  f4_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = (f4_t){0.f, 0.f, 0.f, 0.f};

  Group<QT, MB> gr[2];
  if (ng > 0) load_group<QT, MB>(a, gr[0], rq, rd, rm, rx, 0, lane);
  auto run = [&](Group<QT, MB>& cur, Group<QT, MB>& nxt, int j) {
    if (j + 1 < ng) load_group<QT, MB>(a, nxt, rq, rd, rm, rx, j + 1, lane);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const h8_t bf = decode<QT, MB>(cur, b);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(h8_t, cur.a[mb][b]), bf, acc[mb], 0, 0, 0);
    }
  };
  int j = 0;
  for (; j + 1 < ng; j += 2) {
    run(gr[0], gr[1], j);
    run(gr[1], gr[0], j + 1);
  }
  if (j < ng) run(gr[0], gr[1], j);

  // lane holds D[4*(lane/16) + i][lane%16]: activation row 16mb + 4(lane/16)
  // + i, weight row lane%16. K slices combine in slice order.
  const int col = lane & 15, rq4 = 4 * (lane >> 4);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      part[(wave * 64 + 16 * mb + rq4 + i) * 16 + col] = acc[mb][i];
  __syncthreads();
  for (int o = tid; o < a.m * 16; o += kThreads) {
    const int r = o / 16, c = o % 16;
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += part[(w * 64 + r) * 16 + c];
    const int row = tile * kTileRows + c;
    if (row < a.n) a.y[(size_t)r * a.n + row] = s;
  }
}

template <int QT>
hipError_t launch_typed(const SkinnyArgs& a, int nt, hipStream_t stream) {
  const int mb = (a.m + 15) / 16;
  switch (mb) {
    case 1: skinny_kernel<QT, 1><<<nt, kThreads, 0, stream>>>(a); break;
    case 2: skinny_kernel<QT, 2><<<nt, kThreads, 0, stream>>>(a); break;
    case 3: skinny_kernel<QT, 3><<<nt, kThreads, 0, stream>>>(a); break;
    default: skinny_kernel<QT, 4><<<nt, kThreads, 0, stream>>>(a); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_skinny(const mlq_weight& w, const _Float16* xh, int kp,
                         float* y, int m, hipStream_t stream) {
  if (m < 1 || m > kSkinnyMaxRows || kp % kGroupK != 0) return hipErrorInvalidValue;
  const Geometry geo = geometry(w.n, w.k);
  SkinnyArgs a;
  a.qs = (const uint8_t*)w.base + w.qs_off;
  a.d = (const uint8_t*)w.base + w.d_off;
  a.mn = w.type == MLQ_Q4_1 ? (const uint8_t*)w.base + w.m_off : nullptr;
  a.xh = xh;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.g = geo.g;
  a.kp = kp;
  a.gw = (geo.g + kWaves - 1) / kWaves;
  // 32-bit buffer offsets for the x fragments of a wave
  if ((size_t)m * kp * 2 >= (1ull << 31)) return hipErrorInvalidValue;
  switch (w.type) {
    case MLQ_Q8_0: return launch_typed<MLQ_Q8_0>(a, geo.nt, stream);
    case MLQ_Q4_0: return launch_typed<MLQ_Q4_0>(a, geo.nt, stream);
    default: return launch_typed<MLQ_Q4_1>(a, geo.nt, stream);
  }
}

}  // namespace mlq
