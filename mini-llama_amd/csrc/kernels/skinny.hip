// Skinny GEMM for gfx950: y[m, n] = sum_k W[n, k] x[m, k] for m = 9..64
// (batched decode, SURVEY config c3).
//
// Between the decode GEMV (m <= 8) and the prefill GEMM (128-row tiles)
// neither fits: a 128-row activation tile wastes most of its MFMA rows and,
// with N = 4096, gives only 32 workgroups. This kernel keeps the GEMV's
// grid (workgroups over 16-row weight tiles, their waves splitting K, so the
// weights stream from HBM once with 256+ workgroups in flight) and runs the
// rows of x through v_mfma_f32_16x16x32_f16 in blocks of 16:
//  - x comes from an fp16 copy that mlq_linear_ws makes first (each row
//    scaled by a power of two from its largest |x|, undone on the fp32
//    results, so any finite fp32 row fits fp16), written in MFMA fragment
//    order (rows padded to 16; per 128-k group, row block and
//    32-k block one run of 64 lanes x 16 bytes), so every x fragment load
//    of a wave is 1 KiB contiguous (L2-resident). x is re-read by every
//    workgroup: its load volume, not the weight stream, bounds the kernel
//    once m >= 32.
//  - A workgroup covers T = 1, 2 or 4 weight tiles and reuses each x
//    fragment for all of them (T chosen so that at least 256 workgroups
//    remain), dividing the x traffic by T.
//  - Weights: one 1 KiB (q4) / 2 KiB (q8) line per (tile, 128-k group) as in
//    the GEMV; codes are decoded exactly and scaled by d in fp16 (one
//    rounding, the prefill GEMM's numerics), so the MFMA accumulates across
//    blocks with no per-block fixup.
//  - Group g+1's weight lines and x fragments are requested before group
//    g's MFMAs run. K slices combine through LDS in slice order, one tile
//    at a time.
//  - Every workgroup needs the x fragments of its whole K range, so with
//    one K range per tile group each CU reads all of x (512 KiB at m = 64,
//    K = 4096; 2.4 MiB at K = 18944: that read, not the weights, bounds the
//    kernel). The K range can be split over S workgroups (S = 2..8): each
//    reads 1/S of x and writes fp32 partial outputs to the workspace, and
//    the prefill GEMM's reduce kernel sums the S slices in order and
//    applies the epilogue (deterministic). Handing the partials to the last
//    workgroup to finish inside the kernel instead (atomic count + device
//    fences) measured 10-20x slower on MI355X: a device-scope release
//    writes back the XCD's L2 and the acquire invalidates it.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"
#include "row_copy.h"

namespace mlq {
namespace {

constexpr int kWaves = 8;  // K slices per workgroup
constexpr int kThreads = 64 * kWaves;

struct SkinnyArgs {
  const uint8_t* qs;
  const uint8_t* d;
  const uint8_t* mn;
  const _Float16* xf;  // fragment-ordered fp16 copy of x (skinny_x_bytes)
  const int* rexp;     // row exponents of the copy: row r holds x[r] * 2^rexp[r]
  float* y;
  int m, n, g, nt;
  Epilogue epi;
  int ny;              // output columns: n, or n/2 under kEpiSwiGLU
  int splits;          // K ranges per tile group (workgroups per tile group)
  float* part;         // splits > 1: partial outputs [splits][m][n]
};

// One 128-k group of T weight tiles and the x fragments of all row blocks.
template <int QT, int MB, int T>
struct Group {
  uint4 q[T], q2[T];  // weight line chunk(s) per tile
  uint2 d[T], mm[T];  // four fp16 scales / mins per tile
  uint4 a[MB][4];     // x fragments: m block, weight block
};

template <int QT, int MB, int T>
__device__ __forceinline__ void load_group(Group<QT, MB, T>& gr, const rsrc_t (&rq)[T],
                                           const rsrc_t (&rd)[T], const rsrc_t (&rm)[T],
                                           rsrc_t rx, int j, int lane) {
  const uint32_t unit = (uint32_t)j;  // relative to the wave's first unit
#pragma unroll
  for (int t = 0; t < T; ++t) {
    if (QT == MLQ_Q8_0) {
      gr.q[t] = buf_load16_stream(rq[t], ((unit * 2) * 64 + lane) * 16, 0);
      gr.q2[t] = buf_load16_stream(rq[t], ((unit * 2 + 1) * 64 + lane) * 16, 0);
    } else {
      gr.q[t] = buf_load16_stream(rq[t], (unit * 64 + lane) * 16, 0);
    }
    const uint32_t soff = (unit * kTileRows + (lane & 15)) * 8;
    gr.d[t] = buf_load8(rd[t], soff, 0);
    if (QT == MLQ_Q4_1) gr.mm[t] = buf_load8(rm[t], soff, 0);
  }
  // A fragment of block b, row block mb: 64 lanes x 16 bytes, contiguous
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      gr.a[mb][b] = buf_load16(rx, (uint32_t)((((j * MB + mb) * 4 + b) * 64 + lane) * 16), 0);
}

__device__ __forceinline__ h2_t splat(uint2 s, int b) {
  const uint32_t w = (b & 2) ? s.y : s.x;
  const _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)((b & 1) ? (w >> 16) : (w & 0xffffu)));
  return (h2_t){v, v};
}

// B fragment of block b of tile t: 8 codes of quarter lane/16 of row
// lane%16, decoded exactly and scaled in fp16.
template <int QT, int MB, int T>
__device__ __forceinline__ h8_t decode(const Group<QT, MB, T>& gr, int t, int b) {
  const h2_t d2 = splat(gr.d[t], b);
  uint4 o;
  if (QT == MLQ_Q8_0) {
    const uint4 q = b < 2 ? gr.q[t] : gr.q2[t];
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
    const uint4 qq = gr.q[t];
    const uint32_t w = b == 0 ? qq.x : b == 1 ? qq.y : b == 2 ? qq.z : qq.w;
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
      const h2_t m2 = splat(gr.mm[t], b);
      o.x = as_u32(__builtin_elementwise_fma(as_h2(p.p0) - blo, d2, m2));
      o.y = as_u32(__builtin_elementwise_fma(as_h2(p.p1) - bhi, d2, m2));
      o.z = as_u32(__builtin_elementwise_fma(as_h2(p.p2) - blo, d2, m2));
      o.w = as_u32(__builtin_elementwise_fma(as_h2(p.p3) - bhi, d2, m2));
    }
  }
  return __builtin_bit_cast(h8_t, o);
}

template <int QT, int MB, int T>
__global__ __launch_bounds__(kThreads) void skinny_kernel(SkinnyArgs a) {
  __shared__ float part[kWaves * 64 * 16];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // consecutive workgroups take consecutive K ranges of one tile group
  // (hardware places workgroup b on XCD b % 8, so with S | 8 each XCD's
  // L2 holds the x fragments of one K range only)
  const int sp = blockIdx.x % a.splits;
  const int tg = blockIdx.x / a.splits;
  const int t0 = tg * T;
  const int kg0 = sp * a.g / a.splits, kg1 = (sp + 1) * a.g / a.splits;
  const int gw = (kg1 - kg0 + kWaves - 1) / kWaves;
  const int g0 = kg0 + wave * gw;
  const int ng = max(0, min(gw, kg1 - g0));

  constexpr uint32_t QB = QT == MLQ_Q8_0 ? 2048u : 1024u;
  rsrc_t rq[T], rd[T], rm[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    // tiles past nt read as zero
    const int tile = min(t0 + t, a.nt - 1);
    const uint32_t units = t0 + t < a.nt ? (uint32_t)ng : 0u;
    const size_t unit0 = (size_t)tile * a.g + g0;
    rq[t] = make_rsrc(a.qs + unit0 * QB, units * QB);
    rd[t] = make_rsrc(a.d + unit0 * 128, units * 128u);
    rm[t] = QT == MLQ_Q4_1 ? make_rsrc(a.mn + unit0 * 128, units * 128u) : rd[t];
  }
  // this wave's groups of the fragment-ordered x (padded rows are zero)
  const rsrc_t rx = make_rsrc(a.xf + (size_t)g0 * MB * 16 * kGroupK,
                              (uint32_t)((size_t)ng * MB * 16 * kGroupK * 2));

  f4_t acc[T][MB];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[t][mb] = (f4_t){0.f, 0.f, 0.f, 0.f};

  Group<QT, MB, T> gr[2];
  if (ng > 0) load_group<QT, MB, T>(gr[0], rq, rd, rm, rx, 0, lane);
  auto run = [&](Group<QT, MB, T>& cur, Group<QT, MB, T>& nxt, int j) {
    if (j + 1 < ng) load_group<QT, MB, T>(nxt, rq, rd, rm, rx, j + 1, lane);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const h8_t bf = decode<QT, MB, T>(cur, t, b);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[t][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(h8_t, cur.a[mb][b]), bf, acc[t][mb], 0, 0, 0);
      }
    }
  };
  int j = 0;
  for (; j + 1 < ng; j += 2) {
    run(gr[0], gr[1], j);
    run(gr[1], gr[0], j + 1);
  }
  if (j < ng) run(gr[0], gr[1], j);

  // lane holds D[4*(lane/16) + i][lane%16]: activation row 16mb + 4(lane/16)
  // + i, weight row lane%16 of tile t. Each row is scaled back by 2^-e of
  // its exponent; K slices combine in slice order, one tile at a time.
  const int col = lane & 15, rq4 = 4 * (lane >> 4);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int4 e4 = *(const int4*)(a.rexp + 16 * mb + rq4);
#pragma unroll
    for (int t = 0; t < T; ++t) {
      acc[t][mb][0] = ldexp_f(acc[t][mb][0], -e4.x);
      acc[t][mb][1] = ldexp_f(acc[t][mb][1], -e4.y);
      acc[t][mb][2] = ldexp_f(acc[t][mb][2], -e4.z);
      acc[t][mb][3] = ldexp_f(acc[t][mb][3], -e4.w);
    }
  }
  const bool split = a.splits > 1;
  // outputs of tile t from `sum` (K slices of the workgroup): the epilogue
  // into y
  auto store = [&](auto sum, int t) {
    if (a.epi.act == kEpiSwiGLU) {
      for (int o = tid; o < a.m * 8; o += kThreads) {
        const int r = o / 8, c = o % 8;
        const int row = (t0 + t) * kTileRows + c;
        if (row >= a.n) continue;
        const float g = add_bias(a.epi, sum(r, c, row), row);
        const float u = add_bias(a.epi, sum(r, c + 8, row + 8), row + 8);
        a.y[(size_t)r * a.ny + glu_col(row)] = silu_f(g) * u;
      }
    } else {
      for (int o = tid; o < a.m * 16; o += kThreads) {
        const int r = o / 16, c = o % 16;
        const int row = (t0 + t) * kTileRows + c;
        if (row < a.n) a.y[(size_t)r * a.n + row] = add_bias(a.epi, sum(r, c, row), row);
      }
    }
  };
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        part[(wave * 64 + 16 * mb + rq4 + i) * 16 + col] = acc[t][mb][i];
    __syncthreads();
    auto slice_sum = [&](int r, int c, int) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += part[(w * 64 + r) * 16 + c];
      return s;
    };
    if (!split) {
      store(slice_sum, t);
    } else {
      // this K range's partial outputs (no epilogue)
      float* out = a.part + (size_t)sp * a.m * a.n;
      for (int o = tid; o < a.m * 16; o += kThreads) {
        const int r = o / 16, c = o % 16;
        const int row = (t0 + t) * kTileRows + c;
        if (row < a.n) out[(size_t)r * a.n + row] = slice_sum(r, c, row);
      }
    }
    if (t + 1 < T) __syncthreads();
  }
}

int g_tiles_override = 0;   // mlq_set_skinny_plan; 0 = planner
int g_splits_override = 0;

struct SkinnyPlan {
  int tiles, splits;
};

// Weight tiles per workgroup (T) and K ranges per tile group (S). A
// workgroup reads its K range of x once for all of its T tiles, so per CU
// the x bytes are m_pad * (K / S) * 2 and the weight bytes T * 16 * (K / S)
// * (bytes per weight); more of either per workgroup means fewer
// workgroups. Cost model (us per round of workgroups on the chip): x at
// ~110 GB/s per CU from L2, weights at ~20 GB/s per CU (HBM shared by all
// CUs), the larger of the two, plus ~1.5 us per round; S > 1 adds the
// reduce launch (~2 us) and the partial slices (written, read, and y
// written: (2S + 1) m n 4 bytes at ~4 TB/s).
SkinnyPlan skinny_plan(int type, int m, int n, int k) {
  const Geometry geo = geometry(n, k);
  const int cus = device_cus();
  const double mpad = (double)((m + 15) / 16 * 16);
  const double bpw = type == MLQ_Q8_0 ? 34.0 / 32 : type == MLQ_Q4_1 ? 20.0 / 32 : 18.0 / 32;
  SkinnyPlan best{1, 1};
  double best_t = 0.0;
  bool have = false;
  for (int t : {1, 2, 4}) {
    if (g_tiles_override > 0 && t != g_tiles_override) continue;
    // four tiles of 64 rows spill registers for q8_0 / q4_1 (planner only)
    if (g_tiles_override == 0 && t == 4 && m > 48 && type != MLQ_Q4_0) continue;
    for (int sp : {1, 2, 4, 8, 0}) {
      // candidates 1, 2, 4, 8 within the group count, or the override alone
      if ((g_splits_override > 0) != (sp == 0) || sp > geo.g) continue;
      const int s_eff = sp == 0 ? std::min(g_splits_override, geo.g) : sp;
      const int wgs = (geo.nt + t - 1) / t * s_eff;
      const int rounds = (wgs + cus - 1) / cus;
      const double kr = (double)geo.g * kGroupK / s_eff;  // k per workgroup
      const double x_us = mpad * kr * 2.0 / 110e3;
      const double w_us = t * 16.0 * kr * bpw / 20e3;
      double cost = rounds * (std::max(x_us, w_us) + 1.5);
      if (s_eff > 1) cost += 2.0 + (2.0 * s_eff + 1.0) * m * (double)n * 4.0 / 4e6;
      if (!have || cost < best_t) {
        best = SkinnyPlan{t, s_eff};
        best_t = cost;
        have = true;
      }
    }
  }
  return best;
}

template <int QT, int T>
hipError_t launch_t(const SkinnyArgs& a, hipStream_t stream) {
  const int mb = (a.m + 15) / 16;
  const unsigned grid = (unsigned)((a.nt + T - 1) / T * a.splits);
  switch (mb) {
    case 1: skinny_kernel<QT, 1, T><<<grid, kThreads, 0, stream>>>(a); break;
    case 2: skinny_kernel<QT, 2, T><<<grid, kThreads, 0, stream>>>(a); break;
    case 3: skinny_kernel<QT, 3, T><<<grid, kThreads, 0, stream>>>(a); break;
    default: skinny_kernel<QT, 4, T><<<grid, kThreads, 0, stream>>>(a); break;
  }
  return hipGetLastError();
}

template <int QT>
hipError_t launch_typed(const SkinnyArgs& a, int tiles, hipStream_t stream) {
  switch (tiles) {
    case 1: return launch_t<QT, 1>(a, stream);
    case 2: return launch_t<QT, 2>(a, stream);
    default: return launch_t<QT, 4>(a, stream);
  }
}

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

size_t skinny_x_bytes(int m, int k) {
  const size_t kp = (size_t)(k + kGroupK - 1) / kGroupK * kGroupK;
  return (size_t)(m + 15) / 16 * 16 * kp * 2;
}

void set_skinny_plan(int tiles, int splits) {
  g_tiles_override = tiles;
  g_splits_override = splits;
}

// x copy, its row exponents (one per padded row), then (split K) the
// partial slices.
size_t skinny_exp_offset(int m, int k) { return align256(skinny_x_bytes(m, k)); }
size_t skinny_part_offset(int m, int k) {
  return skinny_exp_offset(m, k) + align256((size_t)(m + 15) / 16 * 16 * sizeof(int));
}

size_t skinny_workspace_bytes(int type, int m, int n, int k) {
  const SkinnyPlan p = skinny_plan(type, m, n, k);
  size_t b = skinny_part_offset(m, k);
  if (p.splits > 1) b += (size_t)p.splits * m * n * 4;
  return b;
}

hipError_t launch_skinny_ws(const mlq_weight& w, const float* x, float* y, int m,
                            void* ws, size_t ws_bytes, hipStream_t stream,
                            const Epilogue& epi) {
  if (m < 1 || m > kSkinnyMaxRows) return hipErrorInvalidValue;
  // 32-bit buffer offsets for the x fragments of a wave
  if (skinny_x_bytes(m, w.k) >= (1ull << 31)) return hipErrorInvalidValue;
  if (ws == nullptr || ws_bytes < skinny_workspace_bytes(w.type, m, w.n, w.k))
    return hipErrorInvalidValue;
  const Geometry geo = geometry(w.n, w.k);
  const SkinnyPlan p = skinny_plan(w.type, m, w.n, w.k);
  SkinnyArgs a;
  a.qs = (const uint8_t*)w.base + w.qs_off;
  a.d = (const uint8_t*)w.base + w.d_off;
  a.mn = w.type == MLQ_Q4_1 ? (const uint8_t*)w.base + w.m_off : nullptr;
  a.xf = (const _Float16*)ws;
  int* rexp = (int*)((uint8_t*)ws + skinny_exp_offset(m, w.k));
  a.rexp = rexp;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.g = geo.g;
  a.nt = geo.nt;
  a.epi = epi;
  a.ny = epi.act == kEpiSwiGLU ? w.n / 2 : w.n;
  a.splits = p.splits;
  a.part = p.splits > 1 ? (float*)((uint8_t*)ws + skinny_part_offset(m, w.k)) : nullptr;
  // fragment-ordered fp16 copy of x
  const int kp = (w.k + kGroupK - 1) / kGroupK * kGroupK;
  const int mbt = (m + 15) / 16;
  const RowCopyArgs ca{x, (_Float16*)ws, rexp, m, w.k, kp, mbt};
  hipError_t e = launch_row_copy<kCopyFragments>(ca, mbt * 16, stream);
  if (e != hipSuccess) return e;
  switch (w.type) {
    case MLQ_Q8_0: e = launch_typed<MLQ_Q8_0>(a, p.tiles, stream); break;
    case MLQ_Q4_0: e = launch_typed<MLQ_Q4_0>(a, p.tiles, stream); break;
    default: e = launch_typed<MLQ_Q4_1>(a, p.tiles, stream); break;
  }
  if (e != hipSuccess || p.splits == 1) return e;
  // the K ranges' partial slices, summed in order, then the epilogue
  return launch_split_reduce(a.part, y, m, w.n, p.splits, epi, stream);
}

}  // namespace mlq
