// Skinny GEMM for gfx950: y[m, n] = sum_k W[n, k] x[m, k] for m = 9..64
// (batched decode: 9..64 tokens through one Linear at once).
//
// Between the decode GEMV (m <= 8) and the prefill GEMM (128-row tiles)
// neither fits: a 128-row activation tile wastes most of its MFMA rows and,
// with N = 4096, gives only 32 workgroups. This kernel keeps the GEMV's
// grid (workgroups over 16-row weight tiles, their 8 waves splitting K, so
// the weights stream from HBM once with 256+ workgroups in flight) and runs
// the rows of x through v_mfma_f32_16x16x32_f16 in blocks of 16.
//
// Every workgroup needs the x columns of its whole K range, so x crosses
// L2 -> CU once per workgroup; next to the weight stream that traffic, and
// the launches, set the time. Measured on MI355X with a probe of the same
// access pattern (256 workgroups, everything in flight): 36 KiB of weights
// per CU plus 128 KiB of x per CU take 4.0 us, plus 256 KiB 5.0 us; a
// second launch in the graph costs ~1.6 us.
//  - 17..64 rows (and longer rows): x comes from an fp16 copy made by a
//    first kernel (each row scaled by a power of two from its largest |x|,
//    undone on the fp32 results, so any finite fp32 row fits fp16), written
//    in MFMA fragment order (rows padded to 16; per 128-k group, row block
//    and 32-k block one run of 64 lanes x 16 bytes), so every x fragment
//    load of a wave is 1 KiB contiguous.
//  - 9..16 rows with K <= 6144 (skinny_x32_kernel): fp32 x read by the
//    kernel itself (one launch), scaled per (row, 128-k group); see there.
//  - A workgroup covers T = 1, 2 or 4 weight tiles and reuses each x
//    fragment for all of them, dividing the x traffic by T.
//  - Weights: one 1 KiB (q4) / 2 KiB (q8) line per (tile, 128-k group) as in
//    the GEMV; codes are decoded exactly and scaled by d in fp16 (one
//    rounding, the prefill GEMM's numerics), so the MFMA accumulates across
//    blocks with no per-block fixup.
//  - A wave keeps D groups (weight lines and x fragments) in flight, its
//    whole K range when it fits in registers, in a ring refilled without
//    branches (every iteration issues the same loads, so the compiler's
//    wait counts stay exact; a conditional refill made it wait for every
//    outstanding load). D never exceeds the wave's group count: a load past
//    the buffer range reads zeros but still costs address-unit cycles.
//  - K slices combine through LDS in slice order, one tile at a time. The K
//    range can be split over S workgroups (S = 2..8): each reads 1/S of x
//    and writes fp32 partial outputs to the workspace, and the prefill
//    GEMM's reduce kernel sums the S slices in order and applies the
//    epilogue (deterministic). At c3's shapes the extra workgroups run as a
//    second round and the reduce adds a launch, so the planner keeps S = 1
//    there. Handing the partials to the last workgroup to finish inside the
//    kernel instead (atomic count + device fences) measured 10-20x slower
//    on MI355X: a device-scope release writes back the XCD's L2 and the
//    acquire invalidates it.
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
  const _Float16* xf;  // fragment-ordered fp16 copy of x (skinny_x_bytes), m > 16
  const int* rexp;     // row exponents of the copy: row r holds x[r] * 2^rexp[r]
  const float* x;      // fp32 x [m][k] (m <= 16: read by the kernel itself)
  float* y;
  int m, n, k, g, nt;
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

// Groups a wave keeps in flight: as many as ~160 registers less the
// accumulators hold (weight line + scales per tile, 16 registers of x
// fragments per row block), at most 4, a power of two.
template <int QT, int MB, int T>
constexpr int ring_depth() {
  constexpr int line = QT == MLQ_Q8_0 ? 10 : QT == MLQ_Q4_1 ? 8 : 6;
  constexpr int regs = T * line + 16 * MB;
  constexpr int fit = (160 - 4 * T * MB) / regs;
  return fit >= 4 ? 4 : fit >= 2 ? 2 : 1;
}

// K slices of a workgroup combined in slice order, one tile at a time, then
// the epilogue into y, or (split K) this K range's partial outputs.
// acc[t][mb] holds D[4*(lane/16) + i][lane%16] of MFMA row block mb: activation
// row 16 mb + 4 (lane/16) + i, weight row lane%16 of tile t, already in x's
// own scale. part: kWaves * 64 * 16 floats of LDS, free for reuse.
template <int T, int MB>
__device__ __forceinline__ void finish(const SkinnyArgs& a, f4_t (&acc)[T][MB], float* part,
                                       int sp, int t0) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, rq4 = 4 * (lane >> 4);
  const bool split = a.splits > 1;
  // outputs of tile t from `sum` (K slices of the workgroup): the epilogue
  // into y
  auto store = [&](auto sum, int t) {
    if (a.epi.act == kEpiSwiGLU) {
      for (int o = tid; o < a.m * 8; o += kThreads) {
        const int r = o / 8, c = o % 8;
        const int row = (t0 + t) * kTileRows + c;
        if (row >= a.n) continue;
        const float g = add_bias(a.epi, sum(r, c), row);
        const float u = add_bias(a.epi, sum(r, c + 8), row + 8);
        a.y[(size_t)r * a.ny + glu_col(row)] = silu_f(g) * u;
      }
    } else {
      for (int o = tid; o < a.m * 16; o += kThreads) {
        const int r = o / 16, c = o % 16;
        const int row = (t0 + t) * kTileRows + c;
        if (row < a.n) a.y[(size_t)r * a.n + row] = add_bias(a.epi, sum(r, c), row);
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
    auto slice_sum = [&](int r, int c) {
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
        if (row < a.n) out[(size_t)r * a.n + row] = slice_sum(r, c);
      }
    }
    if (t + 1 < T) __syncthreads();
  }
}

template <int QT, int MB, int T, int D>
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

  // D groups in flight (the wave's whole K range when it has at most D
  // groups): a ring refilled unconditionally while groups remain, so every
  // iteration issues the same loads in the same order and the compiler's
  // wait counts stay exact. The launch picks D <= the groups per wave, so
  // the only loads past a wave's range (they read zeros through the buffer
  // range and add nothing, but each still costs address-unit cycles) are
  // the last refill's when the group count is not a multiple of D.
  Group<QT, MB, T> gr[D];
#pragma unroll
  for (int i = 0; i < D; ++i) load_group<QT, MB, T>(gr[i], rq, rd, rm, rx, i, lane);
  auto run = [&](const Group<QT, MB, T>& cur) __attribute__((always_inline)) {
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
  for (; j + D < ng; j += D) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      run(gr[i]);
      load_group<QT, MB, T>(gr[i], rq, rd, rm, rx, j + i + D, lane);
    }
  }
#pragma unroll
  for (int i = 0; i < D; ++i) run(gr[i]);

  // lane holds D[4*(lane/16) + i][lane%16]: activation row 16mb + 4(lane/16)
  // + i, weight row lane%16 of tile t. Each row is scaled back by 2^-e of
  // its exponent; K slices combine in slice order, one tile at a time.
  const int rq4 = 4 * (lane >> 4);
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
  finish<T, MB>(a, acc, part, sp, t0);
}

// ---- m <= 16: fp32 x read by the kernel itself --------------------------------
// One row block, so every workgroup's x is 16 rows x its K range: reading
// it as fp32 costs twice the L2 -> CU bytes of the fp16 copy, but saves the
// copy's launch (one launch instead of two, ~2 us at these sizes). Each
// wave takes its groups two at a time (a chunk: 16 rows x 256 columns,
// 16 dwordx4 per lane, four lanes per row reading 64 contiguous bytes), with
// two chunks of x and weight lines in flight. Each (row, 128-k group) gets
// its own power of two (pow2_scale_exp of the group's largest |x|) before
// the fp16 rounding, the chunk is staged in the wave's LDS area in MFMA
// fragment order, and each group's MFMA sum is scaled back in fp32 before
// it joins the accumulator: any finite fp32 row fits, and the rounding of x
// does not depend on how K is split.
constexpr int kX32Chunk = 8 * 1024;  // fp16 fragments of one chunk per wave
constexpr int kX32Smem = kWaves * kX32Chunk + kWaves * 32 * 4;

// Weight lines of a chunk's two groups for T tiles.
template <int QT, int T>
struct Lines2 {
  uint4 q[2][T], q2[2][T];
  uint2 d[2][T], mm[2][T];
};

template <int QT, int T>
__device__ __forceinline__ void load_lines2(Lines2<QT, T>& w, const rsrc_t (&rq)[T],
                                            const rsrc_t (&rd)[T], const rsrc_t (&rm)[T], int c,
                                            int lane) {
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    const uint32_t unit = (uint32_t)(2 * c + gi);  // relative to the wave's first group
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (QT == MLQ_Q8_0) {
        w.q[gi][t] = buf_load16_stream(rq[t], ((unit * 2) * 64 + lane) * 16, 0);
        w.q2[gi][t] = buf_load16_stream(rq[t], ((unit * 2 + 1) * 64 + lane) * 16, 0);
      } else {
        w.q[gi][t] = buf_load16_stream(rq[t], (unit * 64 + lane) * 16, 0);
      }
      const uint32_t soff = (unit * kTileRows + (lane & 15)) * 8;
      w.d[gi][t] = buf_load8(rd[t], soff, 0);
      if (QT == MLQ_Q4_1) w.mm[gi][t] = buf_load8(rm[t], soff, 0);
    }
  }
}

// B fragment of block b of group gi, tile t (decode() of a Group).
template <int QT, int T>
__device__ __forceinline__ h8_t decode2(const Lines2<QT, T>& w, int gi, int t, int b) {
  Group<QT, 1, T> g1;
#pragma unroll
  for (int u = 0; u < T; ++u) {
    g1.q[u] = w.q[gi][u];
    g1.q2[u] = w.q2[gi][u];
    g1.d[u] = w.d[gi][u];
    g1.mm[u] = w.mm[gi][u];
  }
  return decode<QT, 1, T>(g1, t, b);
}

// Largest of a non-negative value over the four lanes of a quad (every lane
// of the quad gets it): DPP quad permutations, compared as integers.
__device__ __forceinline__ float quad_max_nonneg(float v) {
  int b = __builtin_bit_cast(int, v);
  b = max(b, __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  b = max(b, __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  return __builtin_bit_cast(float, b);
}

// Largest |x| of four values joined to m; NaN propagates (a NaN row's
// output is NaN whatever its scale). Two v_maximum3_f32 with abs modifiers.
__device__ __forceinline__ float abs_maximum4(float m, float4 v) {
  m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, __builtin_fabsf(v.x)),
                                    __builtin_fabsf(v.y));
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, __builtin_fabsf(v.z)),
                                       __builtin_fabsf(v.w));
}

// x * 2^e rounded once to fp16 (v_fma_mixlo / mixhi: the scaling is exact,
// so this is the rounding of the scaled value), two values per word.
__device__ __forceinline__ uint32_t scale_pack_h2(float a, float b, float s) {
  h2_t h;
  h.x = (_Float16)__builtin_fmaf(a, s, 0.0f);
  h.y = (_Float16)__builtin_fmaf(b, s, 0.0f);
  return as_u32(h);
}

template <int QT, int T>
__global__ __launch_bounds__(kThreads) void skinny_x32_kernel(SkinnyArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kX32Smem];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint8_t* sx = smem + wave * kX32Chunk;
  int* sexp = (int*)(smem + kWaves * kX32Chunk) + wave * 32;
  const int sp = blockIdx.x % a.splits;
  const int tg = blockIdx.x / a.splits;
  const int t0 = tg * T;
  const int kg0 = sp * a.g / a.splits, kg1 = (sp + 1) * a.g / a.splits;
  const int gw = (kg1 - kg0 + kWaves - 1) / kWaves;
  const int g0 = kg0 + wave * gw;
  const int ng = max(0, min(gw, kg1 - g0));
  const int nc = (ng + 1) / 2;  // chunks of two groups
  const int kend = min(a.k, (g0 + ng) * kGroupK);

  constexpr uint32_t QB = QT == MLQ_Q8_0 ? 2048u : 1024u;
  rsrc_t rq[T], rd[T], rm[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int tile = min(t0 + t, a.nt - 1);
    const uint32_t units = t0 + t < a.nt ? (uint32_t)ng : 0u;
    const size_t unit0 = (size_t)tile * a.g + g0;
    rq[t] = make_rsrc(a.qs + unit0 * QB, units * QB);
    rd[t] = make_rsrc(a.d + unit0 * 128, units * 128u);
    rm[t] = QT == MLQ_Q4_1 ? make_rsrc(a.mn + unit0 * 128, units * 128u) : rd[t];
  }
  const rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.m * a.k * 4));
  // quad rho = lane / 4 reads row rho; lane q = lane % 4 the 16 bytes at
  // column 16 j + 4 q of the chunk (j < 16). Rows past m start at offset
  // 2^31, past the buffer (m * k * 4 < 2^31), so every load of theirs reads
  // zeros; columns past the wave's range load zeros the same way (only the
  // wave's last chunk can hold any: the check is skipped, wave-uniformly,
  // for chunks that lie inside the range).
  const int rho = lane >> 2, q = lane & 3;
  const uint32_t xl = rho < a.m ? (uint32_t)((rho * a.k + 4 * q) * 4) : 0x80000000u;
  auto load_x = [&](float4 (&xv)[16], int c) __attribute__((always_inline)) {
    const int kb = (g0 + 2 * c) * kGroupK;
    const uint32_t base = xl + (uint32_t)kb * 4;
    if (kb + 2 * kGroupK <= kend) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        xv[j] = __builtin_bit_cast(float4, buf_load16(rx, base + 64 * j, 0));
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t off = kb + 16 * j + 4 * q < kend ? base + 64 * j : 0x80000000u;
        xv[j] = __builtin_bit_cast(float4, buf_load16(rx, off, 0));
      }
    }
  };
  // element 16 j + 4 q of the chunk is group j / 8, block (j / 2) % 4,
  // quarter 2 (j % 2) + q / 2, halves 4 (q % 2) .. +3 of fragment row rho
  const int wr_base = (rho + 16 * (q >> 1)) * 16 + 8 * (q & 1);
  const int rq4 = 4 * (lane >> 4);

  f4_t acc[T][1];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t][0] = (f4_t){0.f, 0.f, 0.f, 0.f};

  // chunk c from slot xv / w: exponents, fp16 fragments into LDS, then (with
  // REFILL) chunk c + 2's x requested into the same registers before the
  // MFMAs run
  auto run = [&](float4 (&xv)[16], const Lines2<QT, T>& w, int c, auto refill)
                 __attribute__((always_inline)) {
    float sc[2];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      float mx = 0.0f;
#pragma unroll
      for (int j = 8 * gi; j < 8 * gi + 8; ++j) mx = abs_maximum4(mx, xv[j]);
      // 2^e must be a finite float: groups whose largest |x| is below
      // 2^-112 keep e = 127 (they land below 2^15, coarser but finite)
      const int e = min(pow2_scale_exp(quad_max_nonneg(mx)), 127);
      sc[gi] = ldexp_f(1.0f, e);
      if (q == 0) sexp[gi * 16 + rho] = e;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float s = sc[j >> 3];
      const float4 v = xv[j];
      const uint2 h = make_uint2(scale_pack_h2(v.x, v.y, s), scale_pack_h2(v.z, v.w, s));
      const int frag = (j >> 3) * 4 + ((j >> 1) & 3);
      *(uint2*)(sx + frag * 1024 + (j & 1) * 512 + wr_base) = h;
    }
    if constexpr (decltype(refill)::value) load_x(xv, c + 2);
    // this wave's LDS writes complete before its lanes read them back
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      const int4 e4 = *(const int4*)(sexp + gi * 16 + rq4);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        f4_t sum = (f4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint4 af = *(const uint4*)(sx + (gi * 4 + b) * 1024 + lane * 16);
          sum = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, af),
                                                       decode2<QT, T>(w, gi, t, b), sum, 0, 0, 0);
        }
        acc[t][0][0] += ldexp_f(sum[0], -e4.x);
        acc[t][0][1] += ldexp_f(sum[1], -e4.y);
        acc[t][0][2] += ldexp_f(sum[2], -e4.z);
        acc[t][0][3] += ldexp_f(sum[3], -e4.w);
      }
    }
  };
  // two slots; a refill issues x then lines. A chunk past nc (nc odd, or
  // 1) runs on zeros. The first two chunks: q4_0 / q4_1 request both
  // chunks' weight lines (1 KiB a group, from HBM) before their activations
  // (L2 hits after the first workgroup of the XCD), which lets the lines'
  // longer trip start first (graph-timed, one box: 16 x 4096 x 4096 q4_0
  // 7.68 -> 7.42 us, q4_1 7.65 -> 7.58, 16 x 4608 x 3584 q4_0 9.46 ->
  // 8.87); q8_0's 2 KiB lines keep x and lines per chunk (lines first:
  // 8.14 -> 8.43).
  float4 xv[2][16];
  Lines2<QT, T> wl[2];
  if constexpr (QT == MLQ_Q8_0) {
    load_x(xv[0], 0);
    load_lines2<QT, T>(wl[0], rq, rd, rm, 0, lane);
    load_x(xv[1], 1);
    load_lines2<QT, T>(wl[1], rq, rd, rm, 1, lane);
  } else {
    load_lines2<QT, T>(wl[0], rq, rd, rm, 0, lane);
    load_lines2<QT, T>(wl[1], rq, rd, rm, 1, lane);
    load_x(xv[0], 0);
    load_x(xv[1], 1);
  }
  int c = 0;
  for (; c + 2 < nc; c += 2) {
    run(xv[0], wl[0], c, std::true_type());
    load_lines2<QT, T>(wl[0], rq, rd, rm, c + 2, lane);
    run(xv[1], wl[1], c + 1, std::true_type());
    load_lines2<QT, T>(wl[1], rq, rd, rm, c + 3, lane);
  }
  run(xv[0], wl[0], c, std::false_type());
  run(xv[1], wl[1], c + 1, std::false_type());

  __syncthreads();  // every wave is done with its staging area
  finish<T, 1>(a, acc, (float*)smem, sp, t0);
}

// m <= 16 rows with k % 4 == 0 (16-byte aligned rows) and k <= 6144: the
// fp32-input kernel, one weight tile per workgroup, K unsplit; otherwise
// the fp16 copy. Every workgroup converts its own x (about 4 VALU cycles
// per element per SIMD pair of waves), which for long rows costs more than
// the copy's launch (measured: m = 16, K = 4096: 7.5 us against 7.9 us
// through the copy; K = 18944: 26.9 us against 21.5 us).
bool uses_x32(int m, int k) { return m <= 16 && k % 4 == 0 && k <= 6144; }

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
  // fp32 x in the kernel: x bytes doubled, one tile per workgroup, or two
  // (q4_0) when that saves a round of workgroups: at one workgroup per CU
  // (its registers allow no second) a two-tile workgroup takes ~1.15x a
  // one-tile one (q4_0 M = 16: 4096 x 4096 7.7 vs 8.8 us, one round
  // either way; 4608 x 3584, 288 tiles: 13.8 us in two rounds vs 9.5 in one)
  const bool x32 = uses_x32(m, k);
  if (x32 && g_tiles_override == 0 && g_splits_override == 0) {
    int t = 1;
    if (type == MLQ_Q4_0) {
      const int r1 = (geo.nt + cus - 1) / cus, r2 = ((geo.nt + 1) / 2 + cus - 1) / cus;
      if (1.15 * r2 < r1) t = 2;
    }
    return SkinnyPlan{t, 1};
  }
  const double xb = x32 ? 4.0 : 2.0;
  for (int t : {1, 2, 4}) {
    if (x32) {
      // the fp32-x kernel: one tile, or two for q4_0 when overridden
      if (t != (g_tiles_override == 2 && type == MLQ_Q4_0 ? 2 : 1)) continue;
    } else if (g_tiles_override > 0 && t != g_tiles_override) {
      continue;
    }
    for (int sp : {1, 2, 4, 8, 0}) {
      // candidates 1, 2, 4, 8 within the group count, or the override alone
      if ((g_splits_override > 0) != (sp == 0) || sp > geo.g) continue;
      if (x32 && sp != 1 && g_splits_override == 0) continue;
      const int s_eff = sp == 0 ? std::min(g_splits_override, geo.g) : sp;
      const int wgs = (geo.nt + t - 1) / t * s_eff;
      const int rounds = (wgs + cus - 1) / cus;
      const double kr = (double)geo.g * kGroupK / s_eff;  // k per workgroup
      const double x_us = mpad * kr * xb / 110e3;
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

// Ring depth: the largest power of two <= the groups per wave, capped by
// ring_depth (registers).
template <int QT, int MB, int T>
void launch_d(const SkinnyArgs& a, unsigned grid, int gw, hipStream_t stream) {
  constexpr int cap = ring_depth<QT, MB, T>();
  if (cap >= 4 && gw >= 4)
    skinny_kernel<QT, MB, T, cap >= 4 ? 4 : 1><<<grid, kThreads, 0, stream>>>(a);
  else if (cap >= 2 && gw >= 2)
    skinny_kernel<QT, MB, T, cap >= 2 ? 2 : 1><<<grid, kThreads, 0, stream>>>(a);
  else
    skinny_kernel<QT, MB, T, 1><<<grid, kThreads, 0, stream>>>(a);
}

template <int QT, int T>
hipError_t launch_t(const SkinnyArgs& a, hipStream_t stream) {
  const int mb = (a.m + 15) / 16;
  const unsigned grid = (unsigned)((a.nt + T - 1) / T * a.splits);
  // groups per wave (the K range of a split over kWaves waves)
  const int gw = (a.g / a.splits + kWaves - 1) / kWaves;
  switch (mb) {
    case 1: launch_d<QT, 1, T>(a, grid, gw, stream); break;
    case 2: launch_d<QT, 2, T>(a, grid, gw, stream); break;
    case 3: launch_d<QT, 3, T>(a, grid, gw, stream); break;
    default: launch_d<QT, 4, T>(a, grid, gw, stream); break;
  }
  return hipGetLastError();
}

template <int QT>
hipError_t launch_typed(const SkinnyArgs& a, int tiles, hipStream_t stream) {
  if (uses_x32(a.m, a.k)) {
    // two tiles per workgroup fit the registers without spilling for q4_0
    // only (q8_0 / q4_1 lines are larger)
    if constexpr (QT == MLQ_Q4_0) {
      if (tiles == 2) {
        const unsigned grid2 = (unsigned)((a.nt + 1) / 2 * a.splits);
        skinny_x32_kernel<QT, 2><<<grid2, kThreads, 0, stream>>>(a);
        return hipGetLastError();
      }
    }
    const unsigned grid = (unsigned)(a.nt * a.splits);
    skinny_x32_kernel<QT, 1><<<grid, kThreads, 0, stream>>>(a);
    return hipGetLastError();
  }
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

// fp16 copy path: x copy, its row exponents (one per padded row), then
// (split K) the partial slices; fp32-input kernel: the partial slices only.
size_t skinny_exp_offset(int m, int k) { return uses_x32(m, k) ? 0 : align256(skinny_x_bytes(m, k)); }
size_t skinny_part_offset(int m, int k) {
  return uses_x32(m, k) ? 0
                        : skinny_exp_offset(m, k) +
                              align256((size_t)(m + 15) / 16 * 16 * sizeof(int));
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
  const size_t need = skinny_workspace_bytes(w.type, m, w.n, w.k);
  if (need > 0 && (ws == nullptr || ws_bytes < need)) return hipErrorInvalidValue;
  // fp32-input kernel: 32-bit buffer offsets into x (2^31 marks out of range)
  const bool x32 = uses_x32(m, w.k);
  if (x32 && (size_t)m * w.k * 4 >= (1ull << 31)) return hipErrorInvalidValue;
  const Geometry geo = geometry(w.n, w.k);
  const SkinnyPlan p = skinny_plan(w.type, m, w.n, w.k);
  SkinnyArgs a;
  a.qs = (const uint8_t*)w.base + w.qs_off;
  a.d = (const uint8_t*)w.base + w.d_off;
  a.mn = w.type == MLQ_Q4_1 ? (const uint8_t*)w.base + w.m_off : nullptr;
  a.xf = x32 ? nullptr : (const _Float16*)ws;
  int* rexp = x32 ? nullptr : (int*)((uint8_t*)ws + skinny_exp_offset(m, w.k));
  a.rexp = rexp;
  a.x = x;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.k = w.k;
  a.g = geo.g;
  a.nt = geo.nt;
  a.epi = epi;
  a.ny = epi.act == kEpiSwiGLU ? w.n / 2 : w.n;
  a.splits = p.splits;
  a.part = p.splits > 1 ? (float*)((uint8_t*)ws + skinny_part_offset(m, w.k)) : nullptr;
  hipError_t e = hipSuccess;
  if (!x32) {  // fragment-ordered fp16 copy of x
    const int kp = (w.k + kGroupK - 1) / kGroupK * kGroupK;
    const int mbt = (m + 15) / 16;
    const RowCopyArgs ca{x, (_Float16*)ws, rexp, m, w.k, kp, mbt};
    e = launch_row_copy<kCopyFragments>(ca, mbt * 16, stream);
    if (e != hipSuccess) return e;
  }
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
