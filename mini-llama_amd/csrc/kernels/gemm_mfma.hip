// Prefill / batched GEMM on gfx950 MFMA: y[m, n] = sum_k W[n, k] x[m, k].
//
// The reference never issues m > 1 on the GPU (src/batch.cc:32-55 loops
// tokens); its kernels (src/cuda_quant.cu:78-182) re-stream W once per row
// of x (grid.y = rows). This kernel is a dense contraction instead:
//  - Workgroup tile 128 (m) x 256 (n), four waves side by side in n, each
//    wave 128 x 64 = 4 x 2 v_mfma_f32_32x32x16_f16 (fp32 accumulate). Every
//    weight is decoded by exactly one wave of the workgroup (the VALU decode
//    is the scarce resource next to the MFMAs), and every decoded fragment
//    feeds four MFMAs.
//  - K advances in stages of 64 (half of a 128-k group). Activations go
//    through LDS slabs [row][k] with a 16-byte row pad (every A fragment is
//    one conflict-free ds_read_b128); all four waves read the whole slab.
//  - Weights never touch LDS: each wave loads its own B fragments straight
//    from the tiled layout (two 16-byte chunks per lane cover a stage's four
//    k steps) and decodes them in registers (codes exact, then scaled by d
//    in fp16: one rounding, like d*q rounded to fp16).
//  - Software pipeline, one wave per SIMD per workgroup (two workgroups per
//    CU for q4_0, see OCC below): three LDS slabs (stage s reads
//    slab s%3, x(s+2) is written into slab (s+2)%3, and the first fragments
//    of stage s+1 are read from slab (s+1)%3 before the stage's barrier),
//    weights three stages deep in registers, the A fragments and decoded B
//    fragments of k step t+1 prepared while the MFMAs of step t run. Global
//    loads, LDS reads and LDS writes are spread one at a time between the
//    MFMAs (sched_group_barrier), so neither the texture unit nor the LDS
//    sees a burst from all four waves at once.
//  - Workgroups are numbered XCD-major: the m-tiles of one weight column
//    block run on the same XCD and share its L2.
//  - With a workspace, x is first converted once to an fp16 copy
//    (row_copy.h): the GEMM then moves half the activation bytes per
//    stage and does no conversion work. Without one it reads fp32 x.
//  - Any finite fp32 activations: each row enters the MFMAs as x * 2^e_r
//    (e_r = pow2_scale_exp of the row's largest |x|: from the fp16 copy's
//    row exponents, or found by the workgroup before its K loop when it
//    reads fp32 x), and the epilogue scales row r by 2^-e_r (exact).
// The scale is applied before the MFMA (per weight), so no per-block fixup
// of the accumulators is needed; that is what keeps VALU work independent of
// m (an int8 MFMA variant would need a per-(m, n, block) fp32 fixup).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"
#include "row_copy.h"

namespace mlq {
namespace {

constexpr int kBM = 128;           // x rows per workgroup
constexpr int kBN = 256;           // W rows per workgroup (16 row tiles)
constexpr int kBK = 64;            // k per stage
constexpr int kTiles = kBN / kTileRows;  // 16: wave wn, column block j covers tiles 4wn+2j, +1
constexpr int kThreads = 256;
constexpr int kStride = kBK + 8;   // halves per LDS row (144 B)
constexpr int kXcds = 8;

typedef float f16v_t __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const uint8_t* qs;
  const uint8_t* d;
  const uint8_t* mn;
  const float* x;      // fp32 activations [m][k] (XF32 modes)
  const _Float16* xh;  // fp16 activations [m][kp] (XF16 mode, workspace)
  const int* rexp;     // XF16 mode: row exponents of xh (x[r] * 2^rexp[r])
  float* y;
  float* part;         // split-K partial outputs [splits][m][n] (splits > 1)
  int m, n, k, g, nt;
  int kp;              // row stride of xh: k rounded up to whole stages
  int mtiles, ntiles;  // output tiles
  int splits;          // K ranges per output tile (workgroups per tile)
  Epilogue epi;        // applied here when splits == 1, else by the reduce
  GemmOut out;         // residual / fp16 output (EXT kernels and the reduce)
  int ny;              // output columns: n, or n/2 under kEpiSwiGLU
};

// Activation source: fp32 rows loaded as float4 (k % 4 == 0), fp32 loaded
// element by element, or the fp16 copy made by x_to_f16 in a workspace.
enum XMode { kXF32Vec = 0, kXF32Scalar = 1, kXF16 = 2 };

// Activations of one stage held in registers by one thread: rows t/16 + 16j,
// k 4*(t%16) .. +3 of the stage.
struct XStage {
  float4 xa[8];  // fp32 modes
  uint4 xh[4];   // fp16 mode: rows t/8 + 32j, k 8*(t%8) .. +7
};

// Weight fragments of one stage held in registers by one lane of one wave:
// for each of the wave's two 32-column blocks j, two 16-byte (q8) or 8-byte
// (q4) chunks of the tiled layout (quarters kq = o and 2 + o, o = lane/32)
// and the fp16 scales (and mins) of the stage's two blocks.
template <int QT>
struct WStage {
  uint4 c[2][2];
  uint32_t dd[2];
  uint32_t mm[2];
};

__device__ __forceinline__ h2_t h2_splat(uint32_t bits16) {
  const _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (h2_t){v, v};
}

// VEC: k % 4 == 0, so activation rows are 16-byte aligned and a float4 is
// either wholly inside the range or wholly past it. Otherwise each element
// is loaded (and range-checked) on its own. A compile-time choice: a runtime
// branch around the loads makes the compiler wait for each load in turn.
template <int XM>
__device__ __forceinline__ void load_x(const GemmArgs& a, XStage& st, rsrc_t rx,
                                       int s, int tid) {
  const int k0 = s * kBK;
  if (XM == kXF16) {
    const int c = tid & 7;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = (tid >> 3) + 32 * j;
      st.xh[j] = buf_load16(rx, (uint32_t)((r * a.kp + k0 + 8 * c) * 2), 0);
    }
    return;
  }
  const int c = tid & 15;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = (tid >> 4) + 16 * j;
    const uint32_t off = (uint32_t)((r * a.k + k0 + 4 * c) * 4);
    if (XM == kXF32Vec) {
      st.xa[j] = __builtin_bit_cast(float4, buf_load16(rx, off, 0));
    } else {
      st.xa[j].x = __builtin_bit_cast(float, buf_load4(rx, off, 0));
      st.xa[j].y = __builtin_bit_cast(float, buf_load4(rx, off + 4, 0));
      st.xa[j].z = __builtin_bit_cast(float, buf_load4(rx, off + 8, 0));
      st.xa[j].w = __builtin_bit_cast(float, buf_load4(rx, off + 12, 0));
    }
  }
}

// Activations of a stage into the LDS slab [row][k] (fp32 modes convert;
// the fp16 copy is already zero past k).
template <int XM>
__device__ __forceinline__ void store_x(const GemmArgs& a, XStage& st,
                                        _Float16* as, int s, int tid, const int* sexp) {
  if (XM == kXF16) {
    const int c = tid & 7;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = (tid >> 3) + 32 * j;
      *(uint4*)(as + r * kStride + 8 * c) = st.xh[j];
    }
    return;
  }
  const int k0 = s * kBK;
  const int c = tid & 15;
  // k tail: elements at or past k are zero (the row's next elements belong
  // to the following row)
  if (k0 + kBK > a.k) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kk = k0 + 4 * c;
      if (kk + 0 >= a.k) st.xa[j].x = 0.0f;
      if (kk + 1 >= a.k) st.xa[j].y = 0.0f;
      if (kk + 2 >= a.k) st.xa[j].z = 0.0f;
      if (kk + 3 >= a.k) st.xa[j].w = 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = (tid >> 4) + 16 * j;
    const int e = sexp[r];  // the row's power-of-two scale
    uint2 hv;
    hv.x = pack_h2(ldexp_f(st.xa[j].x, e), ldexp_f(st.xa[j].y, e));
    hv.y = pack_h2(ldexp_f(st.xa[j].z, e), ldexp_f(st.xa[j].w, e));
    *(uint2*)(as + r * kStride + 4 * c) = hv;
  }
}

// The MFMA B operand of v_mfma_f32_32x32x16_f16 for lane L is column L%32
// (W row 16t + n of this wave's block j: t = 4wn + 2j + (L%32)/16,
// n = L%16) at k octet o = L/32 of the 16-k step. In the tiled layout that
// octet is quarter kq = 2*(ks%2) + o of block 2h + ks/2 (stage = half h of
// group gi): the lane's chunks at lane n + 16*o and n + 16*(2+o) of the
// tile's line hold all four k steps of the stage.
template <int QT>
__device__ __forceinline__ void load_w(const GemmArgs& a, WStage<QT>& st,
                                       rsrc_t rq, rsrc_t rd, rsrc_t rm, int s,
                                       int lane, int wn) {
  const int gi = s >> 1, h = s & 1;
  const int n = lane & 15, o = lane >> 5;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = 4 * wn + 2 * j + ((lane >> 4) & 1);
    const uint32_t unit = (uint32_t)(t * a.g + gi);
#pragma unroll
    for (int ci = 0; ci < 2; ++ci) {
      const int lq = n + 16 * (2 * ci + o);  // lane of the line holding kq
      if (QT == MLQ_Q8_0) {
        st.c[j][ci] = buf_load16(rq, ((unit * 2 + h) * 64 + lq) * 16, 0);
      } else {
        const uint2 v = buf_load8(rq, (unit * 64 + lq) * 16 + 8 * h, 0);
        st.c[j][ci] = make_uint4(v.x, v.y, 0, 0);
      }
    }
    const uint32_t soff = ((unit * kTileRows + n) * 4 + 2 * h) * 2;
    st.dd[j] = buf_load4(rd, soff, 0);
    if (QT == MLQ_Q4_1) st.mm[j] = buf_load4(rm, soff, 0);
  }
}

// Decodes the fragment of block j, k step ks: 8 codes -> fp16 d*q (d*(q-8),
// d*q+m), one rounding.
template <int QT>
__device__ __forceinline__ h8_t decode_w(const WStage<QT>& st, int j, int ks) {
  const int ci = ks & 1, blk = ks >> 1;
  const uint32_t dbits = blk ? (st.dd[j] >> 16) : (st.dd[j] & 0xffffu);
  const h2_t d2 = h2_splat(dbits);
  uint4 o;
  if (QT == MLQ_Q8_0) {
    const uint4 c = st.c[j][ci];
    const uint32_t w0 = blk ? c.z : c.x, w1 = blk ? c.w : c.y;
    const h2_t b = {(_Float16)1152.0f, (_Float16)1152.0f};
    uint32_t p0, p1, p2, p3;
    q8_pairs(w0, p0, p1);
    q8_pairs(w1, p2, p3);
    o.x = as_u32((as_h2(p0) - b) * d2);
    o.y = as_u32((as_h2(p1) - b) * d2);
    o.z = as_u32((as_h2(p2) - b) * d2);
    o.w = as_u32((as_h2(p3) - b) * d2);
  } else {
    const uint32_t w = blk ? st.c[j][ci].y : st.c[j][ci].x;
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
      const uint32_t mbits = blk ? (st.mm[j] >> 16) : (st.mm[j] & 0xffffu);
      const h2_t m2 = h2_splat(mbits);
      o.x = as_u32(__builtin_elementwise_fma(as_h2(p.p0) - blo, d2, m2));
      o.y = as_u32(__builtin_elementwise_fma(as_h2(p.p1) - bhi, d2, m2));
      o.z = as_u32(__builtin_elementwise_fma(as_h2(p.p2) - blo, d2, m2));
      o.w = as_u32(__builtin_elementwise_fma(as_h2(p.p3) - bhi, d2, m2));
    }
  }
  return __builtin_bit_cast(h8_t, o);
}

template <int N>
struct Slot { static constexpr int v = N; };

// OCC: workgroups per CU the register budget is sized for; XS: activation
// register slots. q4_0 with the fp16 copy of x fits the whole pipeline in
// 256 registers a lane, so two workgroups share a CU and each hides the
// other's decode and LDS latency (measured 5-12 % faster on 512-2048-row
// shapes, neutral on small grids). q8_0 and q4_1 carry more weight
// registers per stage: they fit two per CU with one activation slot (x of
// stage s+2 requested in k step 0 of stage s, stored in its last), which
// wins only when the grid has more workgroups than CUs (3-8 %; 2-8 % slower
// on smaller grids), so the launcher picks it by grid size.
// EXT: the output epilogue also adds GemmOut.residual (a separate
// instantiation: per-element branches in the store code of every kernel
// measured 3-6 % slower main loops).
template <int QT, int XM, int OCC = 1, int XS = 2, bool EXT = false>
__global__ __launch_bounds__(kThreads, OCC) void gemm_kernel(GemmArgs a) {
  constexpr int kXS = XS;  // activation register slots (1 or 2)
  __shared__ __align__(16) _Float16 as_buf[3][kBM * kStride];
  __shared__ __align__(16) int sexp[kBM];  // row exponents of the m tile

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wn = tid >> 6;  // wave: W rows 64wn .. 64wn+63 of the tile

  // XCD-major numbering: hardware sends workgroup b to XCD b % 8; remap so
  // that each XCD gets a contiguous run of logical ids (m fastest).
  const int nwg = a.mtiles * a.ntiles;
  const int b = blockIdx.x;
  const int full = nwg / kXcds * kXcds;
  const int id = b < full ? (b % kXcds) * (full / kXcds) + b / kXcds : b;
  // m fastest, then the K range, then the weight column block: the
  // workgroups that share a weight block's K range are neighbours
  const int mt = id % a.mtiles, rest = id / a.mtiles;
  const int sp = rest % a.splits, ntile = rest / a.splits;
  const int m0 = mt * kBM;
  const int tile0 = ntile * kTiles;  // first W row tile
  // this workgroup's 128-k groups [g0, g1): 2 stages each
  const int g0 = sp * a.g / a.splits, g1 = (sp + 1) * a.g / a.splits;
  const int sbase = 2 * g0;

  // buffer ranges: rows past m / tiles past nt read as zero
  const int rows = min(kBM, a.m - m0);
  const rsrc_t rx = XM == kXF16
      ? make_rsrc(a.xh + (size_t)m0 * a.kp, (uint32_t)((size_t)rows * a.kp * 2))
      : make_rsrc(a.x + (size_t)m0 * a.k, (uint32_t)((size_t)rows * a.k * 4));
  const int tiles = min(kTiles, a.nt - tile0);
  const uint32_t qbytes = (uint32_t)tiles * a.g * (QT == MLQ_Q8_0 ? 2048u : 1024u);
  const rsrc_t rq = make_rsrc(a.qs + (size_t)tile0 * a.g * (QT == MLQ_Q8_0 ? 2048 : 1024), qbytes);
  const uint32_t sbytes = (uint32_t)tiles * a.g * 128u;
  const rsrc_t rd = make_rsrc(a.d + (size_t)tile0 * a.g * 128, sbytes);
  const rsrc_t rm = QT == MLQ_Q4_1 ? make_rsrc(a.mn + (size_t)tile0 * a.g * 128, sbytes) : rd;

  // Row exponents of the tile's rows: from the fp16 copy, or (fp32 x) from
  // the rows' largest |x| over all of K, 16 threads per row
  if constexpr (XM == kXF16) {
    if (tid < kBM) sexp[tid] = tid < rows ? a.rexp[m0 + tid] : 0;
  } else {
    // a thread scans its eight rows r0 + 16p together, every load of a k
    // step (and of the next, unrolled) in flight at once: one row at a time
    // with a loop-carried maximum kept one load in flight and took ~3x the
    // GEMM itself (rows past m read zero through the buffer range)
    constexpr int kPasses = kBM / (kThreads / 16);
    const int c = tid & 15, r0 = tid >> 4;
    float mx[kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) mx[p] = 0.0f;
    if constexpr (XM == kXF32Vec) {
#pragma unroll 2
      for (int kk = 4 * c; kk < a.k; kk += 64) {
        float4 v[kPasses];
#pragma unroll
        for (int p = 0; p < kPasses; ++p)
          v[p] = __builtin_bit_cast(float4,
                                    buf_load16(rx, (uint32_t)(((r0 + 16 * p) * a.k + kk) * 4), 0));
#pragma unroll
        for (int p = 0; p < kPasses; ++p) mx[p] = abs_max4(mx[p], v[p]);
      }
    } else {
#pragma unroll 4
      for (int kk = c; kk < a.k; kk += 16) {
        float v[kPasses];
#pragma unroll
        for (int p = 0; p < kPasses; ++p)
          v[p] = __builtin_bit_cast(float, buf_load4(rx, (uint32_t)(((r0 + 16 * p) * a.k + kk) * 4), 0));
#pragma unroll
        for (int p = 0; p < kPasses; ++p) mx[p] = fmaxf(mx[p], fabsf(v[p]));
      }
    }
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      float m = mx[p];
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      if (c == 0) sexp[r0 + 16 * p] = pow2_scale_exp(m);
    }
  }
  __syncthreads();

  f16v_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int stages = 2 * (g1 - g0);  // even, >= 2
  const int last = stages - 1;
  // stage indices below are relative to the workgroup's K range
  auto lx = [&](XStage& st, int rel) { load_x<XM>(a, st, rx, sbase + rel, tid); };
  auto lw = [&](WStage<QT>& st, int rel) {
    load_w<QT>(a, st, rq, rd, rm, sbase + rel, lane, wn);
  };
  auto sx = [&](XStage& st, int slab, int rel) {
    store_x<XM>(a, st, as_buf[slab], sbase + rel, tid, sexp);
  };
  // fragment rows of this lane: MFMA operand row/col = lane % 32, k octet
  // = lane / 32
  const int fr = lane & 31, fk = 8 * (lane >> 5);
  auto read_a = [&](h8_t (&af)[4], int slab, int ks) {
    const _Float16* as = as_buf[slab];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *(const h8_t*)(as + (32 * i + fr) * kStride + 16 * ks + fk);
  };

  // prologue: slabs 0 and 1 hold x(0), x(1); W(0), W(1) in slots 0 and 1;
  // with two x slots x(2) waits in slot 0
  XStage xs[kXS];
  WStage<QT> ws[3];
  if constexpr (kXS == 2) {
    lx(xs[0], 0);
    lw(ws[0], 0);
    lx(xs[1], 1);
    lw(ws[1], 1);
    sx(xs[0], 0, 0);
    sx(xs[1], 1, 1);
    lx(xs[0], min(2, last));
  } else {
    lx(xs[0], 0);
    lw(ws[0], 0);
    lw(ws[1], 1);
    sx(xs[0], 0, 0);
    lx(xs[0], 1);
    sx(xs[0], 1, 1);
  }
  __syncthreads();

  // q8_0 two workgroups per CU: A fragments read in their own k step (the
  // other workgroup hides the LDS latency) instead of one step ahead; the
  // 16 registers this frees keep the kernel within 256 without spills (a
  // spill reload in the loop waits for every outstanding load)
  constexpr bool kPrefA = !(OCC == 2 && QT == MLQ_Q8_0);
  h8_t af[4], bf[2];
  if constexpr (kPrefA) read_a(af, 0, 0);
#pragma unroll
  for (int j = 0; j < 2; ++j) bf[j] = decode_w<QT>(ws[0], j, 0);

  // Stage s; the register slots are compile-time (S = s mod 6): weights of
  // stage s in slot s%3 (s+1 in flight in (s+1)%3, s+2 requested into
  // (s+2)%3 in k step 1). Two x slots: x(s+2) in slot s%2, x(s+3) requested
  // into (s+1)%2 in k step 0; one slot: x(s+2) requested in k step 0 and
  // stored in the last. Loads past the last stage re-read the last one, so
  // the ring never branches.
  auto step = [&](int s, auto slot) {
    constexpr int S = decltype(slot)::v;
    constexpr int WC = S % 3, WN = (S + 1) % 3, WA = (S + 2) % 3;
    constexpr int XC = S % kXS, XA = (S + 1) % kXS;
    constexpr int BC = S % 3, BN = (S + 1) % 3, BA = (S + 2) % 3;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      if constexpr (!kPrefA) read_a(af, BC, ks);
      if (ks == 0) lx(xs[XA], min(s + kXS + 1, last));
      if (ks == 1) lw(ws[WA], min(s + 2, last));
      h8_t an[4], bn[2];
      if (ks < kBK / 16 - 1) {
        if constexpr (kPrefA) read_a(an, BC, ks + 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) bn[j] = decode_w<QT>(ws[WC], j, ks + 1);
      } else {
        if (s + 2 < stages) sx(xs[XC], BA, s + 2);
        if constexpr (kPrefA) read_a(an, BN, 0);
#pragma unroll
        for (int j = 0; j < 2; ++j) bn[j] = decode_w<QT>(ws[WN], j, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      // each MFMA followed by four VALU (decode) instructions and at most
      // one memory instruction: LDS reads of the next k step, global loads
      // (x in step 0, weights in step 1), the slab store in step 3
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        if (ks == kBK / 16 - 1) {
          if (q < 4) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
          else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);        // LDS read
        } else {
          if (q % 2 == 0) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          if (ks == 0 && q < 4) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
          if (ks == 1 && q < 6) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kPrefA) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = an[i];
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = bn[j];
    }
    __syncthreads();
  };
  int s = 0;
  for (; s + 6 <= stages; s += 6) {
    step(s, Slot<0>{}); step(s + 1, Slot<1>{}); step(s + 2, Slot<2>{});
    step(s + 3, Slot<3>{}); step(s + 4, Slot<4>{}); step(s + 5, Slot<5>{});
  }
  if (s + 2 <= stages) { step(s, Slot<0>{}); step(s + 1, Slot<1>{}); }
  if (s + 4 <= stages) { step(s + 2, Slot<2>{}); step(s + 3, Slot<3>{}); }

  // epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each
  // 32x32 block; first every row is scaled back by 2^-e of its exponent
  // (four consecutive rows per 16-byte LDS read)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int4 e4 = *(const int4*)(sexp + 32 * i + 8 * q + 4 * (lane >> 5));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[i][j][4 * q + 0] = ldexp_f(acc[i][j][4 * q + 0], -e4.x);
        acc[i][j][4 * q + 1] = ldexp_f(acc[i][j][4 * q + 1], -e4.y);
        acc[i][j][4 * q + 2] = ldexp_f(acc[i][j][4 * q + 2], -e4.z);
        acc[i][j][4 * q + 3] = ldexp_f(acc[i][j][4 * q + 3], -e4.w);
      }
    }
  }
  // Stores go through a buffer resource over this workgroup's rows of the
  // output, with one per-lane offset (row lrow, the lane's column) and one
  // scalar offset per row: no per-element branch or 64-bit address
  // arithmetic (that form took ~80 cycles per output, 5 us of a 128 x 256
  // tile's epilogue). The hardware range check covers the sum of both
  // offsets, so rows past m fall past the resource and are dropped, and a
  // lane whose column lies past n (or, under SwiGLU, holds an up row) takes
  // the base offset 2^31, past every resource. All offsets stay below 2^31
  // (the launcher bounds 128 * n * 4).
  constexpr uint32_t kDropped = 0x80000000u;
  const int lrow = 4 * (lane >> 5);  // first output row of this lane's D
  auto row_off = [&](int i, int r, int stride) {  // wave-uniform
    return (uint32_t)((32 * i + 8 * (r >> 2) + (r & 3)) * stride * 4);
  };
  // with several K ranges each writes its own raw partial slice and the
  // reduce applies the epilogue
  if (a.splits > 1) {
    const rsrc_t rp = make_rsrc(a.part + (size_t)sp * a.m * a.n + (size_t)m0 * a.n,
                                (uint32_t)((size_t)rows * a.n * 4));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ncol = tile0 * kTileRows + 64 * wn + 32 * j + fr;
      const uint32_t lo = ncol < a.n ? (uint32_t)((lrow * a.n + ncol) * 4) : kDropped;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          buf_store4(acc[i][j][r], rp, lo, row_off(i, r, a.n));
          // (each offset computed beside its store: scheduled ahead, the row
          // offsets of a block overflow the registers)
          if ((r & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
    }
    return;
  }
  const rsrc_t ry = make_rsrc(a.y + (size_t)m0 * a.ny, (uint32_t)((size_t)rows * a.ny * 4));
  const rsrc_t rr = EXT ? make_rsrc(a.out.residual + (size_t)m0 * a.ny,
                                    (uint32_t)((size_t)rows * a.ny * 4))
                        : ry;
  // one code path per (bias, SwiGLU) choice; the bias depends on the column
  // only, so a lane loads it once per block
  auto store = [&](auto bias_c, auto glu_c) {
    constexpr bool HB = decltype(bias_c)::v, GL = decltype(glu_c)::v;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ncol = tile0 * kTileRows + 64 * wn + 32 * j + fr;
      const float bj = HB ? a.epi.bias[min(ncol, a.n - 1)] : 0.0f;
      const int col = GL ? glu_col(ncol) : ncol;
      const bool live = ncol < a.n && (!GL || (fr & 8) == 0);
      const uint32_t lo = live ? (uint32_t)((lrow * a.ny + col) * 4) : kDropped;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float v = HB ? acc[i][j][r] + bj : acc[i][j][r];
          float o = v;
          if (GL) {
            // the up row of column ncol (ncol % 16 < 8) is in lane ^ 8
            const float u = __shfl_xor(v, 8);
            o = silu_f(v) * u;
          }
          if constexpr (EXT)
            o += __builtin_bit_cast(float, buf_load4(rr, lo, row_off(i, r, a.ny)));
          buf_store4(o, ry, lo, row_off(i, r, a.ny));
          if ((r & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
    }
  };
  const bool hb = a.epi.bias != nullptr;
  if (a.epi.act == kEpiSwiGLU) {
    if (hb) store(Slot<1>{}, Slot<1>{});
    else store(Slot<0>{}, Slot<1>{});
  } else {
    if (hb) store(Slot<1>{}, Slot<0>{});
    else store(Slot<0>{}, Slot<0>{});
  }
}

// y = epilogue(sum of the split-K partial slices, in slice order:
// deterministic). One thread per four consecutive outputs of a row when
// VEC (n % 4 == 0), else per output.
template <bool VEC>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* part, float* y,
                                                           int m, int n, int splits,
                                                           Epilogue epi, int ny, GemmOut go) {
  constexpr int V = VEC ? 4 : 1;
  const size_t o = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (o >= (size_t)m * ny) return;
  const int r = (int)(o / ny), c = (int)(o % ny);
  const size_t count = (size_t)m * n;
  auto sum = [&](int col, float (&s)[V]) {
    const float* p0 = part + (size_t)r * n + col;
    if (VEC) {
      float4 t = *(const float4*)p0;
      for (int p = 1; p < splits; ++p) {
        const float4 v = *(const float4*)(p0 + (size_t)p * count);
        t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
      }
      s[0] = t.x; s[V > 1 ? 1 : 0] = t.y; s[V > 2 ? 2 : 0] = t.z; s[V > 3 ? 3 : 0] = t.w;
    } else {
      float t = p0[0];
      for (int p = 1; p < splits; ++p) t += p0[(size_t)p * count];
      s[0] = t;
    }
  };
  float out[V];
  if (epi.act == kEpiSwiGLU) {
    // output column c -> gate row 16(c/8) + c%8, up row + 8
    const int row = 16 * (c / 8) + c % 8;
    float g[V], u[V];
    sum(row, g);
    sum(row + 8, u);
#pragma unroll
    for (int e = 0; e < V; ++e)
      out[e] = silu_f(add_bias(epi, g[e], row + e)) * add_bias(epi, u[e], row + 8 + e);
  } else {
    float s[V];
    sum(c, s);
#pragma unroll
    for (int e = 0; e < V; ++e) out[e] = add_bias(epi, s[e], c + e);
  }
  if (go.residual != nullptr) {
#pragma unroll
    for (int e = 0; e < V; ++e) out[e] += go.residual[o + e];
  }
  if (VEC) {
    *(float4*)(y + o) = make_float4(out[0], out[V > 1 ? 1 : 0], out[V > 2 ? 2 : 0], out[V > 3 ? 3 : 0]);
  } else {
    y[o] = out[0];
  }
}

template <int QT, bool EXT>
void launch_f16(const GemmArgs& a, unsigned grid, hipStream_t stream) {
  if constexpr (QT == MLQ_Q4_0)
    gemm_kernel<QT, kXF16, 2, 2, EXT><<<grid, kThreads, 0, stream>>>(a);
  else if ((int)grid > device_cus())  // a second workgroup per CU to run
    gemm_kernel<QT, kXF16, 2, 1, EXT><<<grid, kThreads, 0, stream>>>(a);
  else
    gemm_kernel<QT, kXF16, 1, 2, EXT><<<grid, kThreads, 0, stream>>>(a);
}

template <int QT>
hipError_t launch_typed(const GemmArgs& a, int xm, hipStream_t stream) {
  const unsigned grid = (unsigned)(a.mtiles * a.ntiles * a.splits);
  // residual in the GEMM's own store (split K: the reduce adds it); the
  // prefill paths that set it read the fp16 copy
  const bool ext = a.splits == 1 && a.out.residual != nullptr;
  if (ext && xm != kXF16) return hipErrorInvalidValue;
  switch (xm) {
    case kXF32Vec: gemm_kernel<QT, kXF32Vec><<<grid, kThreads, 0, stream>>>(a); break;
    // (element-wise loads: one activation register slot keeps it spill-free)
    case kXF32Scalar: gemm_kernel<QT, kXF32Scalar, 1, 1><<<grid, kThreads, 0, stream>>>(a); break;
    default:
      if (ext) launch_f16<QT, true>(a, grid, stream);
      else launch_f16<QT, false>(a, grid, stream);
      break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  return launch_split_reduce(a.part, a.y, a.m, a.n, a.splits, a.epi, stream, a.out);
}

int g_split_override = 0;  // mlq_set_gemm_split; 0 = planner

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

}  // namespace

// Compute units of the current device (256 on MI355X), read once.
int device_cus() {
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      return 256;
    return n;
  }();
  return cus;
}

hipError_t launch_split_reduce(const float* part, float* y, int m, int n, int splits,
                               const Epilogue& epi, hipStream_t stream, const GemmOut& out) {
  const int ny = epi.act == kEpiSwiGLU ? n / 2 : n;
  const size_t outs = (size_t)m * ny;
  if (n % 4 == 0) {
    const size_t threads = outs / 4;
    split_reduce_kernel<true><<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(
        part, y, m, n, splits, epi, ny, out);
  } else {
    split_reduce_kernel<false><<<(unsigned)((outs + 255) / 256), 256, 0, stream>>>(
        part, y, m, n, splits, epi, ny, out);
  }
  return hipGetLastError();
}

// Row stride (halves) of the fp16 activation copy: whole 128-k groups, so
// every stage (GEMM) and group (skinny GEMM) of a row stays inside it.
int f16_row_stride(int k) { return (k + kGroupK - 1) / kGroupK * kGroupK; }

// the fp16 rows, then the row exponents
size_t f16_copy_bytes(int m, int k) {
  return align256((size_t)m * f16_row_stride(k) * 2) + (size_t)m * sizeof(int);
}

int* f16_copy_exps(void* copy, int m, int k) {
  return (int*)((uint8_t*)copy + align256((size_t)m * f16_row_stride(k) * 2));
}

void set_gemm_split(int split) { g_split_override = split; }

// K ranges per output tile. One workgroup runs per CU (one wave per SIMD)
// and its K loop is serial, so a shape with few tiles (small m, or small n)
// leaves CUs idle for the whole K loop. Splitting K multiplies the
// workgroups; each split then writes an fp32 partial slice that a reduce
// pass sums in order. Cost model (us), fitted to measurements on MI355X:
// a 64-k stage takes 0.66 us for a lone workgroup and 0.0018 us more per
// workgroup running beside it (shared L2 / HBM), ~2 us of prologue and
// epilogue per round of workgroups, partial slices written and read at
// ~4 TB/s, ~2 us for the reduce launch.
int gemm_splits(int m, int n, int k) {
  const int g = (k + kGroupK - 1) / kGroupK;
  if (g_split_override > 0) return std::min(g_split_override, g);
  const int tiles = (m + kBM - 1) / kBM * ((n + kBN - 1) / kBN);
  const int cus = device_cus();
  int best = 1;
  double best_t = 0.0;
  for (int sp = 1; sp <= 16 && sp <= g; ++sp) {
    const int wgs = tiles * sp;
    const int rounds = (wgs + cus - 1) / cus;
    const int stages = 2 * ((g + sp - 1) / sp);
    const double stage_us = 0.66 + 0.0018 * std::min(wgs, cus);
    double t = rounds * (stages * stage_us + 2.0);
    if (sp > 1) t += (2.0 * sp + 1.0) * m * (double)n * 4.0 / 4.0e6 + 2.0;
    if (sp == 1 || t < best_t) { best = sp; best_t = t; }
  }
  return best;
}

size_t gemm_workspace_bytes(int m, int n, int k) {
  const int sp = gemm_splits(m, n, k);
  return align256(f16_copy_bytes(m, k)) + (sp > 1 ? (size_t)sp * m * n * 4 : 0);
}

hipError_t launch_x_to_f16(const float* x, _Float16* xh, int* rexp, int m, int k,
                           hipStream_t stream) {
  RowCopyArgs a{x, xh, rexp, m, k, f16_row_stride(k), 0};
  return launch_row_copy<kCopyRowMajor>(a, m, stream);
}

size_t gemm_partial_bytes(int m, int n, int k) {
  const int sp = gemm_splits(m, n, k);
  return sp > 1 ? (size_t)sp * m * n * 4 : 0;
}

hipError_t launch_gemm_f16(const mlq_weight& w, const _Float16* xh, const int* rexp, float* y,
                           int m, void* ws, size_t ws_bytes, hipStream_t stream,
                           const Epilogue& epi, const GemmOut& out) {
  if (rexp == nullptr) return hipErrorInvalidValue;
  // a workgroup's output rows (and partial slices) are addressed with 32-bit
  // buffer offsets
  if ((size_t)kBM * (size_t)w.n * 4 >= (1ull << 31)) return hipErrorInvalidValue;
  const Geometry geo = geometry(w.n, w.k);
  GemmArgs a;
  a.qs = (const uint8_t*)w.base + w.qs_off;
  a.d = (const uint8_t*)w.base + w.d_off;
  a.mn = w.type == MLQ_Q4_1 ? (const uint8_t*)w.base + w.m_off : nullptr;
  a.x = nullptr;
  a.xh = xh;
  a.rexp = rexp;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.k = w.k;
  a.g = geo.g;
  a.nt = geo.nt;
  a.kp = f16_row_stride(w.k);
  a.mtiles = (m + kBM - 1) / kBM;
  a.ntiles = (geo.nt + kTiles - 1) / kTiles;
  a.splits = 1;
  a.part = nullptr;
  a.epi = epi;
  a.out = out;
  a.ny = epi.act == kEpiSwiGLU ? w.n / 2 : w.n;
  const int sp = gemm_splits(m, w.n, w.k);
  if (sp > 1 && ws != nullptr && ws_bytes >= gemm_partial_bytes(m, w.n, w.k)) {
    a.splits = sp;
    a.part = (float*)ws;
  }
  switch (w.type) {
    case MLQ_Q8_0: return launch_typed<MLQ_Q8_0>(a, kXF16, stream);
    case MLQ_Q4_0: return launch_typed<MLQ_Q4_0>(a, kXF16, stream);
    default: return launch_typed<MLQ_Q4_1>(a, kXF16, stream);
  }
}

hipError_t launch_gemm(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream) {
  return launch_gemm_ws(w, x, y, m, nullptr, 0, stream);
}

hipError_t launch_gemm_ws(const mlq_weight& w, const float* x, float* y, int m,
                          void* ws, size_t ws_bytes, hipStream_t stream,
                          const Epilogue& epi, const GemmOut& out) {
  const Geometry geo = geometry(w.n, w.k);
  GemmArgs a;
  a.qs = (const uint8_t*)w.base + w.qs_off;
  a.d = (const uint8_t*)w.base + w.d_off;
  a.mn = w.type == MLQ_Q4_1 ? (const uint8_t*)w.base + w.m_off : nullptr;
  a.x = x;
  a.xh = nullptr;
  a.rexp = nullptr;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.k = w.k;
  a.g = geo.g;
  a.nt = geo.nt;
  a.kp = f16_row_stride(w.k);
  a.mtiles = (m + kBM - 1) / kBM;
  a.ntiles = (geo.nt + kTiles - 1) / kTiles;
  a.splits = 1;
  a.part = nullptr;
  a.epi = epi;
  a.out = out;
  a.ny = epi.act == kEpiSwiGLU ? w.n / 2 : w.n;
  // every activation row offset and output row offset of a workgroup must
  // fit a 32-bit buffer offset
  if ((size_t)kBM * (size_t)w.k * 4 >= (1ull << 31) ||
      (size_t)kBM * (size_t)w.n * 4 >= (1ull << 31))
    return hipErrorInvalidValue;
  int xm = (w.k & 3) == 0 ? kXF32Vec : kXF32Scalar;
  if (ws != nullptr && ws_bytes >= f16_copy_bytes(m, w.k)) {
    // one pass over x: fp16 copy, row stride kp, zero tail, row exponents
    a.xh = (_Float16*)ws;
    a.rexp = f16_copy_exps(ws, m, w.k);
    const hipError_t e = launch_x_to_f16(x, (_Float16*)ws, f16_copy_exps(ws, m, w.k), m, w.k,
                                         stream);
    if (e != hipSuccess) return e;
    xm = kXF16;
    // split K when the workspace also holds the partial slices
    const int sp = gemm_splits(m, w.n, w.k);
    if (sp > 1 && ws_bytes >= gemm_workspace_bytes(m, w.n, w.k)) {
      a.splits = sp;
      a.part = (float*)((uint8_t*)ws + align256(f16_copy_bytes(m, w.k)));
    }
  }
  switch (w.type) {
    case MLQ_Q8_0: return launch_typed<MLQ_Q8_0>(a, xm, stream);
    case MLQ_Q4_0: return launch_typed<MLQ_Q4_0>(a, xm, stream);
    default: return launch_typed<MLQ_Q4_1>(a, xm, stream);
  }
}

}  // namespace mlq
