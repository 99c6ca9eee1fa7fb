// Prefill / batched GEMM on gfx950 MFMA: y[m, n] = sum_k W[n, k] x[m, k].
//
// The reference never issues m > 1 on the GPU (src/batch.cc:32-55 loops
// tokens); its kernels (src/cuda_quant.cu:78-182) re-stream W once per row
// of x (grid.y = rows). This kernel is a dense contraction instead:
//  - Workgroup tile 128 (m) x 128 (n), four waves in a 2 x 2 grid, each wave
//    64 x 64 = 2 x 2 v_mfma_f32_32x32x16_f16 (fp32 accumulate). The 32x32
//    shape does twice the work per operand register of 16x16x32, which
//    halves the LDS read traffic per flop.
//  - K advances in stages of 64 (half of a 128-k group). Each stage's
//    activations (fp32 -> fp16) and weights (codes decoded exactly, then
//    scaled by d in fp16: one rounding, like d*q rounded to fp16) are
//    written to LDS in row-major [row][k] slabs with a 16-byte row pad, so
//    every MFMA operand is one conflict-free ds_read_b128.
//  - Two LDS buffers and two register stages: while the waves run stage s
//    from one LDS buffer, stage s+1 (requested a stage earlier) is converted
//    from registers into the other, and stage s+2 is being fetched; one
//    barrier per stage.
//  - 72 KiB of LDS and <= 256 VGPRs per lane, so two workgroups share a CU and one's
//    decode work overlaps the other's MFMAs.
//  - Workgroups are numbered XCD-major: the four m-tiles of one weight
//    column block run on the same XCD and share its L2.
// The scale is applied before the MFMA (per weight), so no per-block fixup
// of the accumulators is needed; that is what keeps VALU work independent of
// m (an int8 MFMA variant would need a per-(m, n, block) fp32 fixup).
#include <hip/hip_runtime.h>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kBM = 128;           // x rows per workgroup
constexpr int kBN = 128;           // W rows per workgroup (8 row tiles)
constexpr int kBK = 64;            // k per stage
constexpr int kTiles = kBN / kTileRows;
constexpr int kThreads = 256;
constexpr int kStride = kBK + 8;   // halves per LDS row (144 B)
constexpr int kXcds = 8;

typedef float f16v_t __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const uint8_t* qs;
  const uint8_t* d;
  const uint8_t* mn;
  const float* x;
  float* y;
  int m, n, k, g, nt;
  int mtiles, ntiles;  // workgroup grid
};

// Registers holding one stage of global data for this thread.
template <int QT>
struct Stage {
  float4 xa[8];   // activations: rows t/16 + 16j, k 4*(t%16) .. +3
  uint4 q[2];     // weight chunks (q8: 16 B; q4: 8 B in .x/.y)
  uint32_t dd[2]; // two fp16 scales (blocks 2h, 2h+1) per chunk
  uint32_t mm[2]; // two fp16 mins (q4_1)
};

__device__ __forceinline__ h2_t h2_splat(uint32_t bits16) {
  const _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (h2_t){v, v};
}

// VEC: k % 4 == 0, so activation rows are 16-byte aligned and a float4 is
// either wholly inside the range or wholly past it. Otherwise each element
// is loaded (and range-checked) on its own. A compile-time choice: a runtime
// branch around the loads makes the compiler wait for each load in turn.
template <int QT, bool VEC>
__device__ __forceinline__ void load_stage(const GemmArgs& a, Stage<QT>& st,
                                           rsrc_t rx, rsrc_t rq, rsrc_t rd,
                                           rsrc_t rm, int s, int tid) {
  const int k0 = s * kBK;
  // activations: 8 float4 per thread (zeros past the last row via the range)
  const int c = tid & 15;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = (tid >> 4) + 16 * j;
    const uint32_t off = (uint32_t)((r * a.k + k0 + 4 * c) * 4);
    if (VEC) {
      st.xa[j] = __builtin_bit_cast(float4, buf_load16(rx, off, 0));
    } else {
      st.xa[j].x = __builtin_bit_cast(float, buf_load4(rx, off, 0));
      st.xa[j].y = __builtin_bit_cast(float, buf_load4(rx, off + 4, 0));
      st.xa[j].z = __builtin_bit_cast(float, buf_load4(rx, off + 8, 0));
      st.xa[j].w = __builtin_bit_cast(float, buf_load4(rx, off + 12, 0));
    }
  }
  // weights: half-group h of group gi for 8 row tiles, two chunks per thread
  const int gi = s >> 1, h = s & 1;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int wt = (tid >> 6) + 4 * j;  // row tile within the workgroup
    const int lane = tid & 63;
    const uint32_t unit = (uint32_t)(wt * a.g + gi);
    if (QT == MLQ_Q8_0) {
      st.q[j] = buf_load16(rq, ((unit * 2 + h) * 64 + lane) * 16, 0);
    } else {
      const uint2 v = buf_load8(rq, (unit * 64 + lane) * 16 + 8 * h, 0);
      st.q[j] = make_uint4(v.x, v.y, 0, 0);
    }
    const uint32_t soff = ((unit * kTileRows + (lane & 15)) * 4 + 2 * h) * 2;
    st.dd[j] = buf_load4(rd, soff, 0);
    if (QT == MLQ_Q4_1) st.mm[j] = buf_load4(rm, soff, 0);
  }
}

// Converts a stage held in registers into LDS (fp16 activations, fp16
// pre-scaled weights).
template <int QT>
__device__ __forceinline__ void store_stage(const GemmArgs& a, Stage<QT>& st,
                                            _Float16* as, _Float16* bs, int s,
                                            int tid) {
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
    uint2 hv;
    hv.x = pack_h2(st.xa[j].x, st.xa[j].y);
    hv.y = pack_h2(st.xa[j].z, st.xa[j].w);
    *(uint2*)(as + r * kStride + 4 * c) = hv;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int wt = (tid >> 6) + 4 * j;
    const int lane = tid & 63;
    const int n = wt * kTileRows + (lane & 15), kq = lane >> 4;
    const h2_t d0 = h2_splat(st.dd[j] & 0xffffu), d1 = h2_splat(st.dd[j] >> 16);
    uint4 o0, o1;  // block 2h (k 8kq..), block 2h+1 (k 32+8kq..)
    if (QT == MLQ_Q8_0) {
      const h2_t b = {(_Float16)1152.0f, (_Float16)1152.0f};
      uint32_t p[8];
      q8_pairs(st.q[j].x, p[0], p[1]);
      q8_pairs(st.q[j].y, p[2], p[3]);
      q8_pairs(st.q[j].z, p[4], p[5]);
      q8_pairs(st.q[j].w, p[6], p[7]);
      o0.x = as_u32((as_h2(p[0]) - b) * d0);
      o0.y = as_u32((as_h2(p[1]) - b) * d0);
      o0.z = as_u32((as_h2(p[2]) - b) * d0);
      o0.w = as_u32((as_h2(p[3]) - b) * d0);
      o1.x = as_u32((as_h2(p[4]) - b) * d1);
      o1.y = as_u32((as_h2(p[5]) - b) * d1);
      o1.z = as_u32((as_h2(p[6]) - b) * d1);
      o1.w = as_u32((as_h2(p[7]) - b) * d1);
    } else {
      const float lo = QT == MLQ_Q4_0 ? 1032.0f : 1024.0f;
      const float hi = QT == MLQ_Q4_0 ? 72.0f : 64.0f;
      const h2_t blo = {(_Float16)lo, (_Float16)lo};
      const h2_t bhi = {(_Float16)hi, (_Float16)hi};
      const Q4Pairs p = q4_pairs(st.q[j].x);
      const Q4Pairs r = q4_pairs(st.q[j].y);
      if (QT == MLQ_Q4_0) {
        o0.x = as_u32((as_h2(p.p0) - blo) * d0);
        o0.y = as_u32((as_h2(p.p1) - bhi) * d0);
        o0.z = as_u32((as_h2(p.p2) - blo) * d0);
        o0.w = as_u32((as_h2(p.p3) - bhi) * d0);
        o1.x = as_u32((as_h2(r.p0) - blo) * d1);
        o1.y = as_u32((as_h2(r.p1) - bhi) * d1);
        o1.z = as_u32((as_h2(r.p2) - blo) * d1);
        o1.w = as_u32((as_h2(r.p3) - bhi) * d1);
      } else {
        const h2_t m0 = h2_splat(st.mm[j] & 0xffffu), m1 = h2_splat(st.mm[j] >> 16);
        o0.x = as_u32(__builtin_elementwise_fma(as_h2(p.p0) - blo, d0, m0));
        o0.y = as_u32(__builtin_elementwise_fma(as_h2(p.p1) - bhi, d0, m0));
        o0.z = as_u32(__builtin_elementwise_fma(as_h2(p.p2) - blo, d0, m0));
        o0.w = as_u32(__builtin_elementwise_fma(as_h2(p.p3) - bhi, d0, m0));
        o1.x = as_u32(__builtin_elementwise_fma(as_h2(r.p0) - blo, d1, m1));
        o1.y = as_u32(__builtin_elementwise_fma(as_h2(r.p1) - bhi, d1, m1));
        o1.z = as_u32(__builtin_elementwise_fma(as_h2(r.p2) - blo, d1, m1));
        o1.w = as_u32(__builtin_elementwise_fma(as_h2(r.p3) - bhi, d1, m1));
      }
    }
    *(uint4*)(bs + n * kStride + 8 * kq) = o0;
    *(uint4*)(bs + n * kStride + 32 + 8 * kq) = o1;
  }
}

template <int QT, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(GemmArgs a) {
  __shared__ __align__(16) _Float16 as_buf[2][kBM * kStride];
  __shared__ __align__(16) _Float16 bs_buf[2][kBN * kStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // XCD-major numbering: hardware sends workgroup b to XCD b % 8; remap so
  // that each XCD gets a contiguous run of logical ids (m fastest).
  const int nwg = a.mtiles * a.ntiles;
  const int b = blockIdx.x;
  const int full = nwg / kXcds * kXcds;
  const int id = b < full ? (b % kXcds) * (full / kXcds) + b / kXcds : b;
  const int mt = id % a.mtiles, ntile = id / a.mtiles;
  const int m0 = mt * kBM;
  const int tile0 = ntile * kTiles;  // first W row tile

  // buffer ranges: rows past m / tiles past nt read as zero
  const rsrc_t rx = make_rsrc(a.x + (size_t)m0 * a.k,
                              (uint32_t)((size_t)min(kBM, a.m - m0) * a.k * 4));
  const int tiles = min(kTiles, a.nt - tile0);
  const uint32_t qbytes = (uint32_t)tiles * a.g * (QT == MLQ_Q8_0 ? 2048u : 1024u);
  const rsrc_t rq = make_rsrc(a.qs + (size_t)tile0 * a.g * (QT == MLQ_Q8_0 ? 2048 : 1024), qbytes);
  const uint32_t sbytes = (uint32_t)tiles * a.g * 128u;
  const rsrc_t rd = make_rsrc(a.d + (size_t)tile0 * a.g * 128, sbytes);
  const rsrc_t rm = QT == MLQ_Q4_1 ? make_rsrc(a.mn + (size_t)tile0 * a.g * 128, sbytes) : rd;

  f16v_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int stages = a.g * 2;
  // Two register stages in flight: stage s+2 is requested while stage s runs
  // on the MFMAs and stage s+1 (requested one stage earlier) is converted
  // into LDS, so each load has two stages of work to arrive.
  Stage<QT> st[2];
  load_stage<QT, VEC>(a, st[0], rx, rq, rd, rm, 0, tid);
  if (stages > 1) load_stage<QT, VEC>(a, st[1], rx, rq, rd, rm, 1, tid);
  store_stage<QT>(a, st[0], as_buf[0], bs_buf[0], 0, tid);
  __syncthreads();

  // fragment rows of this lane: MFMA operand row/col = lane % 32, k octet
  // = lane / 32
  const int fr = lane & 31, fk = 8 * (lane >> 5);
  auto mfma_stage = [&](int cur) {
    const _Float16* as = as_buf[cur];
    const _Float16* bs = bs_buf[cur];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      h8_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *(const h8_t*)(as + (64 * wm + 32 * i + fr) * kStride + 16 * ks + fk);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *(const h8_t*)(bs + (64 * wn + 32 * j + fr) * kStride + 16 * ks + fk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };
  // one stage: register buffer `rb` holds stage s+1 on entry and receives
  // stage s+2
  auto step = [&](int s, Stage<QT>& next, Stage<QT>& after) {
    const int cur = s & 1;
    if (s + 2 < stages) load_stage<QT, VEC>(a, after, rx, rq, rd, rm, s + 2, tid);
    mfma_stage(cur);
    if (s + 1 < stages) store_stage<QT>(a, next, as_buf[cur ^ 1], bs_buf[cur ^ 1], s + 1, tid);
    __syncthreads();
  };
  int s = 0;
  for (; s + 1 < stages; s += 2) {
    step(s, st[1], st[0]);
    step(s + 1, st[0], st[1]);
  }
  if (s < stages) step(s, st[1], st[0]);

  // epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each
  // 32x32 block
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ncol = tile0 * kTileRows + 64 * wn + 32 * j + fr;
      if (ncol >= a.n) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int mrow = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (mrow < a.m) a.y[(size_t)mrow * a.n + ncol] = acc[i][j][r];
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
  a.d = (const uint8_t*)w.base + w.d_off;
  a.mn = w.type == MLQ_Q4_1 ? (const uint8_t*)w.base + w.m_off : nullptr;
  a.x = x;
  a.y = y;
  a.m = m;
  a.n = w.n;
  a.k = w.k;
  a.g = geo.g;
  a.nt = geo.nt;
  a.mtiles = (m + kBM - 1) / kBM;
  a.ntiles = (geo.nt + kTiles - 1) / kTiles;
  // every activation row offset of a workgroup must fit a 32-bit buffer
  // offset
  if ((size_t)kBM * (size_t)w.k * 4 >= (1ull << 31)) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)(a.mtiles * a.ntiles);
  const bool vec = (w.k & 3) == 0;
  switch (w.type) {
    case MLQ_Q8_0:
      if (vec) gemm_kernel<MLQ_Q8_0, true><<<grid, kThreads, 0, stream>>>(a);
      else gemm_kernel<MLQ_Q8_0, false><<<grid, kThreads, 0, stream>>>(a);
      break;
    case MLQ_Q4_0:
      if (vec) gemm_kernel<MLQ_Q4_0, true><<<grid, kThreads, 0, stream>>>(a);
      else gemm_kernel<MLQ_Q4_0, false><<<grid, kThreads, 0, stream>>>(a);
      break;
    default:
      if (vec) gemm_kernel<MLQ_Q4_1, true><<<grid, kThreads, 0, stream>>>(a);
      else gemm_kernel<MLQ_Q4_1, false><<<grid, kThreads, 0, stream>>>(a);
      break;
  }
  return hipGetLastError();
}

}  // namespace mlq
