// Decode GEMV / skinny GEMM for gfx950: y[m, n] = sum_k W[n, k] x[m, k] for
// m = 1..8 activation rows.
//
// Replaces q80LinearKernel / q40LinearKernel / q41LinearKernel
// (src/cuda_quant.cu:78-182) for decode-sized m. The kernel is held to the
// HBM roofline, so its structure follows where the bytes and the VALU issue
// slots go:
//  - A workgroup owns one 16-row tile; its S waves (S = 1..16) split the
//    tile's K range into contiguous slices of `gw` 128-k groups. Per group a
//    wave reads one contiguous 1 KiB (q4) / 2 KiB (q8) line with a dwordx4
//    per lane plus an 8-byte scale load; every weight byte is read from HBM
//    exactly once.
//  - All loads go through buffer resources built per wave (scalar base +
//    byte range), so addresses are one VGPR offset per lane plus a scalar
//    offset per group, and anything past the wave's range (ragged K tails,
//    the groups of a shorter last slice) reads as zero with no branches.
//  - Order of issue: the wave's activation slice first, then the weight
//    lines of its first two groups (GW = groups per wave, a compile-time
//    1..10), then the fp32 -> fp16 hi/lo conversion of the activations into
//    the wave's private LDS slice, then the remaining weight lines. All
//    waves start within ~0.5 us and the activation lines miss L2: issued
//    behind every weight line of the slice they queue behind tens of MB of
//    weight requests (measured: half the waves of the 4096 x 14336 q4_1
//    GEMV staged x only after 5 us with all groups first). Two groups ahead
//    keep HBM busy during the activation fetch without that queueing: 1-3 %
//    faster than all groups first at 4 groups per wave, and faster than no
//    group ahead at every depth (4096 x 14336 q4_1 10.03 -> 9.85 us,
//    3584 x 18944 q4_0 10.75 -> 10.35, the decode step 1459 -> 1415 us).
//    Ring slices stage x before any weight load.
//  - Grids of about one workgroup per CU also hold every weight load until
//    all waves of the workgroup have issued their activation loads (one
//    s_barrier, no wait): the later waves' activation lines then no longer
//    queue behind the earlier waves' first groups (4096 x 4096 q4_0 at
//    M = 4 5.16 -> 4.82 us, the 7B q|k|v 5.03 -> 4.87). Grids of several
//    rounds (the 1184-tile 18944 x 3584 GEMV 8.80 -> 8.92 us with it) and
//    q8_0 at one row, whose activations are a small part of a wave's reads
//    (4096 x 4096 4.93 -> 4.99), run without this barrier. With one
//    activation row the one-round grids then issue one group ahead instead
//    of two (q|k|v 4.96 -> 4.72 us, 4096 x 14336 q4_1 9.77 -> 9.44, the
//    down projection 9.54 -> 9.31; M = 4 keeps two: 4.74 vs 4.96).
//  - The group loop has no data-dependent branch: a shorter last slice
//    processes zero groups (zero scales, zero activations). Slices longer
//    than the register budget run a ring of GW slots instead (GW chosen to
//    pad the slice least), each refilled GW groups ahead as soon as its
//    codes are decoded (refills past the slice read zeros, so they need no
//    branch either).
//  - Lane L = n + 16*kq holds quarter kq of the group's 4 blocks of row n,
//    which is the B operand of v_mfma_f32_16x16x32_f16 for one block. Codes
//    are decoded EXACTLY to fp16 (q-8, q, or q): one AND-OR places a code in
//    the mantissa of 1024 (or 64), one packed fp16 subtract removes the bias.
//  - MFMA row 2r is the fp16 hi part, row 2r+1 the lo part of activation row
//    r (x = hi + lo to ~2^-22): up to 8 rows in one MFMA. Per block:
//    acc += d * (D[hi] + D[lo]) in fp32. Products are exact in fp32, so the
//    result is fp32-class accurate.
//  - q4_1's min term sum_b m_b * sum(x over block b) is one more MFMA per
//    group: A = the group's four block sums (staged in LDS as fp16 hi/lo
//    rows, like x), B = the four fp16 mins of the lane's row (exact), K
//    positions 4..31 zero. Done on the VALU (a float4 of block sums, four
//    converts and FMAs per group) it held ~60 more registers at depth 6,
//    which capped how many groups a wave keeps in flight.
//  - K slices combine through LDS in slice order (deterministic).
//  - Any finite fp32 activations: each wave stages its slice of each row as
//    x * 2^e (e = 0 when the row's largest |x| in the slice lies in
//    [2^-10, 2^15), else the power of two that puts it in [2^14, 2^15)), and
//    scales the row's results by 2^-e before the slices combine (exact
//    power-of-two steps).
//  - One activation row with at most 8 groups per wave, all in flight
//    (every decode projection but the 18944-deep down projection, and
//    c0-c2) runs integer digits instead (DIG): the slice is staged as X = round(x * 2^e) with e
//    from the slice's largest |x| (|X| <= 2^22), three base-256 digits per
//    element as fp16 integers; the codes keep their fp16 bias (1024 + q or
//    64 + q: no subtracts), and per group one chain of five MFMAs (every
//    digit row against -bias, then each block's rows against its codes) is
//    exact because every product and partial sum is an integer below 2^24.
//    The lane quarters then hold block kq's three digit sums: two FMAs
//    combine them, one applies the block's scale (the q4_1 min term is one
//    more FMA with the staged block sum). Per group ~25 VALU instead of
//    ~55: 4096 x 14336 q4_1 9.48 -> 8.88 us, the 7B q|k|v 4.70 -> 4.52,
//    gate|up 14.8 -> 14.4, the decode step 1384 -> 1372 us; ten-group slices
//    (the down projection) measured no faster with it and keep hi/lo pairs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <set>
#include <type_traits>
#include <utility>

#include "../mlq_layout.h"
#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kMaxSplit = 16;       // waves per workgroup (one tile)
constexpr int kTargetWaves = 8192;  // ~32 waves per CU on 256 CUs (measured best)
constexpr int kRowPadHalves = 32;   // 64 B: consecutive LDS rows hit other banks
constexpr int kUnitScaleBytes = kTileRows * kGroupBlocks * 2;  // 128 B
constexpr int kXRegs = 4;           // float4 activation loads held per lane

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
  const uint8_t* d;
  const uint8_t* mn;
  const float* x;
  float* y;
  int m, n, k, g, nt;
  int split;     // waves per workgroup = K slices of its tile
  int gw;        // groups per wave (the last slice may be shorter)
  int xstride;   // fp16 elements per staged activation row
  int wave_lds;  // bytes of LDS per wave (activation slice + block sums)
  Epilogue epi;
  int ny;        // output columns: n, or n/2 under kEpiSwiGLU
  int xbar;      // 1: weight loads wait until every wave issued its activation loads
};

template <int QT>
constexpr uint32_t unit_quant_bytes() {
  return QT == MLQ_Q8_0 ? 2048u : 1024u;
}

template <int QT>
struct Slot {
  uint4 q;
  uint4 q2;  // second 16-byte line (q8_0)
  uint2 d;   // four fp16 scales of the group's blocks
  uint2 m;   // four fp16 mins (q4_1)
};

struct WaveRsrc {
  rsrc_t q, d, m;
};

// Loads group j of the wave's slice (zeros when j is past the slice).
template <int QT>
__device__ __forceinline__ void load_group(const WaveRsrc& r, Slot<QT>& s,
                                           int j, uint32_t qoff, uint32_t soff) {
  const uint32_t qb = (uint32_t)j * unit_quant_bytes<QT>();
  s.q = buf_load16_stream(r.q, qoff, qb);
  if (QT == MLQ_Q8_0) s.q2 = buf_load16_stream(r.q, qoff, qb + 1024u);
  s.d = buf_load8(r.d, soff, (uint32_t)j * kUnitScaleBytes);
  if (QT == MLQ_Q4_1) s.m = buf_load8(r.m, soff, (uint32_t)j * kUnitScaleBytes);
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

__device__ __forceinline__ _Float16 half_at(uint2 s, int j) {
  const uint32_t w = (j & 2) ? s.y : s.x;
  return __builtin_bit_cast(_Float16,
                            (uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu)));
}

// Four activations x[row][4c .. 4c+3] of the slice (zeros past the range).
// vec: the range is a whole number of float4 (k % 4 == 0); otherwise every
// element is range-checked on its own.
__device__ __forceinline__ float4 load_x4(rsrc_t r, int c, bool vec) {
  if (vec) return __builtin_bit_cast(float4, buf_load16(r, (uint32_t)c * 16u, 0));
  float4 v;
  v.x = __builtin_bit_cast(float, buf_load4(r, (uint32_t)c * 16u, 0));
  v.y = __builtin_bit_cast(float, buf_load4(r, (uint32_t)c * 16u + 4u, 0));
  v.z = __builtin_bit_cast(float, buf_load4(r, (uint32_t)c * 16u + 8u, 0));
  v.w = __builtin_bit_cast(float, buf_load4(r, (uint32_t)c * 16u + 12u, 0));
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

// hi/lo split of four activations, scaled by 2^e, written at column kl of
// rows 2r and 2r+1 of the wave's slice; returns their scaled fp32 sum (q4_1
// block sums).
__device__ __forceinline__ float stage4(_Float16* xs, int xstride, int r,
                                        int kl, float4 v, int e) {
  v.x = ldexp_f(v.x, e);
  v.y = ldexp_f(v.y, e);
  v.z = ldexp_f(v.z, e);
  v.w = ldexp_f(v.w, e);
  uint2 hi, lo;
  split2(v.x, v.y, hi.x, lo.x);
  split2(v.z, v.w, hi.y, lo.y);
  *(uint2*)(xs + (size_t)(2 * r) * xstride + kl) = hi;
  *(uint2*)(xs + (size_t)(2 * r + 1) * xstride + kl) = lo;
  return (v.x + v.y) + (v.z + v.w);
}

// ---- one activation row: integer digits ------------------------------------
// Per 128-k group of its slice a wave stages the MFMA A operand of four
// chained MFMAs (one per block) in a record of kDigRec bytes: A row 4b + i
// holds digit i of the scaled activations of block b, as fp16 integers, for
// the lane quarter's 8 elements; rows 4b + 3 are zero (one shared 16-byte zero
// slot at kDigZero). Slot (b, i, kq) sits at ((3b + i) * 4 + kq) * 16.
constexpr int kDigRec = 784;
constexpr int kDigZero = 768;
constexpr int kDigMaxDepth = 8;

// Stages float4 c of the slice (elements 4c .. 4c+3; |v * s| <= 2^22) as
// X = round(v * s) = d0 + 256 d1 + 65536 d2 with d0, d1 in [-128, 127] and
// |d2| <= 64, each digit an fp16 integer, into the record of group c / 32.
// Returns the sum of the four X (q4_1 block sums), exact, as an integer.
__device__ __forceinline__ int stage_dig4(unsigned char* rec, int c, float4 v, float s) {
  // v * s + 1.5 * 2^23 rounds v * s to an integer X once (fma: one rounding)
  // and leaves bits = 0x4B400000 + X; adding 0x19408080 turns that into
  // X + 0x808080 (bytes 0..2: the digits + 128) with 0x64 in byte 3, so one
  // byte permute builds two fp16 values 1024 + digit + 128.
  constexpr float kRound = 12582912.0f;
  const float f0 = fmaf(v.x, s, kRound), f1 = fmaf(v.y, s, kRound);
  const float f2 = fmaf(v.z, s, kRound), f3 = fmaf(v.w, s, kRound);
  const uint32_t u0 = __builtin_bit_cast(uint32_t, f0) + 0x19408080u;
  const uint32_t u1 = __builtin_bit_cast(uint32_t, f1) + 0x19408080u;
  const uint32_t u2 = __builtin_bit_cast(uint32_t, f2) + 0x19408080u;
  const uint32_t u3 = __builtin_bit_cast(uint32_t, f3) + 0x19408080u;
  const h2_t bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  unsigned char* group = rec + (size_t)(c >> 5) * kDigRec;
  unsigned char* slot = group + ((((c >> 3) & 3) * 12 + ((c >> 1) & 3)) * 16 + (c & 1) * 8);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    // bytes [i of the first, 0x64, i of the second, 0x64]
    const uint32_t sel = (uint32_t)i | 0x0300u | ((uint32_t)(4 + i) << 16) | 0x07000000u;
    uint2 w;
    w.x = as_u32(as_h2(__builtin_amdgcn_perm(u1, u0, sel)) + bias);
    w.y = as_u32(as_h2(__builtin_amdgcn_perm(u3, u2, sel)) + bias);
    *(uint2*)(slot + i * 64) = w;
  }
  if ((c & 31) == 0) *(uint4*)(group + kDigZero) = make_uint4(0u, 0u, 0u, 0u);
  // the sum of u = X + 0x64808080 over the four, less 4 * 0x64808080
  // (mod 2^32; integer adds instead of four subtracts and three fp32 adds)
  return (int)(u0 + u1 + u2 + u3 - 0x92020200u);
}

// Sum over each 8-lane group (one block of float4s) of integers: DPP within
// quads, then row_half_mirror pairs the two quads (no LDS round trips,
// unlike shuffles: 4096 x 14336 q4_1 8.93 -> 8.46 us together with the
// integer sums above).
__device__ __forceinline__ int block_sum8_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  return v;
}

// Largest |x| of four activations, NaN propagating (v_maximum3_f32).
__device__ __forceinline__ float abs_maximum4(float m, float4 v) {
  m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(fabsf(v.x), fabsf(v.y)));
  return __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(fabsf(v.z), fabsf(v.w)));
}

// Sum of 8 consecutive lanes' values (one 32-element block = 8 float4):
// quad sums, then the two quads' sums (DPP; the same pairs as xor 1, 2, 4).
__device__ __forceinline__ float block_sum8(float v) { return row_sum<8>(v); }

// VEC: k % 4 == 0 (activation rows in whole float4). A compile-time choice:
// a runtime branch around the activation loads makes the compiler wait for
// all of them before the weight loads are issued.
// Producer side of a pre-scaled RMSNorm input: lanes 0..15 hold the
// tile's outputs v (0 elsewhere); writes v * next_norm to next_x and the
// tile's sum of v^2 (a fixed tree over the 16 lanes) to next_ssq[tile].
// Called by a whole wave.
// g: next_norm of the lane's row (lanes 0..15).
__device__ __forceinline__ void produce_norm_input(const GemvArgs& a, int tile, int lane,
                                                   float v, float g) {
  const float sq = row_sum<16>(v * v);
  const int row = tile * kTileRows + lane;
  if (lane < kTileRows && row < a.n) a.epi.next_x[row] = v * g;
  if (lane == 0) a.epi.next_ssq[tile] = sq;
}

// NM: input RMSNorm mode (one activation row): 0 none, 1 folded (the norm
// weight is loaded beside x and sum(x^2) taken from the staged values), 2
// pre-scaled (x holds x * norm, sum(x^2) comes from the producer's parts).
// PB: a bias (or residual) is given and requested before the slices
// combine (one activation row, NM 0 or 2: the decode step's projections);
// otherwise any bias is read at the end.
template <int QT, int MR, int GW, bool RING, int NM, bool VEC, bool PB>
__global__ __launch_bounds__(1024) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int M = a.m;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // = K slice
  const int tile = blockIdx.x;
  const int g0 = wave * a.gw;
  const int ng = min(a.gw, a.g - g0);  // >= 1 (the planner guarantees it)
  // groups processed: a whole number of ring passes (zero groups past ng)
  const int nch = RING ? (ng + GW - 1) / GW : 1;
  const int npad = nch * GW;
  const int n = lane & 15;   // W row within the tile (and MFMA A row)
  const int kq = lane >> 4;  // quarter of each block (and D row group)

  unsigned char* wl = smem + (size_t)wave * a.wave_lds;
  _Float16* xs = (_Float16*)wl;
  // q4_1 block sums, per group the MFMA A operand: 16 rows (hi/lo of each
  // activation row) x 4 halves (the group's blocks)
  _Float16* xsa = (_Float16*)(wl + (size_t)2 * M * a.xstride * 2);
  float* part = (float*)(smem + (size_t)a.split * a.wave_lds);
  // One activation row, every group of the slice in flight, at most
  // kDigMaxDepth of them (DIG): the digit records of the slice's groups,
  // then (q4_1) four block sums per group. (Ring slices keep the hi/lo
  // pairs: their records would not fit LDS at the longest K.)
  constexpr bool DIG = MR == 1 && GW <= kDigMaxDepth && !RING;
  unsigned char* arec = wl;
  float* ssum = (float*)(wl + (size_t)npad * kDigRec);

  // ---- per-wave buffer ranges --------------------------------------------
  const size_t unit0 = (size_t)tile * a.g + g0;
  WaveRsrc rs;
  rs.q = make_rsrc(a.qs + unit0 * unit_quant_bytes<QT>(),
                   (uint32_t)ng * unit_quant_bytes<QT>());
  rs.d = make_rsrc(a.d + unit0 * kUnitScaleBytes, (uint32_t)ng * kUnitScaleBytes);
  rs.m = rs.d;
  if (QT == MLQ_Q4_1)
    rs.m = make_rsrc(a.mn + unit0 * kUnitScaleBytes, (uint32_t)ng * kUnitScaleBytes);
  const uint32_t qoff = (uint32_t)lane * 16u;
  const uint32_t soff = (uint32_t)n * 8u;

  // ---- activations of the slice: loads first --------------------------------
  // c4 float4 per staged activation row (npad groups); elements past the
  // slice or past k read as zero.
  const int kbase = g0 * kGroupK;
  const int c4 = npad * (kGroupK / 4);
  const uint32_t xbytes = (uint32_t)min(ng * kGroupK, a.k - kbase) * 4u;
  constexpr bool vec = VEC;
  // Register-held part: MR == 1 covers the whole slice of a non-ring wave
  // (one float4 per lane per two groups, at least 4), 8 groups for ring
  // slices; MR > 1 covers one float4 per lane of every row (2 groups). The
  // rest, if any, is read twice more (its maximum, then the staging): each
  // a round trip that every weight load after the staging waits for (the
  // 3584 x 18944 down projection at 10 groups per wave staged at 4.4 us
  // median with 8 groups held, against ~1.3 us for 4-group slices).
  constexpr int XR = MR == 1 ? (!RING && GW > 2 * kXRegs ? (GW + 1) / 2 : kXRegs)
                             : kGemvMaxRows;
  // Input RMSNorm (one row): the norm weight is loaded beside x, the staged
  // values are x * weight and the lanes keep sum(x^2) of their elements.
  // (its register-held part is loaded with x: reading it at staging time
  // instead delays the first MFMA by a round trip, measured slower)
  constexpr bool norm = NM == 1 && MR == 1;
  constexpr bool pre = NM == 2 && MR == 1;
  const rsrc_t rg = make_rsrc(norm ? a.epi.norm + kbase : a.x, norm ? xbytes : 0u);
  float4 xr[XR], gr[norm ? XR : 1];
#pragma unroll
  for (int i = 0; i < XR; ++i) {
    const int r = MR == 1 ? 0 : i;
    const int c = MR == 1 ? lane + 64 * i : lane;
    if (r < M && (MR > 1 || 64 * i < c4)) {  // wave-uniform
      const rsrc_t rx = make_rsrc(a.x + (size_t)r * a.k + kbase, xbytes);
      xr[i] = load_x4(rx, c < c4 ? c : 0x2000000, vec);
      if constexpr (norm) gr[i] = load_x4(rg, c < c4 ? c : 0x2000000, vec);
    }
  }
  // producer of a pre-scaled input: wave 0's lanes 0..15 hold the norm
  // weight of their output row, requested now (not behind the final barrier)
  constexpr bool can_produce = MR == 1 && NM == 0;
  float gnext = 0.0f;
  if (can_produce && a.epi.next_x != nullptr) {  // uniform
    const rsrc_t rn = make_rsrc(a.epi.next_norm + (size_t)tile * kTileRows,
                                wave == 0 ? (uint32_t)min(kTileRows, a.n - tile * kTileRows) * 4u
                                          : 0u);
    gnext = __builtin_bit_cast(float, buf_load4(rn, (uint32_t)(lane & 15) * 4u, 0));
  }
  // pre-scaled input: the producer's partial sums of x^2, requested now and
  // added after the group loop (lane l holds parts 4l .. 4l+3; past
  // ssq_count they read zero). Only wave 0's range is non-empty (the other
  // waves' load moves no data); its scale reaches the workgroup via LDS.
  float4 sp4 = {0.f, 0.f, 0.f, 0.f};
  if constexpr (pre) {
    const rsrc_t rp =
        make_rsrc(a.epi.ssq_parts, wave == 0 ? (uint32_t)a.epi.ssq_count * 4u : 0u);
    sp4 = __builtin_bit_cast(float4, buf_load16(rp, (uint32_t)lane * 16u, 0));
  }
  float ssq = 0.0f;  // this lane's sum of x^2 (norm only)
  auto normed = [&](float4 v, float4 g) {
    ssq += v.x * v.x;
    ssq += v.y * v.y;
    ssq += v.z * v.z;
    ssq += v.w * v.w;
    return float4{v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w};
  };

  // ---- per-row scale of the slice ------------------------------------------
  // Every activation row of the slice is staged as x * 2^e, so any finite
  // fp32 row fits the fp16 hi/lo pair: e = 0 while the row's largest |x| in
  // the slice lies in [2^-10, 2^15), else e from that maximum
  // (pow2_scale_exp). The row's results are scaled back by 2^-e before the
  // slices combine. Values beyond the register-held part are read once more
  // for this maximum.
  constexpr int NR = MR == 1 ? 1 : kGemvMaxRows;
  // Slices longer than the register-held part (MR == 1: ring slices past 8
  // groups; MR > 1: > 2 groups) read the rest once for the maximum and once
  // to stage it.
  const int c_done = MR == 1 ? 64 * XR : 64;
  // this lane's largest |x| of row r in the register-held part
  auto reg_max = [&](int r) __attribute__((always_inline)) {
    float mx = 0.0f;
    if constexpr (MR == 1) {
#pragma unroll
      for (int i = 0; i < XR; ++i)
        if (64 * i < c4 && lane + 64 * i < c4) mx = abs_max4(mx, xr[i]);
    } else {
#pragma unroll
      for (int q = 0; q < NR; ++q)
        if (q == r && lane < c4) mx = abs_max4(mx, xr[q]);
    }
    return mx;
  };
  // ... and in the rest of a long slice (read once more)
  auto rest_max = [&](int r) __attribute__((always_inline)) {
    float mx = 0.0f;
    const rsrc_t rx = make_rsrc(a.x + (size_t)r * a.k + kbase, xbytes);
    for (int cb = c_done; cb < c4; cb += 64) {
      float4 v = load_x4(rx, cb + lane, vec);
      if constexpr (norm) {
        const float4 g = load_x4(rg, cb + lane, vec);
        v = float4{v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w};
      }
      mx = abs_max4(mx, v);
    }
    return mx;
  };
  // ---- stage hi/lo activations (+ q4_1 block sums) -----------------------
  // block sum of row r, block blk (of the slice) -> hi/lo halves at rows
  // 2r, 2r+1 of group blk/4's A operand, stored as sum * 2^-6 (a block of
  // 32 scaled values sums to at most 2^20; the MFMA result is scaled back by
  // 64, exactly)
  auto stage_sum = [&](int r, int blk, float sx) {
    sx = ldexp_f(sx, -6);
    const _Float16 hi = (_Float16)sx;
    const _Float16 lo = (_Float16)(sx - (float)hi);
    _Float16* g = xsa + (size_t)(blk >> 2) * kTileRows * kGroupBlocks + (blk & 3);
    g[(2 * r) * kGroupBlocks] = hi;
    g[(2 * r + 1) * kGroupBlocks] = lo;
  };
  // Stages the slice, every row r scaled by 2^ex[r] (SCALED) or by 1. The
  // unscaled pass also folds the input RMSNorm's sum of squares (once).
  int ex[NR];  // wave-uniform: scalar registers
#pragma unroll
  for (int r = 0; r < NR; ++r) ex[r] = 0;
  auto stage = [&](auto scaled_c) __attribute__((always_inline)) {
    constexpr bool SCALED = decltype(scaled_c)::value;
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      const int r = MR == 1 ? 0 : i;
      const int c = MR == 1 ? lane + 64 * i : lane;
      if (r < M && (MR > 1 || 64 * i < c4)) {  // wave-uniform
        float sx = 0.0f;
        if (c < c4) sx = stage4(xs, a.xstride, r, 4 * c, xr[i], SCALED ? ex[MR == 1 ? 0 : i] : 0);
        if (QT == MLQ_Q4_1) {
          sx = block_sum8(sx);
          if (c < c4 && (c & 7) == 0) stage_sum(r, c >> 3, sx);
        }
      }
    }
    // the rest of long slices
    if (c4 > c_done) {
      // (rows unrolled: a runtime row index into ex[] would put it in
      // scratch memory)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (r >= M) break;  // wave-uniform
        const rsrc_t rx = make_rsrc(a.x + (size_t)r * a.k + kbase, xbytes);
        const int er = ex[r];
        for (int cb = c_done; cb < c4; cb += 64) {
          const int c = cb + lane;
          float sx = 0.0f;
          float4 v = load_x4(rx, c, vec);
          if constexpr (norm) {
            if constexpr (SCALED) {
              const float4 g = load_x4(rg, c, vec);
              v = float4{v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w};
            } else {
              v = normed(v, load_x4(rg, c, vec));
            }
          }
          if (c < c4) sx = stage4(xs, a.xstride, r, 4 * c, v, SCALED ? er : 0);
          if (QT == MLQ_Q4_1) {
            sx = block_sum8(sx);
            if (c < c4 && (c & 7) == 0) stage_sum(r, c >> 3, sx);
          }
        }
      }
    }
  };
  // One activation row (DIG): the slice is staged once as integers
  // X = round(x * 2^e), e from the slice's largest |x| (2^21 <= |X| max
  // < 2^22: 22 bits below the slice's largest element, any finite fp32 x,
  // the exponent moves with power-of-two scalings of x); three digits per
  // element (stage_dig4). A slice holding inf or NaN yields NaN outputs.
  bool nonfin = false;
  auto stage_dig = [&](float s, float pre) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
      const int c = lane + 64 * i;
      if (64 * i < c4) {  // wave-uniform
        int sx = 0;
        if (c < c4) sx = stage_dig4(arec, c, xr[i], s);
        if (QT == MLQ_Q4_1) {
          sx = block_sum8_i(sx);
          if (c < c4 && (c & 7) == 0) ssum[c >> 3] = (float)sx;
        }
      }
    }
    if (c4 > c_done) {
      const rsrc_t rx = make_rsrc(a.x + kbase, xbytes);
      for (int cb = c_done; cb < c4; cb += 64) {
        const int c = cb + lane;
        float4 v = load_x4(rx, c, vec);
        if constexpr (norm) v = normed(v, load_x4(rg, c, vec));
        v = float4{v.x * pre, v.y * pre, v.z * pre, v.w * pre};
        int sx = 0;
        if (c < c4) sx = stage_dig4(arec, c, v, s);
        if (QT == MLQ_Q4_1) {
          sx = block_sum8_i(sx);
          if (c < c4 && (c & 7) == 0) ssum[c >> 3] = (float)sx;
        }
      }
    }
  };
  // Rows whose largest |x| lies in [2^-10, 2^15) (the common case) keep
  // scale 1: hi stays finite and the lo part's fp16 subnormal floor (2^-25)
  // is below 2^-15 of the row's largest element, far inside the stated
  // tolerance. The slice is staged with scale 1 right away while a
  // wave-wide vote checks the window; only when a row falls outside it do
  // the rows pay for their exact maxima (a cross-lane reduction) and a
  // second, scaled staging pass. Returns whether every row kept scale 1
  // (the DIG path, which always scales: false).
  auto stage_slice = [&]() __attribute__((always_inline)) {
    if constexpr (norm) {
#pragma unroll
      for (int i = 0; i < XR; ++i)
        if (64 * i < c4) xr[i] = normed(xr[i], gr[i]);  // wave-uniform
    }
    if constexpr (DIG) {
      float mx = 0.0f;
#pragma unroll
      for (int i = 0; i < XR; ++i)
        if (64 * i < c4 && lane + 64 * i < c4) mx = abs_maximum4(mx, xr[i]);
      if (c4 > c_done) {
        const rsrc_t rx = make_rsrc(a.x + kbase, xbytes);
        for (int cb = c_done; cb < c4; cb += 64) {
          float4 v = load_x4(rx, cb + lane, vec);
          if constexpr (norm) {
            const float4 g = load_x4(rg, cb + lane, vec);
            v = float4{v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w};
          }
          mx = abs_maximum4(mx, v);
        }
      }
      mx = wave_max_nonneg(mx);  // NaN sorts above inf
      nonfin = !(mx <= 3.402823466e38f);
      int e = nonfin ? 0 : 22 - __builtin_amdgcn_frexp_expf(mx);
      ex[0] = e;
      // slices whose largest |x| is below 2^-104 first gain 2^64 (2^e
      // must be a normal float)
      float pre = 1.0f;
      if (e > 126) {
        e -= 64;
        pre = 0x1p64f;
#pragma unroll
        for (int i = 0; i < XR; ++i)
          xr[i] = float4{xr[i].x * pre, xr[i].y * pre, xr[i].z * pre, xr[i].w * pre};
      }
      stage_dig(ldexp_f(1.0f, e), pre);
      return false;
    } else {
    stage(std::false_type{});
    // Per lane: bit r = row r has a value >= 2^-10 here, bit 31 = some row
    // has a value >= 2^15 here; one OR across the wave (VALU and a few scalar
    // instructions: the scalar unit is shared by the CU's waves).
    uint32_t flags = 0;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      if (r >= M) break;  // wave-uniform
      const float mx = reg_max(r);
      flags |= (mx >= 0x1p-10f ? 1u << r : 0u) | (mx >= 0x1p15f ? 1u << 31 : 0u);
    }
    if (c4 > c_done) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (r >= M) break;  // wave-uniform
        const float mx = rest_max(r);
        flags |= (mx >= 0x1p-10f ? 1u << r : 0u) | (mx >= 0x1p15f ? 1u << 31 : 0u);
      }
    }
    const uint32_t all = wave_or(flags);
    const bool unit = all == ((1u << M) - 1u);
    if (!unit) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (r >= M) break;  // wave-uniform
        float mx = reg_max(r);
        if (c4 > c_done) mx = fmaxf(mx, rest_max(r));
        ex[r] = __builtin_amdgcn_readfirstlane(pow2_scale_exp(wave_max_nonneg(mx)));
      }
      stage(std::true_type{});
    }
    return unit;
    }
  };

  // ---- weight loads around the staging --------------------------------------
  // Issued group by group (not clustered by kind), so group 0 can start as
  // soon as its own line and scales land. Non-ring slices issue two groups
  // ahead of the staging, or, in grids of one round (xbar), hold every
  // weight load until all waves of the workgroup issued their activation
  // loads and then issue one (one activation row) or two (see the order of
  // issue above). Both orders are written out so that each path's wait
  // counts stay exact.
  Slot<QT> ring[GW];
  constexpr int kPre = RING ? 0 : (GW < 2 ? GW : 2);
  constexpr int kPreX = MR == 1 ? (kPre < 1 ? kPre : 1) : kPre;  // xbar path
  auto issue = [&](int s) __attribute__((always_inline)) {
    load_group<QT>(rs, ring[s], s, qoff, soff);
    __builtin_amdgcn_sched_barrier(0);
  };
  if (a.xbar) {  // workgroup-uniform
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  }
  bool unit;
  if (kPreX < kPre && a.xbar) {
#pragma unroll
    for (int s = 0; s < kPreX; ++s) issue(s);
    unit = stage_slice();
#pragma unroll
    for (int s = kPreX; s < kPre; ++s) issue(s);
  } else {
#pragma unroll
    for (int s = 0; s < kPre; ++s) issue(s);
    unit = stage_slice();
  }
  // ---- weight loads: the rest of the first GW groups ------------------------
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = kPre; s < GW; ++s) {
    load_group<QT>(rs, ring[s], s, qoff, soff);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the slice is private to this wave: only LDS completion is needed
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();

  // MFMA A row `n` carries activation row n/2 (hi for even n, lo for odd n).
  // Rows past 2m read row 0 again: their D rows are never used, and an
  // unmasked read costs no VALU work.
  const _Float16* arow = xs + (size_t)(n < 2 * M ? n : 0) * a.xstride + 8 * kq;
  const _Float16* asum = xsa + (size_t)(n < 2 * M ? n : 0) * kGroupBlocks;
  const int r0 = 2 * kq, r1 = 2 * kq + 1;  // activation rows of this lane's D
  float acc0 = 0.0f, acc1 = 0.0f;

  // Group j from `slot`: decode the B fragments, (ring) refill the slot with
  // group j + GW, four MFMAs, then the fp32 fixups.
  // DIG: per group, the corrections and four blocks run as one chain of
  // MFMAs into D: first A = every digit row against -bias (the codes' fp16
  // bias per k position), then block b with A = the rows of block b only
  // (other lanes read the zero slot) against the biased codes of block b.
  // Every product and partial sum is an integer below 2^24 (|digit| <= 128,
  // codes below 1280, 32 products), so D holds exactly
  // sum(digit_i * (q - bias')) for block kq, digit i = 0..2, in this lane's
  // D[i]; the digits combine in fp32 and take the block's scale (and the
  // q4_1 min times the block's sum of X).
  const int dmb = n >> 2, dmi = n & 3;  // A row n = 4 * block + digit
  const uint32_t off_all =
      dmi < 3 ? (uint32_t)(((dmb * 3 + dmi) * 4 + kq) * 16) : (uint32_t)kDigZero;
  const uint32_t dsel = (uint32_t)(2 * kq) | ((uint32_t)(2 * kq + 1) << 8) | 0x0C0C0000u;
  constexpr float kBias0 = QT == MLQ_Q8_0 ? 1152.0f : QT == MLQ_Q4_0 ? 1032.0f : 1024.0f;
  constexpr float kBias1 = QT == MLQ_Q8_0 ? 1152.0f : QT == MLQ_Q4_0 ? 72.0f : 64.0f;
  const h8_t negb = {(_Float16)-kBias0, (_Float16)-kBias0, (_Float16)-kBias1, (_Float16)-kBias1,
                     (_Float16)-kBias0, (_Float16)-kBias0, (_Float16)-kBias1, (_Float16)-kBias1};
  auto group = [&](Slot<QT>& slot, int j) {
    if constexpr (DIG) {
      uint4 bq[kGroupBlocks];  // biased codes, fp16
#pragma unroll
      for (int b = 0; b < kGroupBlocks; ++b) {
        if (QT == MLQ_Q8_0) {
          const uint4 q = (b < 2) ? slot.q : slot.q2;
          q8_pairs((b & 1) ? q.z : q.x, bq[b].x, bq[b].y);
          q8_pairs((b & 1) ? q.w : q.y, bq[b].z, bq[b].w);
        } else {
          const uint32_t w0 = b == 0 ? slot.q.x : b == 1 ? slot.q.y
                            : b == 2 ? slot.q.z : slot.q.w;
          const Q4Pairs p = q4_pairs(w0);
          bq[b] = make_uint4(p.p0, p.p1, p.p2, p.p3);
        }
      }
      const uint2 dd = slot.d;
      const uint2 mm = slot.m;
      if (RING) load_group<QT>(rs, slot, j + GW, qoff, soff);
      const unsigned char* rj = arec + (size_t)j * kDigRec;
      const f4_t zero = {0.f, 0.f, 0.f, 0.f};
      f4_t D = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(h8_t, *(const uint4*)(rj + off_all)), negb, zero, 0, 0, 0);
#pragma unroll
      for (int b = 0; b < kGroupBlocks; ++b) {
        const uint32_t off = dmb == b ? off_all : (uint32_t)kDigZero;
        D = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, *(const uint4*)(rj + off)),
                                                   __builtin_bit_cast(h8_t, bq[b]), D, 0, 0, 0);
      }
      const float v = fmaf(D[2], 65536.0f, fmaf(D[1], 256.0f, D[0]));
      acc0 = fmaf(half_bits_to_float((uint16_t)__builtin_amdgcn_perm(dd.y, dd.x, dsel)), v, acc0);
      if (QT == MLQ_Q4_1)
        acc0 = fmaf(half_bits_to_float((uint16_t)__builtin_amdgcn_perm(mm.y, mm.x, dsel)),
                    ssum[j * kGroupBlocks + kq], acc0);
      return;
    }
    h8_t bfrag[kGroupBlocks];
#pragma unroll
    for (int b = 0; b < kGroupBlocks; ++b) {
      if (QT == MLQ_Q8_0) {
        const uint4 q = (b < 2) ? slot.q : slot.q2;
        bfrag[b] = decode8<QT>((b & 1) ? q.z : q.x, (b & 1) ? q.w : q.y);
      } else {
        const uint32_t w0 = b == 0 ? slot.q.x : b == 1 ? slot.q.y
                          : b == 2 ? slot.q.z : slot.q.w;
        bfrag[b] = decode8<QT>(w0, 0);
      }
    }
    const uint2 dd = slot.d;
    const uint2 mm = slot.m;
    if (RING) load_group<QT>(rs, slot, j + GW, qoff, soff);
    const f4_t zero = {0.f, 0.f, 0.f, 0.f};
    f4_t D[kGroupBlocks];
#pragma unroll
    for (int b = 0; b < kGroupBlocks; ++b) {
      const uint4 av = *(const uint4*)(arow + j * kGroupK + b * kQK);
      D[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(h8_t, av), bfrag[b], zero, 0, 0, 0);
    }
    // q4_1: sum_b m_b * S_b on the MFMA (A row n: the hi/lo block sums of
    // activation row n/2 at K 0..3; B: the row's four mins at K 0..3; the
    // lanes of quarters 1..3 hold K 8..31, all zero)
    f4_t Dm = zero;
    if (QT == MLQ_Q4_1) {
      const uint2 sv = kq == 0 ? *(const uint2*)(asum + (size_t)j * kTileRows * kGroupBlocks)
                               : make_uint2(0u, 0u);
      const uint4 av = make_uint4(sv.x, sv.y, 0u, 0u);
      const uint4 bv = kq == 0 ? make_uint4(mm.x, mm.y, 0u, 0u) : make_uint4(0u, 0u, 0u, 0u);
      Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, av),
                                                  __builtin_bit_cast(h8_t, bv), zero, 0, 0, 0);
    }
#pragma unroll
    for (int b = 0; b < kGroupBlocks; ++b) {
      const float df = (float)half_at(dd, b);
      acc0 = fmaf(df, D[b][0] + D[b][1], acc0);
      if (MR > 1) acc1 = fmaf(df, D[b][2] + D[b][3], acc1);
    }
    if (QT == MLQ_Q4_1) {
      acc0 += 64.0f * (Dm[0] + Dm[1]);
      if (MR > 1) acc1 += 64.0f * (Dm[2] + Dm[3]);
    }
  };

  // The scheduling barrier between groups keeps each group's LDS reads and
  // temporaries local (hoisting them across groups costs registers, hence
  // occupancy, for no gain: the weight lines are what the wave waits for).
  if (RING) {
    for (int jb = 0; jb < npad; jb += GW) {
#pragma unroll
      for (int s = 0; s < GW; ++s) {
        group(ring[s], jb + s);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < GW; ++s) {
      group(ring[s], s);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // PB: the bias (or residual) entries of the rows this thread writes,
  // requested before the slices combine: loaded after the final barrier
  // they added a memory round trip to the tail of every workgroup, and
  // requested with the activations they held registers through the group
  // loop. Row tile*16 + (tid & 15); under SwiGLU with several slices the
  // thread writes gate row (tid & 7) and up row (tid & 7) + 8. Only waves 0
  // and 1 write outputs (the other waves' loads move no data); rows past n
  // read zero. (A compile-time choice: a runtime branch around these loads
  // cost the group loop registers, and empty loads without a bias cost the
  // short GEMVs 1-3 %.)
  float bias0 = 0.0f, bias8 = 0.0f;
  if constexpr (PB) {
    __builtin_amdgcn_sched_barrier(0);
    const rsrc_t rb = make_rsrc(a.epi.bias + (size_t)tile * kTileRows,
                                wave < 2 ? (uint32_t)min(kTileRows, a.n - tile * kTileRows) * 4u
                                         : 0u);
    const bool pairs = a.epi.act == kEpiSwiGLU && a.split > 1;
    const uint32_t bc = pairs ? (uint32_t)(tid & 7) : (uint32_t)(tid & 15);
    bias0 = __builtin_bit_cast(float, buf_load4(rb, bc * 4u, 0));
    bias8 = __builtin_bit_cast(float, buf_load4(rb, (bc + 8u) * 4u, 0));
    __builtin_amdgcn_sched_barrier(0);
  }
  // output v of row `row`; b: its prefetched entry
  auto biased = [&](float v, float b, int row) {
    if constexpr (PB) return v + b;
    return add_bias(a.epi, v, row);
  };

  // ---- output ------------------------------------------------------------
  if constexpr (DIG) {
    // the lane quarters hold the sums over blocks kq of the groups: add
    // them (every lane gets the same bits)
    acc0 = xor32_sum(xor16_sum(acc0));
    if (nonfin) acc0 = __builtin_nanf("");
  }
  // undo the slice's power-of-two scale of activation rows r0 and r1
  if (!unit) {
    int e0 = ex[0], e1 = ex[0];
#pragma unroll
    for (int q = 1; q < NR; ++q) {
      if (q == r0) e0 = ex[q];
      if (q == r1) e1 = ex[q];
    }
    acc0 = ldexp_f(acc0, -e0);
    if (MR > 1) acc1 = ldexp_f(acc1, -e1);
  }
  // RMSNorm scale of the (single) row: sum(x^2) over lanes, then over the
  // K slices of the workgroup in slice order
  float nscale = 1.0f;
  if constexpr (norm) {
    ssq = wave_sum(ssq);
    if (a.split == 1) nscale = sqrtf(ssq / (float)a.k + a.epi.norm_eps);
  }
  if constexpr (pre) {
    // the parts added in one fixed order (DPP and scalar adds: short enough
    // for every wave's tail; computed here rather than before the group
    // loop, where it delayed the first MFMA; wave 0's value is the one used)
    const float t = wave_sum((sp4.x + sp4.y) + (sp4.z + sp4.w));
    nscale = sqrtf(t / (float)a.k + a.epi.norm_eps);
  }
  if (a.split == 1) {
    const int row = tile * kTileRows + n;
    if (norm || pre) {
      acc0 = acc0 / nscale;
      acc1 = acc1 / nscale;
    }
    const float v0 = biased(acc0, bias0, min(row, a.n - 1));
    const float v1 = biased(acc1, bias0, min(row, a.n - 1));
    if (can_produce && a.epi.next_x != nullptr) {  // one row, no activation
      produce_norm_input(a, tile, lane, kq == 0 && row < a.n ? v0 : 0.0f, gnext);
      if (kq == 0 && row < a.n) a.y[row] = v0;
      return;
    }
    if (a.epi.act == kEpiSwiGLU) {
      // the up row of lane n (< 8) sits in lane n + 8
      const float u0 = __shfl_xor(v0, 8);
      const float u1 = __shfl_xor(v1, 8);
      if (n < 8 && row < a.n) {
        if (r0 < M) a.y[(size_t)r0 * a.ny + glu_col(row)] = silu_f(v0) * u0;
        if (MR > 1 && r1 < M) a.y[(size_t)r1 * a.ny + glu_col(row)] = silu_f(v1) * u1;
      }
      return;
    }
    if (row < a.n) {
      if (r0 < M) a.y[(size_t)r0 * a.n + row] = v0;
      if (MR > 1 && r1 < M) a.y[(size_t)r1 * a.n + row] = v1;
    }
    return;
  }
  // K slices combine in slice order (deterministic)
  if (r0 < M) part[(wave * M + r0) * kTileRows + n] = acc0;
  if (MR > 1 && r1 < M) part[(wave * M + r1) * kTileRows + n] = acc1;
  float* ssp = part + (size_t)a.split * M * kTileRows;  // per-slice sum(x^2)
  if (norm && lane == 0) ssp[wave] = ssq;
  if (pre && wave == 0 && lane == 0) ssp[0] = nscale;
  __syncthreads();
  if constexpr (norm) {
    float t = 0.0f;
    for (int w = 0; w < a.split; ++w) t += ssp[w];
    nscale = sqrtf(t / (float)a.k + a.epi.norm_eps);
  }
  if constexpr (pre) nscale = ssp[0];  // wave 0's

  auto slice_sum = [&](int r, int nn) {
    float s = 0.0f;
    for (int w = 0; w < a.split; ++w) s += part[(w * M + r) * kTileRows + nn];
    return norm || pre ? s / nscale : s;
  };
  if (can_produce && a.epi.next_x != nullptr) {  // one row, no activation
    if (wave == 0) {
      const int row = tile * kTileRows + (lane & 15);
      const bool live = lane < kTileRows && row < a.n;
      const float v = live ? biased(slice_sum(0, lane & 15), bias0, row) : 0.0f;
      produce_norm_input(a, tile, lane, v, gnext);
      if (live) a.y[row] = v;
    }
    return;
  }
  if (a.epi.act == kEpiSwiGLU) {
    for (int o = tid; o < M * 8; o += blockDim.x) {
      const int r = o / 8, c = o % 8;
      const int row = tile * kTileRows + c;
      if (row >= a.n) continue;
      const float g = biased(slice_sum(r, c), bias0, row);
      const float u = biased(slice_sum(r, c + 8), bias8, row + 8);
      a.y[(size_t)r * a.ny + glu_col(row)] = silu_f(g) * u;
    }
    return;
  }
  for (int o = tid; o < M * kTileRows; o += blockDim.x) {
    const int r = o / kTileRows, nn = o % kTileRows;
    const int row = tile * kTileRows + nn;
    if (row < a.n) a.y[(size_t)r * a.n + row] = biased(slice_sum(r, nn), bias0, row);
  }
}

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

// Split override: set through mlq_set_gemv_split, initialised from the
// MLQ_GEMV_SPLIT environment variable (0 = automatic).
int g_split_override = -1;

int split_override() {
  if (g_split_override < 0) g_split_override = env_int("MLQ_GEMV_SPLIT", 0);
  return g_split_override;
}

struct Plan {
  int split, gw;
  int depth;  // GW: groups in flight per wave (1..10)
  bool ring;  // slices longer than max_depth groups: ring of `depth` slots
  int padded; // groups staged per wave (gw, or whole ring passes)
  size_t wave_lds, lds;
};

// Groups in flight per wave without spilling (VGPR budget of a 1024-thread
// workgroup): every group of the slice when gw <= max_depth, else a ring.
// q4_1 carries mins and block sums per group, so its budgets are smaller
// (seven groups for one row, a ring of at most four); one activation row
// leaves room for ten (long-K shapes with few tiles, e.g. the 3584 x 18944
// down-projection, keep more bytes in flight).
constexpr int kMaxDepth = 8;
constexpr int kMaxDepthOneRow = 10;
int max_depth(int type, int m) {
  if (type == MLQ_Q4_1) return m == 1 ? 7 : 3;
  // q8_0 lines are twice as long: one group less than q4_0 fits
  if (type == MLQ_Q8_0) return m == 1 ? kMaxDepthOneRow - 1 : kMaxDepth - 1;
  return m == 1 ? kMaxDepthOneRow : kMaxDepth;
}
// Ring depths that compile without spills, per type and row class.
int ring_depth_lo(int type, int m) { return type == MLQ_Q4_1 ? (m == 1 ? 3 : 2) : 4; }
int ring_depth_hi(int type, int m) { return type == MLQ_Q4_1 ? (m == 1 ? 4 : 2) : 8; }

// Ring depth for a slice of gw groups: the one that pads the slice least to
// whole passes (padded groups cost decode and MFMA work on zeros), the
// deeper one on ties.
int ring_depth(int type, int m, int gw) {
  int best = ring_depth_hi(type, m), best_pad = 1 << 30;
  for (int d = ring_depth_hi(type, m); d >= ring_depth_lo(type, m); --d) {
    const int pad = (gw + d - 1) / d * d - gw;
    if (pad < best_pad) {
      best = d;
      best_pad = pad;
    }
  }
  return best;
}

// Groups a wave of `gw` processes (and stages activations for).
int padded_groups(int type, int m, int gw) {
  if (gw <= max_depth(type, m)) return gw;
  const int rd = ring_depth(type, m, gw);
  return (gw + rd - 1) / rd * rd;
}

// Whether the kernel a plan launches stages digits: one activation row,
// every group of the slice in flight (no ring), at most kDigMaxDepth of
// them. The digit records take 784 bytes a group against ~512 for hi/lo
// pairs, so ring slices keep the pairs: the one-row GEMV then still reaches
// K ~ 38K (70B-class down projections, K = 28672 .. 29568).
bool dig_layout(int type, int m, int gw) {
  return m == 1 && gw <= kDigMaxDepth && gw <= max_depth(type, m);
}

size_t wave_lds_bytes(int type, int m, int gw) {
  const int pg = padded_groups(type, m, gw);
  if (dig_layout(type, m, gw))  // digit records (+ q4_1 block sums)
    return (size_t)pg * kDigRec + (type == MLQ_Q4_1 ? (size_t)pg * kGroupBlocks * 4 : 0);
  const size_t xstride = (size_t)pg * kGroupK + kRowPadHalves;
  size_t b = (size_t)2 * m * xstride * 2;
  if (type == MLQ_Q4_1) b += (size_t)pg * kTileRows * kGroupBlocks * 2;  // block sums
  return (b + 15) / 16 * 16;
}

Plan make_plan(int type, int m, const Geometry& geo) {
  Plan p;
  const int env_split = split_override();
  // Default split: about 32 waves per CU, keeping at least three groups per
  // wave for one activation row (two for more rows: an 8-row wave carries
  // more work per group), and short enough slices that every group of a
  // slice is in flight at once (no ring) when a workgroup of 16 waves
  // allows it. One-row shapes of K = 3584..4096 (14..16 groups) measured
  // faster at four groups per wave than at two (q8_0 W[4096, 4096]
  // 5.22 -> 5.01 us; the decode step's o and q|k|v projections), while
  // W[4096, 4096] at M = 4 measured slower (5.2 -> 6.3 us).
  const int min_groups = m == 1 ? 3 : 2;
  int split = 1;
  if (env_split >= 1 && env_split <= kMaxSplit && (env_split & (env_split - 1)) == 0) {
    split = env_split;
  } else {
    while (split < kMaxSplit && 2 * split <= geo.g) {
      const bool more_waves = geo.nt * split < kTargetWaves &&
                              (geo.g + 2 * split - 1) / (2 * split) >= min_groups;
      const bool shorter = (geo.g + split - 1) / split > max_depth(type, m);
      if (!more_waves && !shorter) break;
      split *= 2;
    }
  }
  split = std::min(split, std::max(1, geo.g));
  // Each wave stages its own K slice: widen the split until they fit in LDS.
  for (;;) {
    p.split = split;
    p.gw = (geo.g + split - 1) / split;
    p.wave_lds = wave_lds_bytes(type, m, p.gw);
    p.lds = p.wave_lds * split +
            (split > 1 ? (size_t)split * (m * kTileRows + 1) * 4 : 0);
    if (p.lds <= lds_limit() || split >= kMaxSplit) break;
    split *= 2;
  }
  // every wave of the workgroup must own at least one group
  p.split = (geo.g + p.gw - 1) / p.gw;
  p.lds = p.wave_lds * p.split +
          (p.split > 1 ? (size_t)p.split * (m * kTileRows + 1) * 4 : 0);
  // Every group of the slice in flight at once (depth = gw) when it fits,
  // otherwise the ring.
  p.ring = p.gw > max_depth(type, m);
  p.depth = p.ring ? ring_depth(type, m, p.gw) : p.gw;
  p.padded = padded_groups(type, m, p.gw);
  return p;
}

template <int QT, int MR, int GW, bool RING, int NM, bool VEC, bool PB>
hipError_t launch_vec(const GemvArgs& a, size_t lds, hipStream_t stream) {
  // Opt in to more than the default 64 KiB of dynamic LDS when needed.
  const hipError_t e =
      allow_dynamic_lds((const void*)gemv_kernel<QT, MR, GW, RING, NM, VEC, PB>, lds);
  if (e != hipSuccess) return e;
  gemv_kernel<QT, MR, GW, RING, NM, VEC, PB><<<a.nt, 64 * a.split, lds, stream>>>(a);
  return hipGetLastError();
}

template <int QT, int MR, int GW, bool RING, int NM>
hipError_t launch_kernel(const GemvArgs& a, size_t lds, hipStream_t stream) {
  if ((a.k & 3) == 0) {
    if constexpr (MR == 1 && NM != 1)
      if (a.epi.bias != nullptr) return launch_vec<QT, MR, GW, RING, NM, true, true>(a, lds, stream);
    return launch_vec<QT, MR, GW, RING, NM, true, false>(a, lds, stream);
  }
  return launch_vec<QT, MR, GW, RING, NM, false, false>(a, lds, stream);
}

// The input-RMSNorm variant exists for one activation row, and not for the
// deepest non-ring slices (q8_0 depth 9-10, q4_1 depth 6), whose register
// budget the norm weight's registers would overflow.
constexpr bool norm_variant(int qt, int gw, bool ring) {
  return ring || !((qt == MLQ_Q8_0 && gw >= 9) || (qt == MLQ_Q4_1 && gw >= 6));
}

// The pre-scaled variant holds four registers more than the plain one: it
// exists except for q4_1 at depth 7 (which would spill).
constexpr bool prenorm_variant(int qt, int gw, bool ring) {
  return ring || !(qt == MLQ_Q4_1 && gw >= 7);
}

template <int QT, int MR, int GW, bool RING>
hipError_t launch_typed(const GemvArgs& a, size_t lds, hipStream_t stream) {
  if (a.epi.ssq_parts != nullptr) {
    if constexpr (MR == 1 && prenorm_variant(QT, GW, RING))
      return launch_kernel<QT, MR, GW, RING, 2>(a, lds, stream);
    return hipErrorInvalidValue;
  }
  if (a.epi.norm != nullptr) {
    if constexpr (MR == 1 && norm_variant(QT, GW, RING))
      return launch_kernel<QT, MR, GW, RING, 1>(a, lds, stream);
    return hipErrorInvalidValue;
  }
  return launch_kernel<QT, MR, GW, RING, 0>(a, lds, stream);
}

template <int QT, int MR>
hipError_t launch_depth(const GemvArgs& a, const Plan& p, hipStream_t stream) {
  if (p.ring) {
    if constexpr (QT == MLQ_Q4_1 && MR > 1) {
      return launch_typed<QT, MR, 2, true>(a, p.lds, stream);
    } else if constexpr (QT == MLQ_Q4_1) {
      if (p.depth == 3) return launch_typed<QT, MR, 3, true>(a, p.lds, stream);
      return launch_typed<QT, MR, 4, true>(a, p.lds, stream);
    } else {
    switch (p.depth) {
      case 4: return launch_typed<QT, MR, 4, true>(a, p.lds, stream);
      case 5: return launch_typed<QT, MR, 5, true>(a, p.lds, stream);
      case 6: return launch_typed<QT, MR, 6, true>(a, p.lds, stream);
      case 7: return launch_typed<QT, MR, 7, true>(a, p.lds, stream);
      default: return launch_typed<QT, MR, 8, true>(a, p.lds, stream);
    }
    }
  }
  // (depths above max_depth(QT, m) are never planned)
  switch (p.depth) {
    case 1: return launch_typed<QT, MR, 1, false>(a, p.lds, stream);
    case 2: return launch_typed<QT, MR, 2, false>(a, p.lds, stream);
    case 3: return launch_typed<QT, MR, 3, false>(a, p.lds, stream);
    case 4: return launch_typed<QT, MR, (QT == MLQ_Q4_1 && MR > 1) ? 3 : 4, false>(a, p.lds, stream);
    case 5: return launch_typed<QT, MR, (QT == MLQ_Q4_1 && MR > 1) ? 3 : 5, false>(a, p.lds, stream);
    case 6: return launch_typed<QT, MR, (QT == MLQ_Q4_1 && MR > 1) ? 3 : 6, false>(a, p.lds, stream);
    case 7: return launch_typed<QT, MR, (QT == MLQ_Q4_1 && MR > 1) ? 3 : 7, false>(a, p.lds, stream);
    case 8:
      return launch_typed<QT, MR, QT == MLQ_Q4_1 ? (MR > 1 ? 3 : 7)
                                  : (QT == MLQ_Q8_0 && MR > 1) ? 7 : 8, false>(a, p.lds, stream);
    default:
      // 9 and 10: one activation row, q8_0 (9) / q4_0 (10) only
      if constexpr (QT == MLQ_Q8_0 && MR == 1) {
        return launch_typed<QT, MR, 9, false>(a, p.lds, stream);
      } else if constexpr (QT == MLQ_Q4_0 && MR == 1) {
        if (p.depth == 9) return launch_typed<QT, MR, 9, false>(a, p.lds, stream);
        return launch_typed<QT, MR, 10, false>(a, p.lds, stream);
      }
      return launch_typed<QT, MR, QT == MLQ_Q4_1 ? (MR > 1 ? 3 : 7)
                                  : (QT == MLQ_Q8_0 && MR > 1) ? 7 : 8, false>(a, p.lds, stream);
  }
}

template <int QT>
hipError_t launch_rows(const GemvArgs& a, const Plan& p, hipStream_t stream) {
  if (a.m == 1) return launch_depth<QT, 1>(a, p, stream);
  return launch_depth<QT, kGemvMaxRows>(a, p, stream);
}

}  // namespace

hipError_t allow_dynamic_lds(const void* kernel, size_t lds) {
  constexpr size_t kDefaultLds = 64 * 1024;
  if (lds <= kDefaultLds) return hipSuccess;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  static std::mutex mu;
  static std::set<std::pair<int, const void*>> raised;  // (device, kernel)
  std::lock_guard<std::mutex> lock(mu);
  if (raised.count({dev, kernel}) != 0) return hipSuccess;
  int max_bytes = 0;
  e = hipDeviceGetAttribute(&max_bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) return e;
  if ((size_t)max_bytes < lds) return hipErrorInvalidValue;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, max_bytes);
  if (e == hipSuccess) raised.insert({dev, kernel});
  return e;
}

void set_gemv_split(int split) { g_split_override = split; }

bool gemv_norm_supported(const mlq_weight& w) {
  if (w.type != MLQ_Q8_0 && w.type != MLQ_Q4_0 && w.type != MLQ_Q4_1) return false;
  const Plan p = make_plan(w.type, 1, geometry(w.n, w.k));
  if (p.lds > lds_limit()) return false;
  // the variant launch_depth would pick for this plan
  int depth = p.depth;
  if (!p.ring && w.type == MLQ_Q4_1) depth = std::min(depth, 7);
  return norm_variant(w.type, depth, p.ring);
}

bool gemv_prenorm_supported(const mlq_weight& w) {
  if (w.type != MLQ_Q8_0 && w.type != MLQ_Q4_0 && w.type != MLQ_Q4_1) return false;
  const Plan p = make_plan(w.type, 1, geometry(w.n, w.k));
  if (p.lds > lds_limit()) return false;
  int depth = p.depth;
  if (!p.ring && w.type == MLQ_Q4_1) depth = std::min(depth, 7);
  return prenorm_variant(w.type, depth, p.ring);
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
                       hipStream_t stream, const Epilogue& epi) {
  const Geometry geo = geometry(w.n, w.k);
  if (m < 1 || m > kGemvMaxRows) return hipErrorInvalidValue;
  if (epi.norm != nullptr && m != 1) return hipErrorInvalidValue;
  if (epi.ssq_parts != nullptr &&
      (m != 1 || epi.norm != nullptr || epi.ssq_count < 1 || epi.ssq_count > kSsqPartsMax ||
       ((uintptr_t)epi.ssq_parts & 15) != 0))
    return hipErrorInvalidValue;
  if (epi.next_x != nullptr && (m != 1 || epi.act != kEpiNone || epi.next_norm == nullptr ||
                                epi.next_ssq == nullptr || epi.norm != nullptr ||
                                epi.ssq_parts != nullptr))
    return hipErrorInvalidValue;
  const Plan p = make_plan(w.type, m, geo);
  if (p.lds > lds_limit()) return hipErrorInvalidValue;
  GemvArgs a;
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
  a.split = p.split;
  a.gw = p.gw;
  a.xstride = p.padded * kGroupK + kRowPadHalves;
  a.wave_lds = (int)p.wave_lds;
  a.epi = epi;
  a.ny = epi.act == kEpiSwiGLU ? w.n / 2 : w.n;
  // Activation loads ahead of every weight load of the workgroup: for grids
  // of at most ~1.25 workgroups per CU whose waves read at least a third as
  // many activation bytes as weight bytes (all but q8_0 at one row).
  const int unit_bytes = (w.type == MLQ_Q8_0 ? 2048 : 1024) + kUnitScaleBytes +
                         (w.type == MLQ_Q4_1 ? kUnitScaleBytes : 0);
  a.xbar = p.split > 1 && 4 * (long)geo.nt <= 5 * (long)device_cus() &&
           3 * m * kGroupK * 4 >= unit_bytes;
  switch (w.type) {
    case MLQ_Q8_0: return launch_rows<MLQ_Q8_0>(a, p, stream);
    case MLQ_Q4_0: return launch_rows<MLQ_Q4_0>(a, p, stream);
    default: return launch_rows<MLQ_Q4_1>(a, p, stream);
  }
}

}  // namespace mlq
