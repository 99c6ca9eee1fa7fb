// Decode-step operators around the quantized Linear: RMSNorm, RoPE with the
// KV-cache write, decode attention over the cache, token embedding,
// elementwise SiLU / product / sum and the greedy argmax. All activations are
// fp32, as in the reference's device path (src/cuda_ops.cu:129-560,
// src/cuda_attention.cu:142-270).
//
// Positions and tokens may come from device memory (pos_dev / token_dev) so a
// whole decode step can be captured once in a HIP graph and replayed for
// every token: grids are then sized for the cache capacity and workgroups
// past the live length exit at once.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <stdint.h>

#include "device_common.h"

namespace mlq {
namespace {

__device__ __forceinline__ int read_scalar(const int32_t* dev, int host) {
  return dev != nullptr ? *dev : host;
}

// ---- RMSNorm ------------------------------------------------------------------
// y = x * w / sqrt(mean(x^2) + eps) per row (rmsNorm, src/ops.cc:43-72: the
// product x*w is divided by the scale, in that order). One workgroup per row.
constexpr int kNormThreads = 256;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const float* __restrict__ x, const float* __restrict__ w,
    float* __restrict__ y, int dim, float eps) {
  __shared__ float part[kNormThreads / 64];
  const float* xr = x + (size_t)blockIdx.x * dim;
  float* yr = y + (size_t)blockIdx.x * dim;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < dim; i += kNormThreads) ss += xr[i] * xr[i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) total += part[i];
  const float scale = sqrtf(total / (float)dim + eps);
  for (int i = threadIdx.x; i < dim; i += kNormThreads)
    yr[i] = xr[i] * w[i] / scale;
}

// Row held in registers: R float4 of x and of the weight per thread, every
// load issued before the reduction (one memory round trip), no second read. dim % 4 == 0 and
// 16-byte aligned rows.
template <int R>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_vec_kernel(
    const float* __restrict__ x, const float* __restrict__ w,
    float* __restrict__ y, int dim, float eps) {
  __shared__ float part[kNormThreads / 64];
  const int n4 = dim >> 2;
  const f4_t* xr = (const f4_t*)(x + (size_t)blockIdx.x * dim);
  f4_t* yr = (f4_t*)(y + (size_t)blockIdx.x * dim);
  const f4_t* w4 = (const f4_t*)w;
  f4_t v[R], wv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = threadIdx.x + r * kNormThreads;
    v[r] = i < n4 ? xr[i] : f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    wv[r] = i < n4 ? w4[i] : f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  float ss = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    ss += v[r].x * v[r].x;
    ss += v[r].y * v[r].y;
    ss += v[r].z * v[r].z;
    ss += v[r].w * v[r].w;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) total += part[i];
  const float scale = sqrtf(total / (float)dim + eps);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = threadIdx.x + r * kNormThreads;
    if (i < n4)
      yr[i] = f4_t{v[r].x * wv[r].x / scale, v[r].y * wv[r].y / scale,
                   v[r].z * wv[r].z / scale, v[r].w * wv[r].w / scale};
  }
}

// ---- elementwise ----------------------------------------------------------------
__device__ __forceinline__ float silu_exact(float g) { return g / (1.0f + expf(-g)); }

template <int OP>
__global__ __launch_bounds__(256) void eltwise_kernel(const float* __restrict__ a,
                                                      const float* __restrict__ b,
                                                      float* __restrict__ y,
                                                      int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    if constexpr (OP == kEltAdd) y[i] = a[i] + b[i];
    if constexpr (OP == kEltMul) y[i] = a[i] * b[i];
    if constexpr (OP == kEltSilu) y[i] = silu_exact(a[i]);
    if constexpr (OP == kEltSwiGLU) y[i] = silu_exact(a[i]) * b[i];
  }
}

// ---- softmax ----------------------------------------------------------------------
// y = exp(x - max) / sum over one vector (softmax, src/ops.cc:74-109;
// cudaSoftmax, src/cuda_ops.cu:567-600): one workgroup, three passes over x
// (max, then exp and sum, then the division); the fp32 sum is a tree, not
// the CPU's sequential one.
constexpr int kSoftmaxThreads = 1024;
__global__ __launch_bounds__(kSoftmaxThreads) void softmax_kernel(const float* __restrict__ x,
                                                                  float* __restrict__ y,
                                                                  int64_t n) {
  __shared__ float part[kSoftmaxThreads / 64];
  const int tid = threadIdx.x;
  auto block_reduce = [&](float v, bool is_max) {
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if ((tid & 63) == 0) part[tid >> 6] = v;
    __syncthreads();
    float r = part[0];
    for (int i = 1; i < kSoftmaxThreads / 64; ++i) r = is_max ? fmaxf(r, part[i]) : r + part[i];
    return r;
  };
  float mx = -INFINITY;
  for (int64_t i = tid; i < n; i += kSoftmaxThreads) mx = fmaxf(mx, x[i]);
  mx = block_reduce(mx, true);
  float sum = 0.0f;
  for (int64_t i = tid; i < n; i += kSoftmaxThreads) {
    const float e = expf(x[i] - mx);
    y[i] = e;
    sum += e;
  }
  sum = block_reduce(sum, false);
  for (int64_t i = tid; i < n; i += kSoftmaxThreads) y[i] = y[i] / sum;
}

// ---- embedding ------------------------------------------------------------------
// y = table[token] (embeddingLookupKernel, src/cuda_ops.cu:415-421). A device
// token outside [0, vocab) yields a NaN row instead of a wild read.
// With rope_cs non-null, workgroup 0 also writes the step's RoPE table for
// position pos: rope_cs[i] = cos(pos * f_i), rope_cs[hd/2 + i] = sin(pos * f_i)
// with f_i = 1 / theta^(2i/hd), the angle of pair i in both pairings
// (src/ops.cc:146-151, 168-173), shared by every layer of the step.
__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ table,
                                                    int vocab, int dim,
                                                    const int32_t* token_dev, int token,
                                                    float* __restrict__ y, float* rope_cs,
                                                    const int32_t* pos_dev, int pos, int hd,
                                                    float theta, NormInput ni) {
  const int t = read_scalar(token_dev, token);
  const bool ok = t >= 0 && t < vocab;
  // the grid covers dim, one element per thread (launch_embedding)
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const float v = i < dim ? (ok ? table[(size_t)t * dim + i] : __builtin_nanf("")) : 0.0f;
  if (i < dim) y[i] = v;
  if (ni.norm != nullptr) {
    // the first layer's pre-scaled RMSNorm input: v * norm, and per 16
    // elements the sum of v^2 (the decode GEMV producer's tree)
    const float sq = row_sum<16>(v * v);
    if (i < dim) ni.xn[i] = v * ni.norm[i];
    if ((threadIdx.x & 15) == 0 && i < dim) ni.parts[i >> 4] = sq;
  }
  if (rope_cs != nullptr && blockIdx.x == 0) {
    const int p = read_scalar(pos_dev, pos);
    const int half = hd >> 1;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      const float freq = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
      float sn, cs;
      sincosf((float)p * freq, &sn, &cs);
      rope_cs[i] = cs;
      rope_cs[half + i] = sn;
    }
  }
}

// ---- RoPE + KV-cache write ---------------------------------------------------------
// One thread per rotated pair of q (n_heads) and k (n_kv_heads). Pair i of a
// head rotates (x[2i], x[2i+1]) (normal, src/ops.cc:143-160) or (x[i],
// x[i + hd/2]) (NeoX, :163-184) by pos * theta^(-2i/hd). With a cache, the
// rotated k and the matching v elements go to cache row (layer, pos) instead
// of back into k; a position at or past the cache capacity writes nothing.
struct RopeArgs {
  float* q;
  float* k;
  const float* v;
  float* keys;    // cache or nullptr
  float* values;
  int n_heads, n_kv, hd, neox;
  int layer, max_seq;
  int pos_limit;  // positions >= pos_limit (<= max_seq) write nothing
  const int32_t* pos_dev;
  int pos;
  float theta;
};

__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const int half = a.hd >> 1;
  const int total = (a.n_heads + a.n_kv) * half;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= total) return;
  const int pos = read_scalar(a.pos_dev, a.pos);
  const bool cache = a.keys != nullptr;
  if (cache && (pos < 0 || pos >= a.pos_limit)) return;
  const int head = p / half;
  const int i = p - head * half;
  const int i0 = a.neox ? i : 2 * i;
  const int i1 = a.neox ? i + half : 2 * i + 1;
  const float freq = 1.0f / powf(a.theta, (float)(2 * i) / (float)a.hd);
  float s, c;
  sincosf((float)pos * freq, &s, &c);
  const bool is_q = head < a.n_heads;
  const int kh = head - a.n_heads;
  float* xr = is_q ? a.q + (size_t)head * a.hd : a.k + (size_t)kh * a.hd;
  const float x0 = xr[i0], x1 = xr[i1];
  const float y0 = x0 * c - x1 * s;
  const float y1 = x0 * s + x1 * c;
  if (is_q || !cache) {
    xr[i0] = y0;
    xr[i1] = y1;
    return;
  }
  const size_t row = (((size_t)a.layer * a.max_seq + pos) * a.n_kv + kh) * a.hd;
  a.keys[row + i0] = y0;
  a.keys[row + i1] = y1;
  const float* vr = a.v + (size_t)kh * a.hd;
  a.values[row + i0] = vr[i0];
  a.values[row + i1] = vr[i1];
}

// Plain cache write of one position's k and v (CudaKvCache::writeDevice,
// src/cuda_kv_cache.cc).
__global__ __launch_bounds__(256) void kv_write_kernel(float* __restrict__ keys,
                                                       float* __restrict__ values,
                                                       const float* __restrict__ k,
                                                       const float* __restrict__ v,
                                                       size_t row, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  keys[row + i] = k[i];
  values[row + i] = v[i];
}

// Prefill: RoPE of `rows` consecutive positions pos0 + r (row r of q, k and
// v at their row strides); q rotated in place, rotated k and v written to
// cache rows (layer, pos0 + r). Same arithmetic as rope_kernel.
struct RopeRowsArgs {
  float* q;
  float* k;
  const float* v;
  int q_stride, k_stride, v_stride, rows;
  float* keys;
  float* values;
  int n_heads, n_kv, hd, neox, layer, max_seq, pos0;
  float theta;
  const float* cs;  // [rows][hd] angle table, or null
};

// Angle of pair i at position pos (the one formula both RoPE row paths use).
__device__ __forceinline__ void rope_angle(int pos, int i, int hd, float theta, float& sn,
                                           float& c) {
  const float freq = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
  sincosf((float)pos * freq, &sn, &c);
}

__global__ __launch_bounds__(256) void rope_table_kernel(float* cs, int rows, int pos0, int hd,
                                                         float theta) {
  const int half = hd >> 1;
  const int r = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= half || r >= rows) return;
  float sn, c;
  rope_angle(pos0 + r, i, hd, theta, sn, c);
  cs[(size_t)r * hd + i] = c;
  cs[(size_t)r * hd + half + i] = sn;
}

__global__ __launch_bounds__(256) void rope_rows_kernel(RopeRowsArgs a) {
  const int half = a.hd >> 1;
  const int per_row = (a.n_heads + a.n_kv) * half;
  const int r = blockIdx.y;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= per_row) return;
  const int pos = a.pos0 + r;
  const int head = p / half;
  const int i = p - head * half;
  const int i0 = a.neox ? i : 2 * i;
  const int i1 = a.neox ? i + half : 2 * i + 1;
  float sn, c;
  if (a.cs != nullptr) {
    c = a.cs[(size_t)r * a.hd + i];
    sn = a.cs[(size_t)r * a.hd + half + i];
  } else {
    rope_angle(pos, i, a.hd, a.theta, sn, c);
  }
  const bool is_q = head < a.n_heads;
  const int kh = head - a.n_heads;
  float* xr = is_q ? a.q + (size_t)r * a.q_stride + (size_t)head * a.hd
                   : a.k + (size_t)r * a.k_stride + (size_t)kh * a.hd;
  const float x0 = xr[i0], x1 = xr[i1];
  const float y0 = x0 * c - x1 * sn;
  const float y1 = x0 * sn + x1 * c;
  if (is_q) {
    xr[i0] = y0;
    xr[i1] = y1;
    return;
  }
  const size_t crow = (((size_t)a.layer * a.max_seq + pos) * a.n_kv + kh) * a.hd;
  a.keys[crow + i0] = y0;
  a.keys[crow + i1] = y1;
  const float* vr = a.v + (size_t)r * a.v_stride + (size_t)kh * a.hd;
  a.values[crow + i0] = vr[i0];
  a.values[crow + i1] = vr[i1];
}

// Prefill: embedding rows y[r] = table[tokens[r]] (tokens checked by the host).
__global__ __launch_bounds__(256) void embed_rows_kernel(const float* __restrict__ table,
                                                         int dim, const int32_t* tokens,
                                                         float* __restrict__ y) {
  const int r = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < dim) y[(size_t)r * dim + i] = table[(size_t)tokens[r] * dim + i];
}

// ---- decode attention ----------------------------------------------------------------
// softmax(q . K^T / sqrt(hd)) . V for one query position against cache
// positions 0..pos of one layer, query head h reading kv head h / group
// (src/forward.cc:526-565, src/cuda_attention.cu:142-270).
//
// Pass 1 (attn_chunk_kernel): one wave per (chunk of positions,
// kv head), covering every query head of the group, so each K/V row is read
// from HBM once per step (the reference reads it once per query head).
//   K rows of the chunk -> LDS (coalesced float4), one lane per position
//   computes the group's scores with q broadcast from LDS, the chunk's max m
//   and l = sum exp(s - m) come from wave reductions, then lanes switch to
//   head dims and accumulate sum_t exp(s_t - m) V[t] with V rows reusing the
//   LDS slab. Partials (m, l, acc[hd]) go to the workspace.
// Pass 2 (attn_combine_kernel): per query head, rescale the chunk partials to
// the global max and divide by the global sum.
// Two kernels share the partial format:
//  - head_dim 64 / 128 / 256 (aligned buffers): attn_reg_kernel keeps its
//    chunk in registers. L = hd/16 lanes share one position (16 dims of K
//    each), so a wave covers P = 64/L positions (16, 8, 4) and issues every
//    K and V load of the chunk before it uses any: one memory round trip
//    per wave instead of one per row. Four waves per workgroup merge their
//    partials in LDS, so a partial covers 4P positions (64, 32, 16). The
//    kernel is VALU-bound at decode contexts (scores and P.V of the
//    workgroup's query heads on each lane's positions), so small grids also
//    split a kv head's query heads over several workgroups (launch_attention).
//    Measured per decode step with that split (Qwen2-7B shape, head_dim
//    128): 4 waves x 8 positions 1.433 ms, 8 x 8 1.452, 8 waves of 4
//    positions (8 dims of K per lane) 1.443, 4 x 4 1.583.
//  - any other head_dim <= 256: attn_chunk_kernel stages 32-position chunks
//    of K, then V, through LDS.
constexpr int kAttnMaxGroup = 16;
constexpr int kAttnMaxHd = 256;
constexpr int kAttnLdsChunk = 32;
constexpr int kAttnRegWaves = 4;  // waves per workgroup of the register kernel
constexpr int kAttnRegKD = 16;    // head dims of K per lane
__host__ __device__ constexpr bool attn_reg_hd(int hd) { return hd == 64 || hd == 128 || hd == 256; }
// positions per workgroup: kAttnRegWaves waves of 64 * kAttnRegKD / hd positions
__host__ __device__ constexpr int attn_reg_chunk(int hd) {
  return kAttnRegWaves * 64 * kAttnRegKD / hd;
}

struct AttnArgs {
  const float* q;       // [n_heads][hd]
  const float* keys;    // [layers][max_seq][n_kv][hd]
  const float* values;
  float* out;           // [n_heads][hd]
  float* part;          // workspace: m, l [n_heads][chunks]; acc [n_heads][chunks][hd]
  int layer, max_seq, n_kv, hd, group, chunks, chunk_len;
  // Positions at or past pos_limit (the smaller of the cache capacity, the
  // caller's limit and what `chunks` partials cover) write no cache row and
  // give NaN outputs.
  int pos_limit;
  int vec;              // K/V rows are float4-aligned (hd % 4 == 0, aligned cache)
  // Query rows (grid z): row r sits at position pos + r and reads q at
  // q + r * q_stride, writes out + r * out_stride; partials are [rows] x
  // [n_heads] x [chunks]. One row for a decode step.
  int rows, q_stride, out_stride;
  const int32_t* pos_dev;
  int pos;
  float scale;
  // Fused RoPE + cache write (register kernel only): q is the raw projection,
  // k_new / v_new the raw k and v of position pos ([n_kv][hd]), rope_cs the
  // step's table; the workgroup holding pos writes its rotated k and its v
  // to cache row (layer, pos) and every read of that row takes the raw
  // values instead.
  const float* k_new;
  const float* v_new;
  const float* rope_cs;
  float* kc;             // the cache, writable (same arrays as keys / values)
  float* vc;
  int neox;
  // register kernel: the kv head's query heads split over hsplit workgroups
  // of hper heads (the last may have fewer); 1 and group otherwise
  int hsplit = 1, hper = 1;
};

// Partial arrays of query row r: m and l [n_heads][chunks], acc
// [n_heads][chunks][hd], each array holding every row.
struct Partials {
  float* m;
  float* l;
  float* acc;
};
__device__ __forceinline__ Partials partials_of(const AttnArgs& a, int r) {
  const size_t per = (size_t)a.group * a.n_kv * a.chunks;  // n_heads * chunks
  Partials p;
  p.m = a.part + (size_t)r * per;
  p.l = a.part + (size_t)a.rows * per + (size_t)r * per;
  p.acc = a.part + 2 * (size_t)a.rows * per + (size_t)r * per * a.hd;
  return p;
}

template <int HD, int GMAX>
__global__ __launch_bounds__(64) void attn_chunk_kernel(AttnArgs a) {
  constexpr int CH = kAttnLdsChunk;
  const int hd = HD ? HD : a.hd;
  const int hdp = (hd + 3) & ~3;
  const int stride = hdp + 4;  // padded LDS row: ds_read_b128 by position lanes stays conflict-free
  extern __shared__ float lds[];
  float* rows = lds;                   // [CH][stride]
  float* qs = lds + CH * stride;       // [GMAX][hdp]
  float* ps = qs + GMAX * hdp;         // [GMAX][CH]

  const int qrow = blockIdx.z;
  const int pos = read_scalar(a.pos_dev, a.pos) + qrow;
  const int len = pos + 1;
  const int t0 = blockIdx.x * CH;
  if (pos < 0 || pos >= a.pos_limit || t0 >= len) return;
  const int nt = min(CH, len - t0);
  const int kvh = blockIdx.y;
  const int lane = threadIdx.x;
  const int G = a.group;
  const float* qrow_ptr = a.q + (size_t)qrow * a.q_stride;
  const size_t row_stride = (size_t)a.n_kv * hd;
  const size_t base = ((size_t)a.layer * a.max_seq + t0) * row_stride + (size_t)kvh * hd;

  auto stage = [&](const float* src) {
    if (a.vec) {
      const int q4 = hd >> 2;
      for (int i = lane; i < nt * q4; i += 64) {
        const int r = i / q4;
        const int c = i - r * q4;
        const f4_t v = *(const f4_t*)(src + base + r * row_stride + 4 * c);
        *(f4_t*)(rows + r * stride + 4 * c) = v;
      }
    } else {
      for (int r = 0; r < nt; ++r)
        for (int c = lane; c < hdp; c += 64)
          rows[r * stride + c] = c < hd ? src[base + r * row_stride + c] : 0.0f;
    }
  };

  // q of the group's heads, zero-padded to hdp
  for (int i = lane; i < G * hdp; i += 64) {
    const int g = i / hdp;
    const int c = i - g * hdp;
    qs[i] = c < hd ? qrow_ptr[(size_t)(kvh * G + g) * hd + c] : 0.0f;
  }
  stage(a.keys);
  __syncthreads();

  // scores: lane = position, sequential over head dims
  float s[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) s[g] = 0.0f;
  const float* kr = rows + min(lane, nt - 1) * stride;
  for (int d = 0; d < hdp; d += 4) {
    const f4_t kv = *(const f4_t*)(kr + d);
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (g < G) {
        const f4_t qv = *(const f4_t*)(qs + g * hdp + d);
        s[g] += qv.x * kv.x;
        s[g] += qv.y * kv.y;
        s[g] += qv.z * kv.z;
        s[g] += qv.w * kv.w;
      }
    }
  }
  const bool valid = lane < nt;
  float m[GMAX], l[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      const float sc = valid ? s[g] * a.scale : -INFINITY;
      m[g] = wave_max(sc);
      const float p = valid ? expf(sc - m[g]) : 0.0f;
      l[g] = wave_sum(p);
      if (lane < CH) ps[g * CH + lane] = p;
    }
  }
  __syncthreads();  // every lane is done reading K rows before V overwrites them
  stage(a.values);
  __syncthreads();

  // acc[g][d] = sum_t p[g][t] * V[t][d]; lane owns dims lane + 64 j
  constexpr int kJ = (HD ? (HD + 63) / 64 : kAttnMaxHd / 64);
  float acc[GMAX][kJ];
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int j = 0; j < kJ; ++j) acc[g][j] = 0.0f;
  for (int t = 0; t < nt; ++t) {
    float v[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int d = lane + 64 * j;
      v[j] = d < hdp ? rows[t * stride + d] : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (g < G) {
        const float p = ps[g * CH + t];
#pragma unroll
        for (int j = 0; j < kJ; ++j) acc[g][j] += p * v[j];
      }
    }
  }
  const int chunk = blockIdx.x;
  const Partials pp = partials_of(a, qrow);
  float* pm = pp.m;
  float* pl = pp.l;
  float* pa = pp.acc;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      const size_t slot = (size_t)(kvh * G + g) * a.chunks + chunk;
      if (lane == 0) {
        pm[slot] = m[g];
        pl[slot] = l[g];
      }
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int d = lane + 64 * j;
        if (d < hd) pa[slot * hd + d] = acc[g][j];
      }
    }
  }
}

// One rotated element of a head: element d of x (raw), its RoPE partner
// (d ^ 1 normal, d +- hd/2 NeoX) and the step's table.
template <int HD>
__device__ __forceinline__ float rope_elem(const float* x, int d, int neox, const float* cs) {
  constexpr int H = HD / 2;
  const int i = neox ? (d < H ? d : d - H) : (d >> 1);
  const bool first = neox ? d < H : (d & 1) == 0;
  const float c = cs[i], sn = cs[H + i];
  const float x0 = first ? x[d] : x[neox ? d - H : d - 1];
  const float x1 = first ? x[neox ? d + H : d + 1] : x[d];
  return first ? x0 * c - x1 * sn : x0 * sn + x1 * c;
}

template <int HD, int GMAX, bool FUSED>
__global__ __launch_bounds__(kAttnRegWaves * 64) void attn_reg_kernel(AttnArgs a) {
  constexpr int KD = kAttnRegKD;  // dims of K per lane
  constexpr int L = HD / KD;      // lanes per position
  constexpr int P = 64 / L;       // positions per wave
  constexpr int KF = KD / 4;      // float4 of K per lane
  constexpr int VJ = HD / 64;     // V dims per lane per position
  constexpr int W = kAttnRegWaves;
  __shared__ f4_t qs[GMAX * HD / 4];
  __shared__ __align__(16) float ps[W][GMAX * P];
  __shared__ float wm[W][GMAX], wl[W][GMAX];
  __shared__ float wacc[W][GMAX][HD];

  const int qrow = blockIdx.z;
  const int pos = read_scalar(a.pos_dev, a.pos) + qrow;
  const int len = pos + 1;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // grid x: chunks, or with a head split (hsplit > 1) chunks x splits laid
  // out so that the splits of one chunk have workgroup ids of equal residue
  // mod 8 (the XCD a workgroup runs on): they read the chunk's K/V rows
  // through one L2
  int chunk = blockIdx.x, hs = 0;
  if (a.hsplit > 1) {
    const int q = blockIdx.x >> 3;
    hs = q % a.hsplit;
    chunk = (q / a.hsplit) * 8 + (blockIdx.x & 7);
  }
  const int tb = chunk * (W * P);  // first position of the workgroup
  if (chunk >= a.chunks || pos < 0 || pos >= a.pos_limit || tb >= len) return;
  const int t0 = tb + wave * P;         // first position of this wave
  const int nt = max(0, min(P, len - t0));  // 0: an idle wave past the end
  // this workgroup takes query heads h0 .. h0 + G - 1 of the kv head's
  // group (hper per split, the last split fewer)
  const int kvh = blockIdx.y;
  const int h0 = kvh * a.group + hs * a.hper;
  const int G = min(a.hper, a.group - hs * a.hper);
  const int tp = lane % P;        // position of this lane in the wave's chunk
  const int part = lane / P;      // which KD dims of K
  const size_t row_stride = (size_t)a.n_kv * HD;
  const size_t base = ((size_t)a.layer * a.max_seq + min(t0, len - 1)) * row_stride +
                      (size_t)kvh * HD;
  const int last = max(nt - 1, 0);

  // (fused) the RoPE inputs of this thread's first q element, requested
  // ahead of the K / V rows so that q is rotated while they are in flight
  float qx0 = 0.0f, qx1 = 0.0f, qc = 0.0f, qsn = 0.0f;
  bool qfirst = true;
  const bool qlive = FUSED && (int)threadIdx.x < GMAX * HD && (int)threadIdx.x / HD < G;
  if constexpr (FUSED) {
    if (qlive) {
      constexpr int H = HD / 2;
      const int g = threadIdx.x / HD, d = threadIdx.x - g * HD;
      const float* x = a.q + (size_t)qrow * a.q_stride + (size_t)(h0 + g) * HD;
      const int ii = a.neox ? (d < H ? d : d - H) : (d >> 1);
      qfirst = a.neox ? d < H : (d & 1) == 0;
      qc = a.rope_cs[ii];
      qsn = a.rope_cs[H + ii];
      qx0 = qfirst ? x[d] : x[a.neox ? d - H : d - 1];
      qx1 = qfirst ? x[a.neox ? d + H : d + 1] : x[d];
    }
  }
  // every load of the chunk first: K piece, V columns, the group's q
  const f4_t* kr = (const f4_t*)(a.keys + base + (size_t)min(tp, last) * row_stride + part * KD);
  f4_t kreg[KF];
#pragma unroll
  for (int i = 0; i < KF; ++i) kreg[i] = kr[i];
  float vreg[P][VJ];
  const float* vnew = FUSED ? a.v_new + (size_t)kvh * HD : nullptr;
#pragma unroll
  for (int t = 0; t < P; ++t) {
    // (fused: the current position's row is not in the cache yet; rows past
    // it only feed weights of zero and read the current row too)
    const float* vrow = FUSED && t0 + t >= pos ? vnew
                                               : a.values + base + (size_t)min(t, last) * row_stride;
#pragma unroll
    for (int j = 0; j < VJ; ++j) vreg[t][j] = vrow[j * 64 + lane];
  }
  // q of the group's heads; heads G..GMAX-1 are zero so every head loop
  // below runs a fixed GMAX times with no per-head branches (their results
  // are never stored), which lets the heads' reductions interleave
  if constexpr (FUSED) {
    const float* qraw = a.q + (size_t)qrow * a.q_stride + (size_t)h0 * HD;
    float* qf = (float*)qs;
    if ((int)threadIdx.x < GMAX * HD)
      qf[threadIdx.x] = qlive ? (qfirst ? qx0 * qc - qx1 * qsn : qx0 * qsn + qx1 * qc) : 0.0f;
    for (int i = threadIdx.x + W * 64; i < GMAX * HD; i += W * 64) {
      const int g = i / HD;
      qf[i] = g < G ? rope_elem<HD>(qraw + (size_t)g * HD, i - g * HD, a.neox, a.rope_cs) : 0.0f;
    }
    if (t0 + tp == pos) {  // this lane's piece of the current key, rotated
      const float* kraw = a.k_new + (size_t)kvh * HD;
#pragma unroll
      for (int i = 0; i < KF; ++i) {
        const int d = part * KD + 4 * i;
        kreg[i] = f4_t{rope_elem<HD>(kraw, d, a.neox, a.rope_cs),
                       rope_elem<HD>(kraw, d + 1, a.neox, a.rope_cs),
                       rope_elem<HD>(kraw, d + 2, a.neox, a.rope_cs),
                       rope_elem<HD>(kraw, d + 3, a.neox, a.rope_cs)};
      }
    }
    if (hs == 0 && tb + W * P > pos) {  // the workgroup holding pos: write the cache row
      const int d = threadIdx.x;
      const size_t row = (((size_t)a.layer * a.max_seq + pos) * a.n_kv + kvh) * HD;
      if (d < HD) {
        a.kc[row + d] = rope_elem<HD>(a.k_new + (size_t)kvh * HD, d, a.neox, a.rope_cs);
        a.vc[row + d] = vnew[d];
      }
    }
  } else {
    const f4_t* q4 = (const f4_t*)(a.q + (size_t)qrow * a.q_stride + (size_t)h0 * HD);
    for (int i = threadIdx.x; i < GMAX * HD / 4; i += W * 64)
      qs[i] = i < G * HD / 4 ? q4[i] : f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __syncthreads();

  // scores: this lane's KD dims, then the L parts summed across lanes
  float s[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    s[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < KF; ++i) {
      const f4_t qv = qs[(g * HD + part * KD) / 4 + i];
      s[g] += qv.x * kreg[i].x;
      s[g] += qv.y * kreg[i].y;
      s[g] += qv.z * kreg[i].z;
      s[g] += qv.w * kreg[i].w;
    }
  }
  // (lanes p, p + P, p + 2P, ... hold the parts of position p: xor steps P
  // .. 32, the ones within a row as DPP, across rows as lane swaps)
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
#pragma unroll
    for (int off = P; off < 8; off <<= 1) s[g] += __shfl_xor(s[g], off);
    if constexpr (P <= 8) s[g] += dpp<kDppRor8>(s[g]);
    if constexpr (P <= 16) s[g] = xor16_sum(s[g]);
    s[g] = xor32_sum(s[g]);
  }
  // every part holds the full score now: reduce over the P positions only
  // (P lanes of a 16-lane row, or two rows when P = 32)
  const bool valid = tp < nt;
  float m[GMAX], l[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    const float sc = valid ? s[g] * a.scale : -INFINITY;
    m[g] = row_max<P>(sc);  // an idle wave keeps m = -inf: it adds nothing below
    s[g] = valid ? expf(sc - m[g]) : 0.0f;
    l[g] = row_sum<P>(s[g]);
  }
  if (part == 0) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) ps[wave][g * P + tp] = s[g];
  }
  __syncthreads();

  // acc[g][j] = sum_t p[g][t] * V[t][lane + 64 j], positions in order
  float acc[GMAX][VJ];
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int j = 0; j < VJ; ++j) acc[g][j] = 0.0f;
#pragma unroll
  for (int t = 0; t < P; t += 4) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      const f4_t p4 = *(const f4_t*)&ps[wave][g * P + t];
#pragma unroll
      for (int j = 0; j < VJ; ++j) {
        acc[g][j] += p4.x * vreg[t][j];
        acc[g][j] += p4.y * vreg[t + 1][j];
        acc[g][j] += p4.z * vreg[t + 2][j];
        acc[g][j] += p4.w * vreg[t + 3][j];
      }
    }
  }
  // the workgroup's W wave partials merged in wave order into one
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      if (lane == 0) {
        wm[wave][g] = m[g];
        wl[wave][g] = l[g];
      }
#pragma unroll
      for (int j = 0; j < VJ; ++j) wacc[wave][g][j * 64 + lane] = acc[g][j];
    }
  }
  __syncthreads();
  const Partials pp = partials_of(a, qrow);
  float* pm = pp.m;
  float* pl = pp.l;
  float* pa = pp.acc;
  for (int g = wave; g < G; g += W) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, wm[w][g]);
    float f[W];
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      f[w] = wm[w][g] == -INFINITY ? 0.0f : expf(wm[w][g] - mx);
      sum += wl[w][g] * f[w];
    }
    const size_t slot = (size_t)(h0 + g) * a.chunks + chunk;
    if (lane == 0) {
      pm[slot] = mx;
      pl[slot] = sum;
    }
#pragma unroll
    for (int j = 0; j < VJ; ++j) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) v += wacc[w][g][j * 64 + lane] * f[w];
      pa[slot * HD + j * 64 + lane] = v;
    }
  }
}

// ---- prefill attention (many query rows) -----------------------------------------------
// Causal attention of query rows pos0 + r (r < rows) on fp32 MFMA
// (v_mfma_f32_16x16x4f32: exact fp32 products). A workgroup owns one tile of
// 16 (query row, head) pairs that read the same kv head: QT = 16 / GP rows
// times GP heads (the group padded to a power of two; padding heads are zero
// and never stored). Its W waves split the tile's key chunks (16 keys;
// wave w takes chunks w, w + W, ...) so the causal triangle's long rows do
// not serialise on one wave, and merge their (max, sum, acc) in LDS at the
// end. Per chunk a wave:
//   stages K (float4 loads, next chunk loaded ahead) into its LDS slab;
//   S = Q K^T: HD/4 MFMA steps in four independent chains, A = q
//   (registers), B = K (LDS float4 reads: the k index of step st is head dim
//   (lane / 16) * HD/4 + st, contiguous per lane);
//   scales, masks (key <= row position), online softmax per row (a D-layout
//   row lives in one 16-lane DPP row);
//   O += P V: P through LDS into the A layout, B = V straight from the
//   cache (L2-hot; loaded ahead with K at head_dim <= 128), HD/16 tiles x 4.
// MFMA layouts (16x16x4 f32): A[i][k] from lane i + 16k, B[k][j] from lane
// j + 16k, D[4*(l/16) + r][l % 16] in register r of lane l.
__host__ __device__ constexpr int prefill_waves(int hd) { return hd == 256 ? 2 : 4; }

template <int HD, int GP>
__global__ __launch_bounds__(prefill_waves(HD) * 64) void attn_prefill_kernel(AttnArgs a) {
  constexpr int W = prefill_waves(HD);
  constexpr int QT = 16 / GP;   // query rows per tile
  constexpr int KC = 16;        // keys per chunk
  constexpr int NT = HD / 16;   // output tiles
  constexpr int KS = HD + 4;    // padded LDS row of K (16-byte aligned)
  constexpr int KF4 = KC * HD / 4 / 64;  // float4 of a K chunk per lane
  constexpr bool VPRE = HD <= 128;       // V of the next chunk loaded ahead
  // LDS row strides chosen so the 64 lanes of a wave hit distinct banks:
  // P rows 4q + i (q = lane / 16) start 16 banks apart (20 floats), merge
  // rows likewise (HD + 4)
  constexpr int PS = 20;                           // P row stride (floats)
  constexpr int MS = HD + 4;                       // merge row stride (floats)
  constexpr int SLAB = KC * KS + 16 * PS;          // per wave: K chunk + P
  constexpr int MERGE = W * (16 * MS + 32);        // partial acc + max / sum
  constexpr int LDSF = W * SLAB > MERGE ? W * SLAB : MERGE;
  __shared__ __align__(16) float lds[LDSF];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int kvh = blockIdx.y;
  const int G = a.group;
  const int r0 = blockIdx.x * QT;  // first query row of the tile
  const int pos0 = a.pos;
  const int last_row = min(r0 + QT, a.rows) - 1;
  const int kmax = pos0 + last_row;  // last key any row of the tile sees
  const int nchunks = kmax / KC + 1;
  const size_t row_stride = (size_t)a.n_kv * HD;
  const size_t cbase = (size_t)a.layer * a.max_seq * row_stride + (size_t)kvh * HD;
  // K / V rows 0 .. kmax of this kv head through buffer resources (32-bit
  // offsets, checked on the host): rows past kmax read as zeros, so no load
  // needs a clamp (their scores are masked and their weights are zero)
  const uint32_t rs4 = (uint32_t)row_stride * 4u;  // bytes per position
  const uint32_t kvbytes = (uint32_t)kmax * rs4 + HD * 4u;
  const rsrc_t rk = make_rsrc(a.keys + cbase, kvbytes);
  const rsrc_t rv = make_rsrc(a.values + cbase, kvbytes);
  // softmax in base 2: scores scaled by scale * log2(e), weights 2^(s - m)
  // with the hardware exp2 (v_exp_f32)
  const float sl2 = a.scale * 1.44269504088896341f;
  float* kw = lds + wave * SLAB;
  float* pw = kw + KC * KS;

  const int ai = lane & 15, ak = lane >> 4;
  const int aq = r0 + ai / GP, ag = ai % GP;
  const bool arow = aq < a.rows && ag < G;
  const float* qp = a.q + (size_t)(arow ? aq : 0) * a.q_stride +
                    (size_t)(kvh * G + (arow ? ag : 0)) * HD + ak * (HD / 4);
  f4_t qa[HD / 16];
#pragma unroll
  for (int s4 = 0; s4 < HD / 16; ++s4)
    qa[s4] = arow ? *(const f4_t*)(qp + 4 * s4) : f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // D-layout rows of this lane: 4 * (lane / 16) + i
  int dq[4], dpos[4];
  bool dvalid[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * (lane >> 4) + i;
    dq[i] = r0 + m / GP;
    dvalid[i] = dq[i] < a.rows && (m % GP) < G;
    dpos[i] = pos0 + dq[i];
  }
  float mrow[4], lrow[4];
  f4_t acc[NT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mrow[i] = -INFINITY;
    lrow[i] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // element f = lane + 64 u of the chunk: key f / (HD/4), float4 f % (HD/4)
  constexpr int kKeysPerLoad = 256 / HD;  // keys covered by one 64-lane load
  auto load_k = [&](int k0, f4_t* kr) {
    const uint32_t voff = (uint32_t)(k0 + lane / (HD / 4)) * rs4 + (uint32_t)(lane % (HD / 4)) * 16u;
#pragma unroll
    for (int u = 0; u < KF4; ++u)
      kr[u] = __builtin_bit_cast(f4_t, buf_load16(rk, voff + (uint32_t)(u * kKeysPerLoad) * rs4, 0));
  };
  // B operand of P V: V[k0 + 4 st + ak][16 t + lane % 16]
  auto load_v = [&](int k0, float* vr) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const uint32_t voff = (uint32_t)(k0 + 4 * st + ak) * rs4 + (uint32_t)(lane & 15) * 4u;
#pragma unroll
      for (int t = 0; t < NT; ++t)
        vr[t * 4 + st] = __builtin_bit_cast(float, buf_load4(rv, voff + 64u * t, 0));
    }
  };
  f4_t kn[KF4];
  float vn[VPRE ? NT * 4 : 1];
  if (wave < nchunks) {
    load_k(wave * KC, kn);
    if constexpr (VPRE) load_v(wave * KC, vn);
  }
  for (int c = wave; c < nchunks; c += W) {
    const int k0 = c * KC;
#pragma unroll
    for (int u = 0; u < KF4; ++u) {
      const int f = lane + 64 * u;
      const int key = f / (HD / 4);
      const int c4 = f - key * (HD / 4);
      *(f4_t*)(kw + key * KS + 4 * c4) = kn[u];
    }
    float vc[NT * 4];
    if constexpr (VPRE) {
#pragma unroll
      for (int e = 0; e < NT * 4; ++e) vc[e] = vn[e];
    }
    if (c + W < nchunks) {
      load_k(k0 + W * KC, kn);
      if constexpr (VPRE) load_v(k0 + W * KC, vn);
    }
    if constexpr (!VPRE) load_v(k0, vc);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes landed
    __builtin_amdgcn_wave_barrier();

    // S = Q K^T for keys k0 .. k0 + 15: four independent accumulator chains
    f4_t sc4[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) sc4[q] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const float* krow = kw + (lane & 15) * KS + ak * (HD / 4);
#pragma unroll
    for (int s4 = 0; s4 < HD / 16; ++s4) {
      const f4_t b4 = *(const f4_t*)(krow + 4 * s4);
      sc4[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s4].x, b4.x, sc4[0], 0, 0, 0);
      sc4[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s4].y, b4.y, sc4[1], 0, 0, 0);
      sc4[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s4].z, b4.z, sc4[2], 0, 0, 0);
      sc4[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s4].w, b4.w, sc4[3], 0, 0, 0);
    }
    const f4_t sacc = (sc4[0] + sc4[1]) + (sc4[2] + sc4[3]);
    const int key = k0 + (lane & 15);
    float pr[4], al[4];
    bool rescale = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = dvalid[i] && key <= dpos[i];
      const float sc = ok ? sacc[i] * sl2 : -INFINITY;
      const float mx = fmaxf(mrow[i], row_max<16>(sc));
      // rows with nothing visible yet keep m = -inf and weight 0
      const float alpha = mx == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(mrow[i] - mx);
      const float p = ok ? __builtin_amdgcn_exp2f(sc - mx) : 0.0f;
      lrow[i] = lrow[i] * alpha + row_sum<16>(p);
      mrow[i] = mx;
      pr[i] = p;
      al[i] = alpha;
      rescale |= alpha != 1.0f;
    }
    // the accumulators (MFMA registers) are rescaled only when some row's
    // maximum moved in this chunk (exactly 1 otherwise)
    if (__any(rescale)) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][i] *= al[i];
    }
    // P (D layout) -> LDS -> A layout
#pragma unroll
    for (int i = 0; i < 4; ++i) pw[(4 * (lane >> 4) + i) * PS + (lane & 15)] = pr[i];
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    float pa[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) pa[st] = pw[(lane & 15) * PS + 4 * st + ak];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int st = 0; st < 4; ++st)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[st], vc[t * 4 + st], acc[t], 0, 0, 0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // reads of this chunk done before the next writes
    __builtin_amdgcn_wave_barrier();
  }

  // merge the W waves' partials of every row (wave order), then store
  __syncthreads();  // every wave is done with its slab: the merge area reuses it
  float* macc = lds;                       // [W][16][MS]
  float* mml = lds + W * 16 * MS;          // [W][16] max, then [W][16] sum
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * (lane >> 4) + i;
#pragma unroll
    for (int t = 0; t < NT; ++t) macc[(wave * 16 + m) * MS + 16 * t + (lane & 15)] = acc[t][i];
    if ((lane & 15) == 0) {
      mml[wave * 16 + m] = mrow[i];
      mml[W * 16 + wave * 16 + m] = lrow[i];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 16 * HD; e += W * 64) {
    const int m = e / HD;
    const int d = e - m * HD;
    const int qr = r0 + m / GP;
    if (qr >= a.rows || (m % GP) >= G) continue;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, mml[w * 16 + m]);
    float lsum = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float mw = mml[w * 16 + m];
      const float f = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mx);
      lsum += mml[W * 16 + w * 16 + m] * f;
      o += macc[(w * 16 + m) * MS + d] * f;
    }
    const size_t at = (size_t)qr * a.out_stride + (size_t)(kvh * G + m % GP) * HD + d;
    a.out[at] = o / lsum;
  }
}

// Pass 2, per (query head, query row): four waves each take 16 chunks of a
// 64-chunk pass. The partials' addresses do not depend on the position, so
// the first pass requests every maximum, sum and accumulator (in bounds:
// chunks < a.chunks) together with the device position: one memory round
// trip instead of four dependent ones. Chunks past the live range are
// masked by selects after the loads (stale partials never enter a product).
// Each wave rescales its chunks to its own maximum in chunk order; the four
// waves then merge through LDS in wave order, and passes in pass order
// (deterministic).
constexpr int kCombineWaves = 4;
constexpr int kCombineCpw = 16;  // chunks per wave and pass
constexpr int kCombinePass = kCombineWaves * kCombineCpw;

// KD: head dims per lane (head_dim <= 64 KD)
template <int KD>
__global__ __launch_bounds__(kCombineWaves * 64) void attn_combine_kernel(AttnArgs a) {
  constexpr int kD = KD;
  __shared__ float sm[kCombineWaves], sl[kCombineWaves];
  __shared__ float sacc[kCombineWaves][kAttnMaxHd];
  const int qrow = blockIdx.y;
  const int head = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const Partials pp = partials_of(a, qrow);
  const float* pm = pp.m + (size_t)head * a.chunks;
  const float* pl = pp.l + (size_t)head * a.chunks;
  const float* pa = pp.acc + (size_t)head * a.chunks * a.hd;
  float* out = a.out + (size_t)qrow * a.out_stride + (size_t)head * a.hd;

  // one pass: this wave's chunks c0 + 16 wave + i; returns the wave's
  // (max, sum, acc) rescaled to that max (m = -inf: nothing live)
  float gm = -INFINITY, gl = 0.0f;  // running over passes (every thread)
  float gacc[kD];
#pragma unroll
  for (int j = 0; j < kD; ++j) gacc[j] = 0.0f;
  int live = 0;  // live chunks (set once the position is known)
  auto pass = [&](int c0, auto first_c) __attribute__((always_inline)) {
    constexpr bool FIRST = decltype(first_c)::value;
    const int cw = c0 + wave * kCombineCpw;
    float m[kCombineCpw], l[kCombineCpw], v[kCombineCpw][kD];
#pragma unroll
    for (int i = 0; i < kCombineCpw; ++i) {
      const int c = min(cw + i, a.chunks - 1);  // in bounds; masked below
      m[i] = pm[c];
      l[i] = pl[c];
#pragma unroll
      for (int j = 0; j < kD; ++j) {
        const int d = min(lane + 64 * j, a.hd - 1);
        v[i][j] = pa[(size_t)c * a.hd + d];
      }
    }
    if constexpr (FIRST) {
      const int pos = read_scalar(a.pos_dev, a.pos) + qrow;
      live = pos < 0 || pos >= a.pos_limit ? -1 : (pos + a.chunk_len) / a.chunk_len;
    }
    if (live < 0) return;
    float wmx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kCombineCpw; ++i) {
      m[i] = cw + i < live ? m[i] : -INFINITY;
      wmx = fmaxf(wmx, m[i]);
    }
    float wl = 0.0f, wacc[kD];
#pragma unroll
    for (int j = 0; j < kD; ++j) wacc[j] = 0.0f;
    if (wmx != -INFINITY) {
#pragma unroll
      for (int i = 0; i < kCombineCpw; ++i) {
        const float f = m[i] == -INFINITY ? 0.0f : expf(m[i] - wmx);
        wl += (cw + i < live ? l[i] : 0.0f) * f;
#pragma unroll
        for (int j = 0; j < kD; ++j) wacc[j] += (cw + i < live ? v[i][j] : 0.0f) * f;
      }
    }
    // the four waves merged in wave order, then into the running result
    __syncthreads();  // (a previous pass's readers are done with the LDS)
    if (lane == 0) {
      sm[wave] = wmx;
      sl[wave] = wl;
    }
#pragma unroll
    for (int j = 0; j < kD; ++j) sacc[wave][lane + 64 * j] = wacc[j];
    __syncthreads();
    float pmx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kCombineWaves; ++w) pmx = fmaxf(pmx, sm[w]);
    const float nm = fmaxf(gm, pmx);
    if (nm == -INFINITY) return;  // nothing live yet (uniform)
    const float fo = gm == -INFINITY ? 0.0f : expf(gm - nm);
    gl *= fo;
#pragma unroll
    for (int j = 0; j < kD; ++j) gacc[j] *= fo;
#pragma unroll
    for (int w = 0; w < kCombineWaves; ++w) {
      const float f = sm[w] == -INFINITY ? 0.0f : expf(sm[w] - nm);
      gl += sl[w] * f;
#pragma unroll
      for (int j = 0; j < kD; ++j) gacc[j] += sacc[w][lane + 64 * j] * f;
    }
    gm = nm;
  };
  pass(0, std::true_type{});
  if (live < 0) {  // only reachable through a device position
    if (wave == 0)
      for (int d = lane; d < a.hd; d += 64) out[d] = __builtin_nanf("");
    return;
  }
  for (int c0 = kCombinePass; c0 < live; c0 += kCombinePass) pass(c0, std::false_type{});
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < kD; ++j) {
      const int d = lane + 64 * j;
      if (d < a.hd) out[d] = gacc[j] / gl;
    }
  }
}

// ---- greedy argmax ----------------------------------------------------------------
// argMax (src/ops.cc:230-246): index of the first maximum, comparisons with
// '>' so NaN entries never win, and index 0 when x[0] is NaN. One workgroup;
// each thread scans a strided slice in increasing index order, then the
// (value, index) pairs merge with ties going to the lower index. Optionally
// stores the result as the next token and advances the device position.
constexpr int kArgmaxThreads = 1024;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ x,
                                                                 int64_t n, int32_t* out,
                                                                 int32_t* pos_dev) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int64_t si[kArgmaxThreads / 64];
  float best = -INFINITY;
  int64_t idx = INT64_MAX;
  constexpr int kU = 8;  // independent loads in flight per thread
  for (int64_t b = 0; b < n; b += (int64_t)kArgmaxThreads * kU) {
    float v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = b + threadIdx.x + (int64_t)u * kArgmaxThreads;
      v[u] = i < n ? x[i] : __builtin_nanf("");
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = b + threadIdx.x + (int64_t)u * kArgmaxThreads;
      if (v[u] > best || (idx == INT64_MAX && v[u] == best)) {
        best = v[u];
        idx = i;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int64_t oi = __shfl_xor(idx, off);
    if (ov > best || (ov == best && oi < idx)) {
      best = ov;
      idx = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w) {
      if (sv[w] > best || (sv[w] == best && si[w] < idx)) {
        best = sv[w];
        idx = si[w];
      }
    }
    // x[0] NaN: the reference never replaces it; all-NaN slices: idx unset
    if (isnan(x[0]) || idx == INT64_MAX) idx = 0;
    *out = (int32_t)idx;
    if (pos_dev != nullptr) *pos_dev += 1;
  }
}

// Two-pass form for long vectors (the vocabulary): pass 1 gives each
// workgroup kArgmaxSlice consecutive elements (16 independent loads per
// thread), pass 2 merges the per-workgroup (value, index) pairs in order.
constexpr int kArgmaxSliceThreads = 256;
constexpr int kArgmaxPerThread = 16;
constexpr int kArgmaxSlice = kArgmaxSliceThreads * kArgmaxPerThread;

__device__ __forceinline__ void argmax_merge(float& best, int64_t& idx, float ov, int64_t oi) {
  if (ov > best || (ov == best && oi < idx)) {
    best = ov;
    idx = oi;
  }
}

template <int NT>
__device__ __forceinline__ void argmax_block(float& best, int64_t& idx) {
  __shared__ float sv[NT / 64];
  __shared__ int64_t si[NT / 64];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    argmax_merge(best, idx, __shfl_xor(best, off), __shfl_xor(idx, off));
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = best;
    si[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < NT / 64; ++w) argmax_merge(best, idx, sv[w], si[w]);
}

__global__ __launch_bounds__(kArgmaxSliceThreads) void argmax_partial_kernel(
    const float* __restrict__ x, int64_t n, float* pv, int64_t* pi) {
  const int64_t b0 = (int64_t)blockIdx.x * kArgmaxSlice;
  float v[kArgmaxPerThread];
#pragma unroll
  for (int u = 0; u < kArgmaxPerThread; ++u) {
    const int64_t i = b0 + threadIdx.x + (int64_t)u * kArgmaxSliceThreads;
    v[u] = i < n ? x[i] : __builtin_nanf("");
  }
  float best = -INFINITY;
  int64_t idx = INT64_MAX;
#pragma unroll
  for (int u = 0; u < kArgmaxPerThread; ++u) {
    const int64_t i = b0 + threadIdx.x + (int64_t)u * kArgmaxSliceThreads;
    if (v[u] > best || (idx == INT64_MAX && v[u] == best)) {
      best = v[u];
      idx = i;
    }
  }
  argmax_block<kArgmaxSliceThreads>(best, idx);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = best;
    pi[blockIdx.x] = idx;
  }
}

__global__ __launch_bounds__(kArgmaxSliceThreads) void argmax_final_kernel(
    const float* __restrict__ pv, const int64_t* __restrict__ pi, int parts,
    const float* __restrict__ x, int32_t* out, int32_t* pos_dev) {
  float best = -INFINITY;
  int64_t idx = INT64_MAX;
  for (int b = threadIdx.x; b < parts; b += kArgmaxSliceThreads) argmax_merge(best, idx, pv[b], pi[b]);
  argmax_block<kArgmaxSliceThreads>(best, idx);
  if (threadIdx.x == 0) {
    if (isnan(x[0]) || idx == INT64_MAX) idx = 0;
    *out = (int32_t)idx;
    if (pos_dev != nullptr) *pos_dev += 1;
  }
}

// rmsnorm_vec_kernel with fp16 output rows of ld halves (zero past dim):
// row r holds y * 2^rexp[r], rexp[r] = pow2_scale_exp(max |y|) (any finite
// row fits fp16; the GEMM reading the copy scales its results back).
template <int R>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_f16_kernel(
    const float* __restrict__ x, const float* __restrict__ w,
    _Float16* __restrict__ yh, int* __restrict__ rexp, int dim, int ld, float eps) {
  __shared__ float part[kNormThreads / 64];
  __shared__ float pmax[kNormThreads / 64];
  const int n4 = dim >> 2;
  const f4_t* xr = (const f4_t*)(x + (size_t)blockIdx.x * dim);
  uint2* yr = (uint2*)(yh + (size_t)blockIdx.x * ld);
  const f4_t* w4 = (const f4_t*)w;
  f4_t v[R], wv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = threadIdx.x + r * kNormThreads;
    v[r] = i < n4 ? xr[i] : f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    wv[r] = i < n4 ? w4[i] : f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  float ss = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    ss += v[r].x * v[r].x;
    ss += v[r].y * v[r].y;
    ss += v[r].z * v[r].z;
    ss += v[r].w * v[r].w;
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) total += part[i];
  const float scale = sqrtf(total / (float)dim + eps);
  // the normalised row, its largest magnitude, and the row's power-of-two
  // scale for the fp16 copy (pow2_scale_exp; the GEMM scales back)
  float mx = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    v[r] = f4_t{v[r].x * wv[r].x / scale, v[r].y * wv[r].y / scale,
                v[r].z * wv[r].z / scale, v[r].w * wv[r].w / scale};
    mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v[r].x), fabsf(v[r].y))), fmaxf(fabsf(v[r].z), fabsf(v[r].w)));
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) pmax[threadIdx.x >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) mx = fmaxf(mx, pmax[i]);
  const int e = pow2_scale_exp(mx);
  if (threadIdx.x == 0) rexp[blockIdx.x] = e;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = threadIdx.x + r * kNormThreads;
    if (i < n4) {
      uint2 o;
      o.x = pack_h2(ldexp_f(v[r].x, e), ldexp_f(v[r].y, e));
      o.y = pack_h2(ldexp_f(v[r].z, e), ldexp_f(v[r].w, e));
      yr[i] = o;
    }
  }
  for (int i = n4 + threadIdx.x; i < (ld >> 2); i += kNormThreads) yr[i] = make_uint2(0u, 0u);
}

__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

// ---- launchers ---------------------------------------------------------------------
hipError_t launch_rmsnorm_f16(const float* x, const float* w, _Float16* yh, int* rexp, int rows,
                              int dim, int ld, float eps, hipStream_t stream) {
  const bool ok = dim % 4 == 0 && ld % 4 == 0 && ld >= dim && ((uintptr_t)x & 15) == 0 &&
                  ((uintptr_t)w & 15) == 0 && ((uintptr_t)yh & 15) == 0;
  const int per = (dim / 4 + kNormThreads - 1) / kNormThreads;
  if (!ok || per > 16) return hipErrorInvalidValue;
  const dim3 grid(rows), block(kNormThreads);
  if (per <= 1) hipLaunchKernelGGL(rmsnorm_f16_kernel<1>, grid, block, 0, stream, x, w, yh, rexp, dim, ld, eps);
  else if (per <= 2) hipLaunchKernelGGL(rmsnorm_f16_kernel<2>, grid, block, 0, stream, x, w, yh, rexp, dim, ld, eps);
  else if (per <= 4) hipLaunchKernelGGL(rmsnorm_f16_kernel<4>, grid, block, 0, stream, x, w, yh, rexp, dim, ld, eps);
  else if (per <= 8) hipLaunchKernelGGL(rmsnorm_f16_kernel<8>, grid, block, 0, stream, x, w, yh, rexp, dim, ld, eps);
  else hipLaunchKernelGGL(rmsnorm_f16_kernel<16>, grid, block, 0, stream, x, w, yh, rexp, dim, ld, eps);
  return hipGetLastError();
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
  const size_t n = bytes / 4;
  if (n == 0) return hipSuccess;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  fill_zero_kernel<<<blocks, 256, 0, stream>>>((uint32_t*)p, n);
  return hipGetLastError();
}
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int dim,
                          float eps, hipStream_t stream) {
  const bool vec = dim % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
                   ((uintptr_t)y & 15) == 0;
  const int per = (dim / 4 + kNormThreads - 1) / kNormThreads;  // float4 per thread
  const dim3 grid(rows), block(kNormThreads);
  if (vec && per <= 1) hipLaunchKernelGGL(rmsnorm_vec_kernel<1>, grid, block, 0, stream, x, w, y, dim, eps);
  else if (vec && per <= 2) hipLaunchKernelGGL(rmsnorm_vec_kernel<2>, grid, block, 0, stream, x, w, y, dim, eps);
  else if (vec && per <= 4) hipLaunchKernelGGL(rmsnorm_vec_kernel<4>, grid, block, 0, stream, x, w, y, dim, eps);
  else if (vec && per <= 8) hipLaunchKernelGGL(rmsnorm_vec_kernel<8>, grid, block, 0, stream, x, w, y, dim, eps);
  else if (vec && per <= 16) hipLaunchKernelGGL(rmsnorm_vec_kernel<16>, grid, block, 0, stream, x, w, y, dim, eps);
  else hipLaunchKernelGGL(rmsnorm_kernel, grid, block, 0, stream, x, w, y, dim, eps);
  return hipGetLastError();
}

static int eltwise_blocks(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (int)(b < 4096 ? b : 4096);
}

hipError_t launch_eltwise(int op, const float* a, const float* b, float* y, int64_t n,
                          hipStream_t stream) {
  const dim3 grid(eltwise_blocks(n)), block(256);
  switch (op) {
    case kEltAdd: hipLaunchKernelGGL(eltwise_kernel<kEltAdd>, grid, block, 0, stream, a, b, y, n); break;
    case kEltMul: hipLaunchKernelGGL(eltwise_kernel<kEltMul>, grid, block, 0, stream, a, b, y, n); break;
    case kEltSilu: hipLaunchKernelGGL(eltwise_kernel<kEltSilu>, grid, block, 0, stream, a, b, y, n); break;
    case kEltSwiGLU: hipLaunchKernelGGL(eltwise_kernel<kEltSwiGLU>, grid, block, 0, stream, a, b, y, n); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_softmax(const float* x, float* y, int64_t n, hipStream_t stream) {
  hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(kSoftmaxThreads), 0, stream, x, y, n);
  return hipGetLastError();
}

hipError_t launch_embedding(const float* table, int vocab, int dim, const int32_t* token_dev,
                            int token, float* y, hipStream_t stream, const RopeTable& rt,
                            const NormInput& ni) {
  const int blocks = (dim + 255) / 256;
  hipLaunchKernelGGL(embed_kernel, dim3(blocks), dim3(256), 0, stream, table, vocab, dim,
                     token_dev, token, y, rt.cs, rt.pos_dev, rt.pos, rt.hd, rt.theta, ni);
  return hipGetLastError();
}

hipError_t launch_rope(const RopeLaunch& r, hipStream_t stream) {
  RopeArgs a;
  a.q = r.q;
  a.k = r.k;
  a.v = r.v;
  a.keys = r.keys;
  a.values = r.values;
  a.n_heads = r.n_heads;
  a.n_kv = r.n_kv;
  a.hd = r.hd;
  a.neox = r.neox;
  a.layer = r.layer;
  a.max_seq = r.max_seq;
  a.pos_limit = r.pos_limit > 0 ? std::min(r.pos_limit, r.max_seq) : r.max_seq;
  a.pos_dev = r.pos_dev;
  a.pos = r.pos;
  a.theta = r.theta;
  const int total = (r.n_heads + r.n_kv) * (r.hd / 2);
  hipLaunchKernelGGL(rope_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_rope_rows(const RopeRows& rr, hipStream_t stream) {
  RopeRowsArgs a;
  a.q = rr.q;
  a.k = rr.k;
  a.v = rr.v;
  a.q_stride = rr.q_stride;
  a.k_stride = rr.k_stride;
  a.v_stride = rr.v_stride;
  a.rows = rr.rows;
  a.keys = rr.keys;
  a.values = rr.values;
  a.n_heads = rr.n_heads;
  a.n_kv = rr.n_kv;
  a.hd = rr.hd;
  a.neox = rr.neox;
  a.layer = rr.layer;
  a.max_seq = rr.max_seq;
  a.pos0 = rr.pos0;
  a.theta = rr.theta;
  a.cs = rr.cs;
  const int per_row = (rr.n_heads + rr.n_kv) * (rr.hd / 2);
  hipLaunchKernelGGL(rope_rows_kernel, dim3((per_row + 255) / 256, rr.rows), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

hipError_t launch_rope_table(float* cs, int rows, int pos0, int hd, float theta,
                             hipStream_t stream) {
  if (rows <= 0 || hd <= 0 || (hd & 1) != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rope_table_kernel, dim3((hd / 2 + 255) / 256, rows), dim3(256), 0, stream, cs,
                     rows, pos0, hd, theta);
  return hipGetLastError();
}

hipError_t launch_embedding_rows(const float* table, int dim, const int32_t* tokens, int rows,
                                 float* y, hipStream_t stream) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3((dim + 255) / 256, rows), dim3(256), 0, stream,
                     table, dim, tokens, y);
  return hipGetLastError();
}

hipError_t launch_kv_write(float* keys, float* values, const float* k, const float* v,
                           size_t row, int n, hipStream_t stream) {
  hipLaunchKernelGGL(kv_write_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, keys,
                     values, k, v, row, n);
  return hipGetLastError();
}

// Chunk count the workspace is sized for: the shorter chunk of the two
// kernels a head dim can take (the register kernel needs aligned buffers).
int attention_chunks(int hd, int max_len) {
  const int ch = attn_reg_hd(hd) ? min(attn_reg_chunk(hd), kAttnLdsChunk) : kAttnLdsChunk;
  return (max_len + ch - 1) / ch;
}

size_t attention_workspace_bytes(int n_heads, int hd, int max_len, int rows) {
  const size_t c = (size_t)attention_chunks(hd, max_len);
  return (size_t)rows * ((size_t)n_heads * c * (2 + (size_t)hd)) * sizeof(float);
}

// The register kernel (and so the fused RoPE + cache write) covers head
// dims 64 / 128 / 256, except head_dim 64 with more than 8 query heads per
// kv head, which would spill.
bool attention_fusable(int hd, int group) {
  return attn_reg_hd(hd) && !(hd == 64 && group > 8);
}

bool attention_supported(int n_heads, int n_kv, int hd) {
  return n_kv > 0 && n_heads % n_kv == 0 && n_heads / n_kv <= kAttnMaxGroup && hd > 0 &&
         hd <= kAttnMaxHd;
}

template <int HD, int GMAX>
static void attn_launch(const AttnArgs& a, hipStream_t stream) {
  if constexpr (HD != 0) {
    const int gx = a.hsplit > 1 ? (a.chunks + 7) / 8 * 8 * a.hsplit : a.chunks;
    if (a.rope_cs != nullptr)
      hipLaunchKernelGGL((attn_reg_kernel<HD, GMAX, true>), dim3(gx, a.n_kv, a.rows),
                         dim3(kAttnRegWaves * 64), 0, stream, a);
    else
      hipLaunchKernelGGL((attn_reg_kernel<HD, GMAX, false>), dim3(gx, a.n_kv, a.rows),
                         dim3(kAttnRegWaves * 64), 0, stream, a);
  } else {
    constexpr int CH = kAttnLdsChunk;
    const int hdp = (a.hd + 3) & ~3;
    const size_t lds = (size_t)(CH * (hdp + 4) + GMAX * hdp + GMAX * CH) * sizeof(float);
    hipLaunchKernelGGL((attn_chunk_kernel<0, GMAX>), dim3(a.chunks, a.n_kv, a.rows), dim3(64), lds,
                       stream, a);
  }
}

template <int HD>
static void attn_launch_g(const AttnArgs& a, hipStream_t stream) {
  const int h = a.hper;  // query heads per workgroup
  if (h <= 1) attn_launch<HD, 1>(a, stream);
  else if (h <= 2) attn_launch<HD, 2>(a, stream);
  else if (h <= 4) attn_launch<HD, 4>(a, stream);
  else if (h <= 8) attn_launch<HD, 8>(a, stream);
  else if constexpr (HD != 64) attn_launch<HD, 16>(a, stream);
}

// Query-head split of the register kernel: MLQ_ATTN_HSPLIT (read once)
// overrides the rule in launch_attention.
int attn_hsplit_override() {
  static const int v = [] {
    const char* e = std::getenv("MLQ_ATTN_HSPLIT");
    return e ? std::atoi(e) : 0;
  }();
  return v;
}

hipError_t launch_attention(const AttnLaunch& r, hipStream_t stream) {
  AttnArgs a;
  a.q = r.q;
  a.keys = r.keys;
  a.values = r.values;
  a.out = r.out;
  a.part = r.ws;
  a.rows = r.rows;
  a.q_stride = r.q_stride;
  a.out_stride = r.out_stride;
  a.layer = r.layer;
  a.max_seq = r.max_seq;
  a.n_kv = r.n_kv;
  a.hd = r.hd;
  a.group = r.n_heads / r.n_kv;
  a.vec = r.hd % 4 == 0 && ((uintptr_t)r.keys & 15) == 0 && ((uintptr_t)r.values & 15) == 0;
  // (head_dim 64 with more than 8 query heads per kv head would spill the
  // register kernel: it takes the LDS kernel)
  const bool reg = attention_fusable(r.hd, a.group) && a.vec && ((uintptr_t)r.q & 15) == 0;
  a.k_new = r.k_new;
  a.v_new = r.v_new;
  a.rope_cs = r.rope_cs;
  a.kc = const_cast<float*>(r.keys);
  a.vc = const_cast<float*>(r.values);
  a.neox = r.neox;
  if (r.rope_cs != nullptr && !reg) return hipErrorInvalidValue;
  a.chunk_len = reg ? attn_reg_chunk(r.hd) : kAttnLdsChunk;
  a.chunks = (r.max_len + a.chunk_len - 1) / a.chunk_len;
  // a row's combine reads pos / chunk_len + 1 partials: at most `chunks`
  a.pos_limit = std::min(r.max_seq, a.chunks * a.chunk_len);
  if (r.pos_limit > 0) a.pos_limit = std::min(a.pos_limit, r.pos_limit);
  a.pos_dev = r.pos_dev;
  a.pos = r.pos;
  a.scale = sqrtf(1.0f / (float)r.hd);
  // The register kernel is VALU-bound at decode contexts: a grid of
  // chunks x kv heads that leaves most CUs idle runs two query heads per
  // workgroup instead of the whole group (7 -> 2 + 2 + 2 + 1 for Qwen2-7B:
  // 1.530 -> 1.503 ms per decode step; 4 + 3 was slower, 1 per workgroup
  // 1.585). Long caches (chunks x kv heads > 2 x CUs) keep one workgroup per
  // group: there the K/V reads, not the VALU, bound the kernel.
  a.hsplit = 1;
  a.hper = a.group;
  if (reg) {
    int hs = attn_hsplit_override();
    if (hs <= 0)
      hs = a.group >= 3 && (int64_t)a.chunks * a.n_kv <= 2 * (int64_t)device_cus()
               ? (a.group + 1) / 2 : 1;
    if (hs > 1) {
      a.hsplit = std::min(hs, a.group);
      a.hper = (a.group + a.hsplit - 1) / a.hsplit;
      a.hsplit = (a.group + a.hper - 1) / a.hper;  // no empty split
    }
  }
  switch (reg ? r.hd : 0) {
    case 64: attn_launch_g<64>(a, stream); break;
    case 128: attn_launch_g<128>(a, stream); break;
    case 256: attn_launch_g<256>(a, stream); break;
    default: attn_launch_g<0>(a, stream); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 cgrid(r.n_heads, a.rows), cblock(kCombineWaves * 64);
  switch ((r.hd + 63) / 64) {
    case 1: hipLaunchKernelGGL(attn_combine_kernel<1>, cgrid, cblock, 0, stream, a); break;
    case 2: hipLaunchKernelGGL(attn_combine_kernel<2>, cgrid, cblock, 0, stream, a); break;
    case 3: hipLaunchKernelGGL(attn_combine_kernel<3>, cgrid, cblock, 0, stream, a); break;
    default: hipLaunchKernelGGL(attn_combine_kernel<4>, cgrid, cblock, 0, stream, a); break;
  }
  return hipGetLastError();
}

bool prefill_attention_supported(int hd, int group) {
  return (hd == 64 || hd == 128 || hd == 256) && group >= 1 && group <= 16;
}

template <int HD, int GP>
static void prefill_launch(const AttnArgs& a, hipStream_t stream) {
  constexpr int QT = 16 / GP;
  const int tiles = (a.rows + QT - 1) / QT;
  hipLaunchKernelGGL((attn_prefill_kernel<HD, GP>), dim3(tiles, a.n_kv),
                     dim3(prefill_waves(HD) * 64), 0, stream, a);
}

template <int HD>
static void prefill_launch_g(const AttnArgs& a, hipStream_t stream) {
  if (a.group <= 1) prefill_launch<HD, 1>(a, stream);
  else if (a.group <= 2) prefill_launch<HD, 2>(a, stream);
  else if (a.group <= 4) prefill_launch<HD, 4>(a, stream);
  else if (a.group <= 8) prefill_launch<HD, 8>(a, stream);
  else prefill_launch<HD, 16>(a, stream);
}

hipError_t launch_attention_prefill(const AttnLaunch& r, hipStream_t stream) {
  AttnArgs a = {};
  a.q = r.q;
  a.keys = r.keys;
  a.values = r.values;
  a.out = r.out;
  a.layer = r.layer;
  a.max_seq = r.max_seq;
  a.n_kv = r.n_kv;
  a.hd = r.hd;
  a.group = r.n_heads / r.n_kv;
  a.pos = r.pos;
  a.rows = r.rows;
  a.q_stride = r.q_stride;
  a.out_stride = r.out_stride;
  a.scale = sqrtf(1.0f / (float)r.hd);
  if (!prefill_attention_supported(r.hd, a.group) || ((uintptr_t)r.keys & 15) != 0 ||
      ((uintptr_t)r.values & 15) != 0)
    return hipErrorInvalidValue;
  // the kernel addresses one layer's K / V rows with 32-bit byte offsets
  if ((uint64_t)r.max_seq * r.n_kv * r.hd * 4 >= (1ull << 32)) return hipErrorInvalidValue;
  switch (r.hd) {
    case 64: prefill_launch_g<64>(a, stream); break;
    case 128: prefill_launch_g<128>(a, stream); break;
    default: prefill_launch_g<256>(a, stream); break;
  }
  return hipGetLastError();
}

hipError_t launch_argmax(const float* x, int64_t n, int32_t* out, int32_t* pos_dev,
                         hipStream_t stream) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgmaxThreads), 0, stream, x, n, out,
                     pos_dev);
  return hipGetLastError();
}

size_t argmax_workspace_bytes(int64_t n) {
  const size_t parts = (size_t)((n + kArgmaxSlice - 1) / kArgmaxSlice);
  return parts * (sizeof(float) + sizeof(int64_t)) + 16;
}

hipError_t launch_argmax_ws(const float* x, int64_t n, int32_t* out, int32_t* pos_dev,
                            void* ws, hipStream_t stream) {
  const int parts = (int)((n + kArgmaxSlice - 1) / kArgmaxSlice);
  int64_t* pi = (int64_t*)ws;
  float* pv = (float*)(pi + parts);
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(parts), dim3(kArgmaxSliceThreads), 0, stream,
                     x, n, pv, pi);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxSliceThreads), 0, stream, pv, pi,
                     parts, x, out, pos_dev);
  return hipGetLastError();
}

}  // namespace mlq
