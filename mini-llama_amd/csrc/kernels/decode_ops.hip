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
#include <stdint.h>

#include "device_common.h"

namespace mlq {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

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

// ---- embedding ------------------------------------------------------------------
// y = table[token] (embeddingLookupKernel, src/cuda_ops.cu:415-421). A device
// token outside [0, vocab) yields a NaN row instead of a wild read.
__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ table,
                                                    int vocab, int dim,
                                                    const int32_t* token_dev, int token,
                                                    float* __restrict__ y) {
  const int t = read_scalar(token_dev, token);
  const bool ok = t >= 0 && t < vocab;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x)
    y[i] = ok ? table[(size_t)t * dim + i] : __builtin_nanf("");
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
  if (cache && (pos < 0 || pos >= a.max_seq)) return;
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
// Positions per chunk: 64 (one per lane) for head dims up to 128; 32 for
// larger or irregular head dims, which keeps the LDS slab under 64 KiB.
constexpr int kAttnMaxGroup = 16;
constexpr int kAttnMaxHd = 256;
__host__ __device__ constexpr int attn_chunk_len(int hd) {
  return (hd == 64 || hd == 128) ? 64 : 32;
}

struct AttnArgs {
  const float* q;       // [n_heads][hd]
  const float* keys;    // [layers][max_seq][n_kv][hd]
  const float* values;
  float* out;           // [n_heads][hd]
  float* part;          // workspace: m, l [n_heads][chunks]; acc [n_heads][chunks][hd]
  int layer, max_seq, n_kv, hd, group, chunks, chunk_len;
  int vec;              // K/V rows are float4-aligned (hd % 4 == 0, aligned cache)
  const int32_t* pos_dev;
  int pos;
  float scale;
};

template <int HD, int GMAX>
__global__ __launch_bounds__(64) void attn_chunk_kernel(AttnArgs a) {
  constexpr int CH = attn_chunk_len(HD);
  const int hd = HD ? HD : a.hd;
  const int hdp = (hd + 3) & ~3;
  const int stride = hdp + 4;  // padded LDS row: ds_read_b128 by position lanes stays conflict-free
  extern __shared__ float lds[];
  float* rows = lds;                   // [CH][stride]
  float* qs = lds + CH * stride;       // [GMAX][hdp]
  float* ps = qs + GMAX * hdp;         // [GMAX][CH]

  const int pos = read_scalar(a.pos_dev, a.pos);
  const int len = pos + 1;
  const int t0 = blockIdx.x * CH;
  if (pos < 0 || pos >= a.max_seq || t0 >= len) return;
  const int nt = min(CH, len - t0);
  const int kvh = blockIdx.y;
  const int lane = threadIdx.x;
  const int G = a.group;
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
    qs[i] = c < hd ? a.q[(size_t)(kvh * G + g) * hd + c] : 0.0f;
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
  float* pm = a.part;
  float* pl = a.part + (size_t)a.group * a.n_kv * a.chunks;
  float* pa = pl + (size_t)a.group * a.n_kv * a.chunks;
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

__global__ __launch_bounds__(64) void attn_combine_kernel(AttnArgs a) {
  const int pos = read_scalar(a.pos_dev, a.pos);
  const int head = blockIdx.x;
  const int n_heads = a.group * a.n_kv;
  float* out = a.out + (size_t)head * a.hd;
  if (pos < 0 || pos >= a.max_seq) {  // only reachable through a device position
    for (int d = threadIdx.x; d < a.hd; d += 64) out[d] = __builtin_nanf("");
    return;
  }
  const int chunks = (pos + a.chunk_len) / a.chunk_len;
  const float* pm = a.part + (size_t)head * a.chunks;
  const float* pl = a.part + (size_t)n_heads * a.chunks + (size_t)head * a.chunks;
  const float* pa = a.part + 2 * (size_t)n_heads * a.chunks + (size_t)head * a.chunks * a.hd;
  float mx = -INFINITY;
  for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, pm[c]);
  float denom = 0.0f;
  for (int c = 0; c < chunks; ++c) denom += pl[c] * expf(pm[c] - mx);
  for (int d = threadIdx.x; d < a.hd; d += 64) {
    float acc = 0.0f;
    for (int c = 0; c < chunks; ++c) acc += pa[(size_t)c * a.hd + d] * expf(pm[c] - mx);
    out[d] = acc / denom;
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
  for (int64_t i = threadIdx.x; i < n; i += kArgmaxThreads) {
    const float v = x[i];
    if (v > best || (idx == INT64_MAX && v == best)) {
      best = v;
      idx = i;
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

}  // namespace

// ---- launchers ---------------------------------------------------------------------
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int dim,
                          float eps, hipStream_t stream) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, stream, x, w, y,
                     dim, eps);
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

hipError_t launch_embedding(const float* table, int vocab, int dim, const int32_t* token_dev,
                            int token, float* y, hipStream_t stream) {
  const int blocks = (dim + 255) / 256;
  hipLaunchKernelGGL(embed_kernel, dim3(blocks), dim3(256), 0, stream, table, vocab, dim,
                     token_dev, token, y);
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
  a.pos_dev = r.pos_dev;
  a.pos = r.pos;
  a.theta = r.theta;
  const int total = (r.n_heads + r.n_kv) * (r.hd / 2);
  hipLaunchKernelGGL(rope_kernel, dim3((total + 255) / 256), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_kv_write(float* keys, float* values, const float* k, const float* v,
                           size_t row, int n, hipStream_t stream) {
  hipLaunchKernelGGL(kv_write_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, keys,
                     values, k, v, row, n);
  return hipGetLastError();
}

int attention_chunks(int hd, int max_len) {
  const int ch = attn_chunk_len(hd == 64 || hd == 128 ? hd : 0);
  return (max_len + ch - 1) / ch;
}

size_t attention_workspace_bytes(int n_heads, int hd, int max_len) {
  const size_t c = (size_t)attention_chunks(hd, max_len);
  return ((size_t)n_heads * c * (2 + (size_t)hd)) * sizeof(float);
}

bool attention_supported(int n_heads, int n_kv, int hd) {
  return n_kv > 0 && n_heads % n_kv == 0 && n_heads / n_kv <= kAttnMaxGroup && hd > 0 &&
         hd <= kAttnMaxHd;
}

template <int HD, int GMAX>
static void attn_launch(const AttnArgs& a, int chunks, hipStream_t stream) {
  constexpr int CH = attn_chunk_len(HD);
  const int hd = HD ? HD : a.hd;
  const int hdp = (hd + 3) & ~3;
  const size_t lds = (size_t)(CH * (hdp + 4) + GMAX * hdp + GMAX * CH) * sizeof(float);
  hipLaunchKernelGGL((attn_chunk_kernel<HD, GMAX>), dim3(chunks, a.n_kv), dim3(64), lds,
                     stream, a);
}

template <int HD>
static void attn_launch_g(const AttnArgs& a, int chunks, hipStream_t stream) {
  if (a.group <= 1) attn_launch<HD, 1>(a, chunks, stream);
  else if (a.group <= 2) attn_launch<HD, 2>(a, chunks, stream);
  else if (a.group <= 4) attn_launch<HD, 4>(a, chunks, stream);
  else if (a.group <= 8) attn_launch<HD, 8>(a, chunks, stream);
  else attn_launch<HD, 16>(a, chunks, stream);
}

hipError_t launch_attention(const AttnLaunch& r, hipStream_t stream) {
  AttnArgs a;
  a.q = r.q;
  a.keys = r.keys;
  a.values = r.values;
  a.out = r.out;
  a.part = r.ws;
  a.layer = r.layer;
  a.max_seq = r.max_seq;
  a.n_kv = r.n_kv;
  a.hd = r.hd;
  a.group = r.n_heads / r.n_kv;
  a.chunks = attention_chunks(r.hd, r.max_len);
  a.chunk_len = attn_chunk_len(r.hd == 64 || r.hd == 128 ? r.hd : 0);
  a.vec = r.hd % 4 == 0 && ((uintptr_t)r.keys & 15) == 0 && ((uintptr_t)r.values & 15) == 0;
  a.pos_dev = r.pos_dev;
  a.pos = r.pos;
  a.scale = sqrtf(1.0f / (float)r.hd);
  const int chunks = a.chunks;
  switch (r.hd) {
    case 64: attn_launch_g<64>(a, chunks, stream); break;
    case 128: attn_launch_g<128>(a, chunks, stream); break;
    case 256: attn_launch_g<256>(a, chunks, stream); break;
    default: attn_launch_g<0>(a, chunks, stream); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(r.n_heads), dim3(64), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_argmax(const float* x, int64_t n, int32_t* out, int32_t* pos_dev,
                         hipStream_t stream) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgmaxThreads), 0, stream, x, n, out,
                     pos_dev);
  return hipGetLastError();
}

}  // namespace mlq
