/*
 * CPU ORACLE — test infrastructure only (see quant_ref.h for the pinning
 * strategy). Plain C restatement of the reference CPU quantized Linear:
 *   src/quant.cc:32-101    fp16 <-> fp32 bit conversions
 *   src/quant.cc:130-392   quantizers / dequantizers
 *   src/quant.cc:401-650   linearQuantizedImpl + per-type dequant + AVX2 Q8_0
 *   src/threadpool.cc:26-57 work partition (spawn-per-call, even chunks)
 *   src/ops.cc:28-40       type dispatch (the callers pick the typed entry)
 *
 * Build flavours mirror the reference's two CMake builds
 * (CMakeLists.txt:16-25 adds -mavx2 -mfma; :192 Release = -O2).
 */
#include "quant_ref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#if defined(__AVX2__)
#include <immintrin.h>
#define REF_AVX2 1
#else
#define REF_AVX2 0
#endif

#define QK 32

int ref_build_flavor(void) { return REF_AVX2; }

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32                                                             */
/* ------------------------------------------------------------------------ */

/* quant.cc:32-70. Round-to-nearest decided by the first dropped mantissa bit
 * alone (ties therefore go away from zero), subnormal results for fp16
 * exponents -10..0, signed zero below that, inf at/after overflow (also for
 * NaN inputs, whose exponent field is all ones). */
uint16_t ref_f32_to_fp16(float value) {
  uint32_t u;
  memcpy(&u, &value, sizeof u);
  const uint32_t sign = (u >> 16) & 0x8000u;
  int32_t e = (int32_t)((u >> 23) & 0xffu) - 112; /* rebias 127 -> 15 */
  uint32_t frac = u & 0x7fffffu;

  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    /* make the hidden bit explicit and align to the fp16 subnormal grid */
    uint32_t sub = (frac | 0x800000u) >> (uint32_t)(1 - e);
    if (sub & (1u << 12)) sub += 1u << 13; /* first dropped bit set: up */
    return (uint16_t)(sign | (sub >> 13));
  }
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (frac & (1u << 12)) {
    frac += 1u << 13;
    if (frac & 0x800000u) { /* mantissa carried into the exponent */
      frac = 0;
      e += 1;
      if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    }
  }
  return (uint16_t)(sign | ((uint32_t)e << 10) | (frac >> 13));
}

/* quant.cc:72-101. Exact IEEE binary16 decode, subnormals normalised. */
float ref_fp16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t frac = h & 0x3ffu;
  uint32_t u;
  if (e == 0x1fu) {
    u = sign | 0x7f800000u | (frac << 13);
  } else if (e != 0) {
    u = sign | ((e + 112u) << 23) | (frac << 13);
  } else if (frac == 0) {
    u = sign;
  } else {
    /* subnormal: shift until the hidden bit appears, tracking the exponent */
    int32_t ee = 1;
    while (!(frac & 0x400u)) {
      frac <<= 1;
      --ee;
    }
    u = sign | ((uint32_t)(ee + 112) << 23) | ((frac & 0x3ffu) << 13);
  }
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

void ref_f32_to_fp16_array(const float* src, uint16_t* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = ref_f32_to_fp16(src[i]);
}

void ref_fp16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = ref_fp16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* Quantizers                                                                */
/* ------------------------------------------------------------------------ */

/* Largest |x| over [lo, hi) with the reference's strict-greater scan. */
static float block_amax(const float* src, int lo, int hi) {
  float amax = 0.0f;
  for (int k = lo; k < hi; ++k) {
    const float a = fabsf(src[k]);
    if (a > amax) amax = a;
  }
  return amax;
}

/* quant.cc:130-190: d = fp16(amax/127); q = clamp(round(x / d_stored), +-127)
 * with round() = half away from zero; partial last block zero padded. */
size_t ref_quantize_q8_0(const float* src, int n_rows, int row_size,
                         ref_block_q8_0* out) {
  if (n_rows <= 0 || row_size <= 0) return 0;
  const int nb = (row_size + QK - 1) / QK;
  size_t count = 0;
  for (int r = 0; r < n_rows; ++r) {
    const float* row = src + (size_t)r * row_size;
    for (int b = 0; b < nb; ++b) {
      const int lo = b * QK;
      const int hi = lo + QK < row_size ? lo + QK : row_size;
      ref_block_q8_0* blk = &out[count++];
      memset(blk, 0, sizeof *blk);
      const float amax = block_amax(row, lo, hi);
      if (amax > 0.0f) {
        blk->d = ref_f32_to_fp16(amax / 127.0f);
        const float ds = ref_fp16_to_f32(blk->d);
        const float inv = ds == 0.0f ? 0.0f : 1.0f / ds;
        for (int i = 0; i < hi - lo; ++i) {
          int q = (int)roundf(row[lo + i] * inv);
          q = q > 127 ? 127 : (q < -127 ? -127 : q);
          blk->qs[i] = (int8_t)q;
        }
      }
    }
  }
  return count;
}

/* quant.cc:228-302: d = fp16(amax/7); q = clamp(round(x/d + 8), 0, 15);
 * element j -> low nibble of qs[j], element j+16 -> high nibble. Elements
 * past the row end quantize the value 0 (q = 8, or q = round(8) = 8). */
size_t ref_quantize_q4_0(const float* src, int n_rows, int row_size,
                         ref_block_q4_0* out) {
  if (n_rows <= 0 || row_size <= 0) return 0;
  const int nb = (row_size + QK - 1) / QK;
  size_t count = 0;
  for (int r = 0; r < n_rows; ++r) {
    const float* row = src + (size_t)r * row_size;
    for (int b = 0; b < nb; ++b) {
      const int lo = b * QK;
      const int hi = lo + QK < row_size ? lo + QK : row_size;
      ref_block_q4_0* blk = &out[count++];
      memset(blk, 0, sizeof *blk);
      const float amax = block_amax(row, lo, hi);
      if (amax > 0.0f) {
        blk->d = ref_f32_to_fp16(amax / 7.0f);
        const float ds = ref_fp16_to_f32(blk->d);
        const float inv = ds == 0.0f ? 0.0f : 1.0f / ds;
        for (int j = 0; j < QK / 2; ++j) {
          const float a = lo + j < hi ? row[lo + j] * inv : 0.0f;
          const float c = lo + j + QK / 2 < hi ? row[lo + j + QK / 2] * inv : 0.0f;
          int qa = (int)roundf(a + 8.0f);
          int qc = (int)roundf(c + 8.0f);
          qa = qa < 0 ? 0 : (qa > 15 ? 15 : qa);
          qc = qc < 0 ? 0 : (qc > 15 ? 15 : qc);
          blk->qs[j] = (uint8_t)(qa | (qc << 4));
        }
      }
    }
  }
  return count;
}

/* ------------------------------------------------------------------------ */
/* Per-element dequant (quant.cc:477-503): value of element idx in a block.  */
/* Called once per element by the scalar Linear, exactly like the reference  */
/* (the software fp16 decode per element is part of the baseline's cost).    */
/* ------------------------------------------------------------------------ */

static float deq_q8_0(const ref_block_q8_0* b, int idx) {
  return ref_fp16_to_f32(b->d) * (float)b->qs[idx];
}

static int nib(const uint8_t* qs, int idx) {
  return idx < 16 ? (qs[idx] & 0x0f) : (qs[idx - 16] >> 4);
}

static float deq_q4_0(const ref_block_q4_0* b, int idx) {
  return ref_fp16_to_f32(b->d) * (float)(nib(b->qs, idx) - 8);
}

static float deq_q4_1(const ref_block_q4_1* b, int idx) {
  return ref_fp16_to_f32(b->d) * (float)nib(b->qs, idx) + ref_fp16_to_f32(b->m);
}

/* ------------------------------------------------------------------------ */
/* Dequantizers (quant.cc:192-223, 304-345, 350-392)                          */
/* ------------------------------------------------------------------------ */

#define DEFINE_DEQUANT(NAME, BLOCK, DEQ)                                     \
  int NAME(const BLOCK* blocks, size_t n_blocks, int n_rows, int row_size,  \
           float* dst) {                                                     \
    if (n_rows <= 0 || row_size <= 0) return REF_ERR_SHAPE;                 \
    const int nb = (row_size + QK - 1) / QK;                                \
    if (n_blocks != (size_t)n_rows * (size_t)nb) return REF_ERR_BLOCKS;     \
    for (int r = 0; r < n_rows; ++r) {                                      \
      for (int b = 0; b < nb; ++b) {                                        \
        const BLOCK* blk = &blocks[(size_t)r * nb + b];                     \
        const int lo = b * QK;                                              \
        const int hi = lo + QK < row_size ? lo + QK : row_size;             \
        for (int k = lo; k < hi; ++k)                                       \
          dst[(size_t)r * row_size + k] = DEQ(blk, k - lo);                 \
      }                                                                     \
    }                                                                       \
    return REF_OK;                                                          \
  }

DEFINE_DEQUANT(ref_dequantize_q8_0, ref_block_q8_0, deq_q8_0)
DEFINE_DEQUANT(ref_dequantize_q4_0, ref_block_q4_0, deq_q4_0)
DEFINE_DEQUANT(ref_dequantize_q4_1, ref_block_q4_1, deq_q4_1)

/* ------------------------------------------------------------------------ */
/* Work partition: threadpool.cc:26-57. Inline when n < 16 * threads; else   */
/* `threads` fresh threads per call over contiguous chunks, the remainder    */
/* going one extra item each to the first chunks.                            */
/* ------------------------------------------------------------------------ */

typedef void (*range_fn)(void* ctx, int begin, int end);

typedef struct {
  range_fn fn;
  void* ctx;
  int begin, end;
} range_job;

static void* run_range(void* arg) {
  range_job* j = (range_job*)arg;
  j->fn(j->ctx, j->begin, j->end);
  return NULL;
}

static int resolve_threads(int n_threads) {
  if (n_threads > 0) return n_threads;
  long hc = sysconf(_SC_NPROCESSORS_ONLN);
  return hc > 0 ? (int)hc : 4;
}

static void submit_task(int n, int n_threads, range_fn fn, void* ctx) {
  if (n <= 0) return;
  int t = resolve_threads(n_threads);
  if (n < 16 * t) {
    fn(ctx, 0, n);
    return;
  }
  if (t > n) t = n;
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)t);
  range_job* jobs = (range_job*)malloc(sizeof(range_job) * (size_t)t);
  const int base = n / t, extra = n % t;
  int start = 0;
  for (int i = 0; i < t; ++i) {
    const int len = base + (i < extra ? 1 : 0);
    jobs[i].fn = fn;
    jobs[i].ctx = ctx;
    jobs[i].begin = start;
    jobs[i].end = start + len;
    start += len;
    pthread_create(&tid[i], NULL, run_range, &jobs[i]);
  }
  for (int i = 0; i < t; ++i) pthread_join(tid[i], NULL);
  free(jobs);
  free(tid);
}

/* ------------------------------------------------------------------------ */
/* Quantized Linear                                                          */
/* ------------------------------------------------------------------------ */

typedef struct {
  const float* x;
  const void* w;
  float* y;
  int in_features, out_features, nb;
  size_t x_len; /* rows * in_features */
} linear_ctx;

/* Shape/block-count validation of linearQuantizedImpl (quant.cc:406-447).
 * The reference logs and returns an empty tensor; the oracle returns an
 * error code instead. */
static int check_linear(int rows, int in_features, size_t n_blocks,
                        int out_features, int w_in_features) {
  if (rows <= 0 || in_features <= 0 || out_features <= 0) return REF_ERR_SHAPE;
  if (w_in_features != in_features) return REF_ERR_SHAPE;
  const size_t nb = (size_t)((in_features + QK - 1) / QK);
  if (n_blocks != (size_t)out_features * nb) return REF_ERR_BLOCKS;
  return REF_OK;
}

/* linearQuantizedImpl's task body (quant.cc:453-472): one fp32 accumulator
 * per output, blocks and elements visited in increasing k. */
#define DEFINE_SCALAR_TASK(NAME, BLOCK, DEQ)                                  \
  static void NAME(void* vctx, int begin, int end) {                         \
    const linear_ctx* c = (const linear_ctx*)vctx;                           \
    const BLOCK* w = (const BLOCK*)c->w;                                     \
    for (int f = begin; f < end; ++f) {                                      \
      const int r = f / c->out_features;                                     \
      const int n = f % c->out_features;                                     \
      const float* xr = c->x + (size_t)r * c->in_features;                   \
      float acc = 0.0f;                                                      \
      const BLOCK* wr = w + (size_t)n * c->nb;                               \
      for (int b = 0; b < c->nb; ++b) {                                      \
        const int lo = b * QK;                                               \
        const int hi = lo + QK < c->in_features ? lo + QK : c->in_features;  \
        for (int k = lo; k < hi; ++k) acc += DEQ(&wr[b], k - lo) * xr[k];    \
      }                                                                      \
      c->y[(size_t)r * c->out_features + n] = acc;                           \
    }                                                                        \
  }

DEFINE_SCALAR_TASK(task_q4_0, ref_block_q4_0, deq_q4_0)
DEFINE_SCALAR_TASK(task_q4_1, ref_block_q4_1, deq_q4_1)

#if REF_AVX2
/* quant.cc:556-626 (AVX2 build): per block, 8-lane FMA over groups of 8
 * weights (d*q in the low lanes); the second FMA of each step multiplies a
 * zero vector by x[k+4 .. k+11] (the reference's widened load), so it adds
 * +-0 for finite x and NaN when one of those x is inf/NaN. The 8 lanes are
 * folded (lanes i + i+4, then two horizontal adds) into a scalar sum after
 * every block; a block's tail (< 8 elements) is added in scalar. */
static void task_q8_0(void* vctx, int begin, int end) {
  const linear_ctx* c = (const linear_ctx*)vctx;
  const ref_block_q8_0* w = (const ref_block_q8_0*)c->w;
  const int K = c->in_features;
  for (int f = begin; f < end; ++f) {
    const int r = f / c->out_features;
    const int n = f % c->out_features;
    const float* xr = c->x + (size_t)r * K;
    const ref_block_q8_0* wr = w + (size_t)n * c->nb;
    float total = 0.0f;
    for (int b = 0; b < c->nb; ++b) {
      const float d = ref_fp16_to_f32(wr[b].d);
      const int lo = b * QK;
      const int hi = lo + QK < K ? lo + QK : K;
      __m256 lanes = _mm256_setzero_ps();
      const __m256 dv = _mm256_set1_ps(d);
      const __m256 zero_w = _mm256_mul_ps(_mm256_setzero_ps(), dv);
      int k = lo;
      for (; k + 8 <= hi; k += 8) {
        const __m128i q8 = _mm_loadl_epi64((const __m128i*)(wr[b].qs + (k - lo)));
        const __m256 wq = _mm256_mul_ps(
            _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q8)), dv);
        lanes = _mm256_fmadd_ps(wq, _mm256_loadu_ps(xr + k), lanes);
        /* (0*d) times x[k+4 .. k+11] of the flat x buffer (crossing into
         * the next row like the reference); past the end of x the oracle
         * uses 0 where the reference reads up to 16 bytes out of bounds */
        float xs[8];
        for (int i = 0; i < 8; ++i) {
          const size_t kk = (size_t)r * K + (size_t)(k + 4 + i);
          xs[i] = kk < c->x_len ? c->x[kk] : 0.0f;
        }
        lanes = _mm256_fmadd_ps(zero_w, _mm256_loadu_ps(xs), lanes);
      }
      __m128 s = _mm_add_ps(_mm256_castps256_ps128(lanes),
                            _mm256_extractf128_ps(lanes, 1));
      s = _mm_hadd_ps(s, s);
      s = _mm_hadd_ps(s, s);
      total += _mm_cvtss_f32(s);
      for (; k < hi; ++k) total += d * (float)wr[b].qs[k - lo] * xr[k];
    }
    c->y[(size_t)r * c->out_features + n] = total;
  }
}
#else
DEFINE_SCALAR_TASK(task_q8_0, ref_block_q8_0, deq_q8_0)
#endif

static int run_linear(range_fn task, const float* x, int rows, int in_features,
                      const void* w, size_t n_blocks, int out_features,
                      int w_in_features, float* y, int n_threads) {
  const int rc = check_linear(rows, in_features, n_blocks, out_features,
                              w_in_features);
  if (rc != REF_OK) return rc;
  linear_ctx c = {x, w, y, in_features, out_features,
                  (in_features + QK - 1) / QK,
                  (size_t)rows * (size_t)in_features};
  submit_task(rows * out_features, n_threads, task, &c);
  return REF_OK;
}

int ref_linear_q8_0(const float* x, int rows, int in_features,
                    const ref_block_q8_0* w, size_t n_blocks, int out_features,
                    int w_in_features, float* y, int n_threads) {
  return run_linear(task_q8_0, x, rows, in_features, w, n_blocks, out_features,
                    w_in_features, y, n_threads);
}

int ref_linear_q4_0(const float* x, int rows, int in_features,
                    const ref_block_q4_0* w, size_t n_blocks, int out_features,
                    int w_in_features, float* y, int n_threads) {
  return run_linear(task_q4_0, x, rows, in_features, w, n_blocks, out_features,
                    w_in_features, y, n_threads);
}

int ref_linear_q4_1(const float* x, int rows, int in_features,
                    const ref_block_q4_1* w, size_t n_blocks, int out_features,
                    int w_in_features, float* y, int n_threads) {
  return run_linear(task_q4_1, x, rows, in_features, w, n_blocks, out_features,
                    w_in_features, y, n_threads);
}
