/*
 * CPU ORACLE — test infrastructure only (see forward_ref.h).
 *
 * Each function restates the reference's CPU code path with the same
 * operation order and float/double types as the C++ source it cites, so the
 * oracle reproduces the reference's rounding where the compiler does (the
 * reference's Release build uses -O2 without fast-math).
 */
#include "forward_ref.h"

#include <math.h>
#include <stddef.h>

/* src/ops.cc:59-69: float sum of squares in index order, scale =
 * sqrt(ss / dim + eps), result = x * w / scale. */
void ref_rmsnorm(const float* x, const float* w, float* y, int dim, float eps) {
  float ss = 0.0f;
  for (int i = 0; i < dim; ++i) ss += x[i] * x[i];
  const float scale = sqrtf(ss / (float)dim + eps);
  for (int i = 0; i < dim; ++i) y[i] = x[i] * w[i] / scale;
}

/* src/ops.cc:89-108: running max from x[0], exp(x - max) summed in order,
 * then each term divided by the sum. */
int ref_softmax(const float* x, float* y, int n) {
  if (n <= 0) return -1;
  float mx = x[0];
  for (int i = 1; i < n; ++i) mx = fmaxf(mx, x[i]);
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) {
    y[i] = expf(x[i] - mx);
    sum += y[i];
  }
  for (int i = 0; i < n; ++i) y[i] /= sum;
  return 0;
}

/* src/ops.cc:111-119: val / (1.0 + std::exp(-val)) — the literal 1.0 is a
 * double, so the quotient is formed in double and rounded once to float. */
void ref_silu(const float* x, float* y, int n) {
  for (int i = 0; i < n; ++i) {
    const float v = x[i];
    y[i] = (float)((double)v / (1.0 + (double)expf(-v)));
  }
}

/* src/ops.cc:137-140 = elementwiseMul(silu(gate), up) (:121-135). */
void ref_swiglu(const float* gate, const float* up, float* y, int n) {
  ref_silu(gate, y, n);
  for (int i = 0; i < n; ++i) y[i] = y[i] * up[i];
}

/* normalRope (src/ops.cc:143-160): pairs (i, i+1) for even i, frequency
 * 1 / theta^(i / hd). */
static void normal_rope(float* x, int n_heads, int hd, int pos, float theta) {
  for (int head = 0; head < n_heads; ++head) {
    for (int i = 0; i < hd; i += 2) {
      const float freq = 1.0f / powf(theta, (float)i / (float)hd);
      const float c = cosf((float)pos * freq);
      const float s = sinf((float)pos * freq);
      const float x0 = x[head * hd + i];
      const float x1 = x[head * hd + i + 1];
      x[head * hd + i] = x0 * c - x1 * s;
      x[head * hd + i + 1] = x0 * s + x1 * c;
    }
  }
}

/* neoxRope (src/ops.cc:163-184): pairs (i, i + hd/2), frequency
 * 1 / theta^(2i / hd). */
static void neox_rope(float* x, int n_heads, int hd, int pos, float theta) {
  const int half = hd / 2;
  for (int head = 0; head < n_heads; ++head) {
    const int base = head * hd;
    for (int i = 0; i < half; ++i) {
      const float freq = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
      const float c = cosf((float)pos * freq);
      const float s = sinf((float)pos * freq);
      const float x0 = x[base + i];
      const float x1 = x[base + half + i];
      x[base + i] = x0 * c - x1 * s;
      x[base + half + i] = x0 * s + x1 * c;
    }
  }
}

/* rope (src/ops.cc:187-228): the same checks (position >= 0, theta finite
 * and positive, head_dim positive and even), q then k. */
int ref_rope(float* q, float* k, int n_heads, int n_kv, int hd, int pos, float theta,
             int type) {
  if (pos < 0) return -1;
  if (!isfinite(theta) || theta <= 0.0f) return -1;
  if (hd <= 0 || hd % 2 != 0) return -1;
  if (type == 1) {
    neox_rope(q, n_heads, hd, pos, theta);
    neox_rope(k, n_kv, hd, pos, theta);
  } else {
    normal_rope(q, n_heads, hd, pos, theta);
    normal_rope(k, n_kv, hd, pos, theta);
  }
  return 0;
}

/* forwardAttention, CPU branch (src/forward.cc:526-565): per head, scores
 * (dot in index order) * sqrt(1 / hd), softmax, then sum_t p[t] * V[t][i] in
 * position order. kv head of query head h: h / (n_heads / n_kv)
 * (mapKVHead, :464-466). */
void ref_attention(const float* q, const float* keys, const float* values, int layer,
                   int pos, int n_heads, int n_kv, int hd, int max_seq, float* out) {
  const float scale = sqrtf(1.0f / (float)hd);
  const int group = n_heads / n_kv;
  float scores[pos + 1];
  float probs[pos + 1];
  for (int head = 0; head < n_heads; ++head) {
    const int kvh = head / group;
    for (int t = 0; t <= pos; ++t) {
      const float* kr = keys + (((size_t)layer * max_seq + t) * n_kv + kvh) * hd;
      float sum = 0.0f;
      for (int j = 0; j < hd; ++j) sum += q[head * hd + j] * kr[j];
      scores[t] = sum * scale;
    }
    ref_softmax(scores, probs, pos + 1);
    for (int i = 0; i < hd; ++i) {
      float sum = 0.0f;
      for (int t = 0; t <= pos; ++t) {
        const float* vr = values + (((size_t)layer * max_seq + t) * n_kv + kvh) * hd;
        sum += probs[t] * vr[i];
      }
      out[head * hd + i] = sum;
    }
  }
}

/* linearNaive (src/matmul_dispatch.cc:32-50). */
void ref_linear_f32(const float* x, const float* w, float* y, int n, int k) {
  for (int i = 0; i < n; ++i) {
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) sum += x[j] * w[(size_t)i * k + j];
    y[i] = sum;
  }
}

/* argMax (src/ops.cc:230-246): strict '>' from x[0]. */
int ref_argmax(const float* x, int n) {
  if (n <= 0) return -1;
  int best = 0;
  float best_val = x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] > best_val) {
      best_val = x[i];
      best = i;
    }
  }
  return best;
}
