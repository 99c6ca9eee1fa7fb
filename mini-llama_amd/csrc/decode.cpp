// C ABI of the decode-step operators and the whole-token decode step
// (declarations and contracts in include/mlq.h). Argument checks follow the
// reference's validators (src/ops.cc:43-72, 187-218; src/cuda_attention.cu
// validateAttentionDeviceInputs; src/forward.cc:27-58) and report through
// return codes; every launch is stream-ordered and nothing synchronizes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "kernels/launch.h"
#include "mlq.h"

using namespace mlq;

namespace {

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

int check_cache(const mlq_kv_cache* c) {
  if (c == nullptr || c->keys == nullptr || c->values == nullptr) return MLQ_ERR_INVALID_ARG;
  if (c->n_layers <= 0 || c->max_seq_len <= 0 || c->n_kv_heads <= 0 || c->head_dim <= 0)
    return MLQ_ERR_SHAPE;
  return MLQ_OK;
}

// Attention shape checks of validateAttentionDeviceInputs
// (src/cuda_attention.cu:84-121) for a given head count.
int check_heads(const mlq_kv_cache* c, int n_heads) {
  if (n_heads <= 0) return MLQ_ERR_SHAPE;
  if (n_heads % c->n_kv_heads != 0) return MLQ_ERR_SHAPE;
  if (!attention_supported(n_heads, c->n_kv_heads, c->head_dim)) return MLQ_ERR_UNSUPPORTED;
  return MLQ_OK;
}

// Every Linear of the model: fused q|k|v when wk.base is null, fused
// gate|up when w_up.base is null.
bool qkv_fused(const mlq_layer& l) { return l.wk.base == nullptr && l.wv.base == nullptr; }
bool glu_fused(const mlq_layer& l) { return l.w_up.base == nullptr; }

struct DecodeBuffers {
  float* x;     // residual stream [dim]
  float* x2;    // residual after attention [dim]
  float* h;     // normalised activations [dim]
  float* xn;    // pre-scaled RMSNorm input of the next Linear: x * norm [dim]
  float* ssq;   // its partial sums of x^2, one per 16 elements [kSsqPartsMax]
  float* qkv;   // q | k | v
  float* attn;  // attention output [n_heads * hd]
  float* ffn;   // silu(gate) * up [hidden]
  float* gate;  // unfused gate / up outputs [hidden] each
  float* up;
  float* apart; // attention partials
  float* rope;  // the step's RoPE table: cos then sin of each pair's angle
  void* lin;    // Linear workspace
  size_t lin_bytes;
  size_t total;
};

int linear_ws(const mlq_weight& w, size_t* need) {
  size_t b = 0;
  const int rc = mlq_linear_workspace(&w, 1, &b);
  if (rc != MLQ_OK) return rc;
  if (b > *need) *need = b;
  return MLQ_OK;
}

// Shape checks of the model against itself (validateLoadedShapes-like) and the
// workspace plan; base may be null (sizes only).
int plan(const mlq_model* m, char* base, DecodeBuffers* b) {
  if (m == nullptr || m->layers == nullptr || m->token_embedding == nullptr ||
      m->final_norm == nullptr)
    return MLQ_ERR_INVALID_ARG;
  if (m->vocab_size <= 0 || m->dim <= 0 || m->hidden_dim <= 0 || m->n_layers <= 0 ||
      m->n_heads <= 0 || m->n_kv_heads <= 0 || m->head_dim <= 0 || m->max_seq_len <= 0)
    return MLQ_ERR_SHAPE;
  if (m->n_heads % m->n_kv_heads != 0) return MLQ_ERR_SHAPE;
  if (m->head_dim % 2 != 0) return MLQ_ERR_SHAPE;
  if (!attention_supported(m->n_heads, m->n_kv_heads, m->head_dim)) return MLQ_ERR_UNSUPPORTED;
  if (!(std::isfinite(m->rope_theta) && m->rope_theta > 0.0f)) return MLQ_ERR_INVALID_ARG;
  if (!(std::isfinite(m->rms_norm_eps) && m->rms_norm_eps > 0.0f)) return MLQ_ERR_INVALID_ARG;
  if (m->rope_type != MLQ_ROPE_NORMAL && m->rope_type != MLQ_ROPE_NEOX) return MLQ_ERR_INVALID_ARG;
  const int dim = m->dim, hid = m->hidden_dim;
  const int qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
  size_t lin = 0;
  auto expect = [&](const mlq_weight& w, int n, int k) -> int {
    if (w.base == nullptr) return MLQ_ERR_INVALID_ARG;
    if (w.n != n || w.k != k) return MLQ_ERR_SHAPE;
    return linear_ws(w, &lin);
  };
  for (int i = 0; i < m->n_layers; ++i) {
    const mlq_layer& l = m->layers[i];
    if (l.attn_norm == nullptr || l.ffn_norm == nullptr) return MLQ_ERR_INVALID_ARG;
    int rc;
    if (qkv_fused(l)) {
      if ((rc = expect(l.wq, qd + 2 * kvd, dim)) != MLQ_OK) return rc;
    } else {
      if ((rc = expect(l.wq, qd, dim)) != MLQ_OK) return rc;
      if ((rc = expect(l.wk, kvd, dim)) != MLQ_OK) return rc;
      if ((rc = expect(l.wv, kvd, dim)) != MLQ_OK) return rc;
    }
    if ((rc = expect(l.wo, dim, qd)) != MLQ_OK) return rc;
    if (glu_fused(l)) {
      if ((rc = expect(l.w_gate, 2 * hid, dim)) != MLQ_OK) return rc;
      if (hid % 8 != 0) return MLQ_ERR_SHAPE;
    } else {
      if ((rc = expect(l.w_gate, hid, dim)) != MLQ_OK) return rc;
      if ((rc = expect(l.w_up, hid, dim)) != MLQ_OK) return rc;
    }
    if ((rc = expect(l.w_down, dim, hid)) != MLQ_OK) return rc;
  }
  int rc = expect(m->lm_head, m->vocab_size, dim);
  if (rc != MLQ_OK) return rc;

  size_t off = 0;
  auto take = [&](size_t floats) {
    float* p = base ? (float*)(base + off) : nullptr;
    off += align256(floats * sizeof(float));
    return p;
  };
  b->x = take(dim);
  b->x2 = take(dim);
  b->h = take(dim);
  b->xn = take(dim);
  b->ssq = take(kSsqPartsMax);
  b->qkv = take((size_t)qd + 2 * kvd);
  b->attn = take(qd);
  b->ffn = take(hid);
  b->gate = take(hid);
  b->up = take(hid);
  b->rope = take(m->head_dim);
  b->apart = (float*)(base ? base + off : nullptr);
  off += align256(attention_workspace_bytes(m->n_heads, m->head_dim, m->max_seq_len));
  b->lin = base ? base + off : nullptr;
  b->lin_bytes = lin;
  off += align256(lin);
  b->total = off;
  return MLQ_OK;
}

// ---- prefill (forwardBatch over [n, K] Linears) -------------------------------
// Query rows per attention launch: bounds the partial workspace.
constexpr int kPrefillAttnRows = 64;

struct PrefillBuffers {
  int32_t* tokens;  // [n]
  float* x;         // residual stream [n][dim]
  float* x2;        // after attention [n][dim]
  float* h;         // normalised activations / projection output [n][dim]
  float* qkv;       // [n][qd + 2 kvd] (fused) or q [n][qd]
  float* k;         // unfused: [n][kvd] each
  float* v;
  float* attn;      // [n][qd]
  float* ffn;       // [n][hidden]
  float* gate;      // unfused: [n][hidden] each
  float* up;
  float* apart;     // attention partials for kPrefillAttnRows rows
  float* rope;      // [n][head_dim] RoPE angle table of the prompt's positions
  void* lin;        // Linear workspace for n rows (and 1 row)
  size_t lin_bytes;
  // n > kSkinnyMaxRows (prefill GEMM): the fp16 GEMM input written by the
  // RMSNorm producer, with its row exponents
  _Float16* xh;     // [n][f16_row_stride(dim)]
  int* xexp;        // [n]
  size_t total;
};

int plan_prefill(const mlq_model* m, int n, char* base, PrefillBuffers* b) {
  DecodeBuffers d;
  int rc = plan(m, nullptr, &d);  // model checks
  if (rc != MLQ_OK) return rc;
  if (n <= 0) return MLQ_ERR_SHAPE;
  const int dim = m->dim, hid = m->hidden_dim;
  const int qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
  bool any_unfused_qkv = false, any_unfused_glu = false;
  size_t lin = d.lin_bytes;
  auto need = [&](const mlq_weight& w) {
    size_t bytes = 0;
    if (mlq_linear_workspace(&w, n, &bytes) == MLQ_OK && bytes > lin) lin = bytes;
  };
  for (int i = 0; i < m->n_layers; ++i) {
    const mlq_layer& l = m->layers[i];
    any_unfused_qkv |= !qkv_fused(l);
    any_unfused_glu |= !glu_fused(l);
    need(l.wq);
    if (!qkv_fused(l)) {
      need(l.wk);
      need(l.wv);
    }
    need(l.wo);
    need(l.w_gate);
    if (!glu_fused(l)) need(l.w_up);
    need(l.w_down);
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  const size_t f = sizeof(float), rows = (size_t)n;
  b->tokens = (int32_t*)take(rows * sizeof(int32_t));
  b->x = (float*)take(rows * dim * f);
  b->x2 = (float*)take(rows * dim * f);
  b->h = (float*)take(rows * dim * f);
  b->qkv = (float*)take(rows * (qd + 2 * kvd) * f);
  b->k = any_unfused_qkv ? (float*)take(rows * kvd * f) : nullptr;
  b->v = any_unfused_qkv ? (float*)take(rows * kvd * f) : nullptr;
  b->attn = (float*)take(rows * qd * f);
  b->ffn = (float*)take(rows * hid * f);
  b->gate = any_unfused_glu ? (float*)take(rows * hid * f) : nullptr;
  b->up = any_unfused_glu ? (float*)take(rows * hid * f) : nullptr;
  b->apart = (float*)take(attention_workspace_bytes(m->n_heads, m->head_dim, m->max_seq_len,
                                                    std::min(n, kPrefillAttnRows)));
  b->lin_bytes = lin;
  b->rope = (float*)take(rows * m->head_dim * f);
  b->lin = take(lin);
  const bool gemm_rows = n > kSkinnyMaxRows;
  b->xh = gemm_rows ? (_Float16*)take(rows * f16_row_stride(dim) * 2) : nullptr;
  b->xexp = gemm_rows ? (int*)take(rows * sizeof(int)) : nullptr;
  b->total = off;
  return MLQ_OK;
}

}  // namespace

extern "C" {

int mlq_rmsnorm(const float* x, const float* weight, float* y, int rows, int dim, float eps,
                mlq_stream_t stream) {
  if (x == nullptr || weight == nullptr || y == nullptr) return MLQ_ERR_INVALID_ARG;
  if (rows <= 0 || dim <= 0) return MLQ_ERR_SHAPE;
  // cudaRmsNormDeviceWeight (src/cuda_ops.cu:99-101)
  if (!(std::isfinite(eps) && eps > 0.0f)) return MLQ_ERR_INVALID_ARG;
  return record_hip(launch_rmsnorm(x, weight, y, rows, dim, eps, (hipStream_t)stream));
}

static int eltwise(int op, const float* a, const float* b, float* y, int64_t n,
                   mlq_stream_t stream) {
  if (a == nullptr || y == nullptr || (op != kEltSilu && b == nullptr)) return MLQ_ERR_INVALID_ARG;
  if (n <= 0) return MLQ_ERR_SHAPE;
  return record_hip(launch_eltwise(op, a, b, y, n, (hipStream_t)stream));
}

int mlq_add(const float* a, const float* b, float* y, int64_t n, mlq_stream_t stream) {
  return eltwise(kEltAdd, a, b, y, n, stream);
}
int mlq_mul(const float* a, const float* b, float* y, int64_t n, mlq_stream_t stream) {
  return eltwise(kEltMul, a, b, y, n, stream);
}
int mlq_silu(const float* x, float* y, int64_t n, mlq_stream_t stream) {
  return eltwise(kEltSilu, x, nullptr, y, n, stream);
}
int mlq_swiglu(const float* gate, const float* up, float* y, int64_t n, mlq_stream_t stream) {
  return eltwise(kEltSwiGLU, gate, up, y, n, stream);
}

int mlq_softmax(const float* x, float* y, int64_t n, mlq_stream_t stream) {
  if (x == nullptr || y == nullptr) return MLQ_ERR_INVALID_ARG;
  if (n <= 0) return MLQ_ERR_SHAPE;
  return record_hip(launch_softmax(x, y, n, (hipStream_t)stream));
}

int mlq_embedding(const float* table, int vocab, int dim, int token, float* y,
                  mlq_stream_t stream) {
  if (table == nullptr || y == nullptr) return MLQ_ERR_INVALID_ARG;
  if (vocab <= 0 || dim <= 0) return MLQ_ERR_SHAPE;
  if (token < 0 || token >= vocab) return MLQ_ERR_INVALID_ARG;
  return record_hip(launch_embedding(table, vocab, dim, nullptr, token, y, (hipStream_t)stream));
}

int mlq_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos,
             float theta, int rope_type, mlq_stream_t stream) {
  if (q == nullptr || k == nullptr) return MLQ_ERR_INVALID_ARG;
  if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0)
    return MLQ_ERR_SHAPE;
  if (pos < 0 || !(std::isfinite(theta) && theta > 0.0f)) return MLQ_ERR_INVALID_ARG;
  if (rope_type != MLQ_ROPE_NORMAL && rope_type != MLQ_ROPE_NEOX) return MLQ_ERR_INVALID_ARG;
  RopeLaunch r;
  r.q = q;
  r.k = k;
  r.n_heads = n_heads;
  r.n_kv = n_kv_heads;
  r.hd = head_dim;
  r.neox = rope_type == MLQ_ROPE_NEOX;
  r.pos = pos;
  r.theta = theta;
  return record_hip(launch_rope(r, (hipStream_t)stream));
}

int mlq_kv_cache_bytes(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                       size_t* bytes) {
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  if (n_layers <= 0 || max_seq_len <= 0 || n_kv_heads <= 0 || head_dim <= 0)
    return MLQ_ERR_SHAPE;
  *bytes = (size_t)n_layers * max_seq_len * n_kv_heads * head_dim * sizeof(float);
  return MLQ_OK;
}

int mlq_kv_write(const mlq_kv_cache* c, int layer, int pos, const float* k, const float* v,
                 mlq_stream_t stream) {
  int rc = check_cache(c);
  if (rc != MLQ_OK) return rc;
  if (k == nullptr || v == nullptr) return MLQ_ERR_INVALID_ARG;
  if (layer < 0 || layer >= c->n_layers || pos < 0 || pos >= c->max_seq_len)
    return MLQ_ERR_SHAPE;
  const int n = c->n_kv_heads * c->head_dim;
  const size_t row = ((size_t)layer * c->max_seq_len + pos) * n;
  return record_hip(launch_kv_write(c->keys, c->values, k, v, row, n, (hipStream_t)stream));
}

int mlq_attention_workspace(const mlq_kv_cache* c, int n_heads, size_t* bytes) {
  int rc = check_cache(c);
  if (rc != MLQ_OK) return rc;
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  if ((rc = check_heads(c, n_heads)) != MLQ_OK) return rc;
  *bytes = attention_workspace_bytes(n_heads, c->head_dim, c->max_seq_len);
  return MLQ_OK;
}

int mlq_attention_decode(const mlq_kv_cache* c, int layer, int pos, const float* q,
                         int n_heads, float* out, void* ws, size_t ws_bytes,
                         mlq_stream_t stream) {
  int rc = check_cache(c);
  if (rc != MLQ_OK) return rc;
  if (q == nullptr || out == nullptr || ws == nullptr) return MLQ_ERR_INVALID_ARG;
  if ((rc = check_heads(c, n_heads)) != MLQ_OK) return rc;
  if (layer < 0 || layer >= c->n_layers || pos < 0 || pos >= c->max_seq_len)
    return MLQ_ERR_SHAPE;
  if (ws_bytes < attention_workspace_bytes(n_heads, c->head_dim, pos + 1))
    return MLQ_ERR_BUFFER_TOO_SMALL;
  AttnLaunch a;
  a.q = q;
  a.keys = c->keys;
  a.values = c->values;
  a.out = out;
  a.ws = (float*)ws;
  a.layer = layer;
  a.max_seq = c->max_seq_len;
  a.n_heads = n_heads;
  a.n_kv = c->n_kv_heads;
  a.hd = c->head_dim;
  a.max_len = pos + 1;
  a.pos = pos;
  return record_hip(launch_attention(a, (hipStream_t)stream));
}

int mlq_argmax(const float* x, int64_t n, int32_t* out, mlq_stream_t stream) {
  if (x == nullptr || out == nullptr) return MLQ_ERR_INVALID_ARG;
  if (n <= 0) return MLQ_ERR_SHAPE;
  return record_hip(launch_argmax(x, n, out, nullptr, (hipStream_t)stream));
}

int mlq_argmax_workspace(int64_t n, size_t* bytes) {
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  if (n <= 0) return MLQ_ERR_SHAPE;
  *bytes = argmax_workspace_bytes(n);
  return MLQ_OK;
}

int mlq_greedy_next(const float* logits, int vocab, int32_t* token_dev, int32_t* pos_dev,
                    void* ws, size_t ws_bytes, mlq_stream_t stream) {
  if (logits == nullptr || token_dev == nullptr || pos_dev == nullptr || ws == nullptr)
    return MLQ_ERR_INVALID_ARG;
  if (vocab <= 0) return MLQ_ERR_SHAPE;
  if (((uintptr_t)ws & 7u) != 0) return MLQ_ERR_INVALID_ARG;
  if (ws_bytes < argmax_workspace_bytes(vocab)) return MLQ_ERR_BUFFER_TOO_SMALL;
  return record_hip(
      launch_argmax_ws(logits, vocab, token_dev, pos_dev, ws, (hipStream_t)stream));
}

int mlq_decode_workspace(const mlq_model* m, size_t* bytes) {
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  DecodeBuffers b;
  const int rc = plan(m, nullptr, &b);
  if (rc != MLQ_OK) return rc;
  *bytes = b.total;
  return MLQ_OK;
}

int mlq_decode_token(const mlq_model* m, const mlq_kv_cache* c, int token, int pos,
                     const int32_t* token_dev, const int32_t* pos_dev, float* logits,
                     void* ws, size_t ws_bytes, mlq_stream_t stream) {
  DecodeBuffers b;
  int rc = plan(m, (char*)ws, &b);
  if (rc != MLQ_OK) return rc;
  if ((rc = check_cache(c)) != MLQ_OK) return rc;
  if (logits == nullptr || ws == nullptr) return MLQ_ERR_INVALID_ARG;
  if (((uintptr_t)ws & 255u) != 0) return MLQ_ERR_INVALID_ARG;
  if (ws_bytes < b.total) return MLQ_ERR_BUFFER_TOO_SMALL;
  if (c->n_layers != m->n_layers || c->n_kv_heads != m->n_kv_heads ||
      c->head_dim != m->head_dim || c->max_seq_len < m->max_seq_len)
    return MLQ_ERR_SHAPE;
  // validateForwardInputs (src/forward.cc:27-58) for host-side scalars
  if (token_dev == nullptr && (token < 0 || token >= m->vocab_size)) return MLQ_ERR_INVALID_ARG;
  if (pos_dev == nullptr && (pos < 0 || pos >= m->max_seq_len)) return MLQ_ERR_INVALID_ARG;

  const hipStream_t s = (hipStream_t)stream;
  const int dim = m->dim, hd = m->head_dim;
  const int qd = m->n_heads * hd, kvd = m->n_kv_heads * hd;
  auto linear = [&](const mlq_weight& w, const float* x, float* y, const float* bias,
                    int act) {
    return mlq_linear_epi(&w, x, y, 1, bias, act, b.lin, b.lin_bytes, stream);
  };
  auto hip = [](hipError_t e) { return record_hip(e); };
  // Linear of rmsNorm(x, norm): folded into the decode GEMV's activation
  // staging when that kernel runs the weight (quantized, one row), else a
  // separate RMSNorm pass into b.h first.
  auto norm_linear = [&](const mlq_weight& w, const float* x, const float* norm, float* y,
                         const float* bias, int act) {
    if (w.type != MLQ_F32 && w.k <= gemv_max_k(w.type, 1) && gemv_norm_supported(w)) {
      Epilogue e;
      e.bias = bias;
      e.act = act == MLQ_EPI_SWIGLU ? kEpiSwiGLU : kEpiNone;
      e.norm = norm;
      e.norm_eps = m->rms_norm_eps;
      return hip(launch_gemv(w, x, y, 1, s, e));
    }
    int rc = hip(launch_rmsnorm(x, norm, b.h, 1, dim, m->rms_norm_eps, s));
    if (rc != MLQ_OK) return rc;
    return linear(w, b.h, y, bias, act);
  };

  // Pre-scaled RMSNorm inputs: when every Linear of the step runs on the
  // decode GEMV, the producer of each residual-stream vector (the
  // embedding, the o and down projections) also writes x * next_norm and one
  // sum of x^2 per 16 elements, so the GEMVs that consume rmsNorm(x) read a
  // single vector and add those parts (no norm weight beside x in every
  // workgroup).
  const int parts = (dim + 15) / 16;
  auto gemv_pre = [&](const mlq_weight& w) {
    return w.type != MLQ_F32 && w.k <= gemv_max_k(w.type, 1) && gemv_prenorm_supported(w);
  };
  bool prenorm = parts <= kSsqPartsMax && gemv_pre(m->lm_head);
  for (int li = 0; li < m->n_layers && prenorm; ++li) {
    const mlq_layer& l = m->layers[li];
    prenorm = gemv_pre(l.wq) && gemv_pre(l.wo) && gemv_pre(l.w_gate) && gemv_pre(l.w_down) &&
              (qkv_fused(l) || (gemv_pre(l.wk) && gemv_pre(l.wv))) &&
              (glu_fused(l) || gemv_pre(l.w_up));
  }
  // Linear of rmsNorm(x, norm) from the pre-scaled input b.xn / b.ssq
  auto pre_linear = [&](const mlq_weight& w, float* y, const float* bias, int act) {
    Epilogue e;
    e.bias = bias;
    e.act = act == MLQ_EPI_SWIGLU ? kEpiSwiGLU : kEpiNone;
    e.ssq_parts = b.ssq;
    e.ssq_count = parts;
    e.norm_eps = m->rms_norm_eps;
    return hip(launch_gemv(w, b.xn, y, 1, s, e));
  };
  // y = residual + w . x, and the pre-scaled input rmsNorm(y, next_norm)
  auto produce = [&](const mlq_weight& w, const float* x, float* y, const float* residual,
                     const float* next_norm) {
    Epilogue e;
    e.bias = residual;
    e.next_norm = next_norm;
    e.next_x = b.xn;
    e.next_ssq = b.ssq;
    return hip(launch_gemv(w, x, y, 1, s, e));
  };
  auto any_norm_linear = [&](const mlq_weight& w, const float* x, const float* norm, float* y,
                             const float* bias, int act) {
    return prenorm ? pre_linear(w, y, bias, act) : norm_linear(w, x, norm, y, bias, act);
  };

  // RoPE and the cache write ride in the attention kernel where it can take
  // them (register kernel: head_dim 64 / 128 / 256, 16-byte aligned cache);
  // the embedding launch then also writes the step's RoPE table.
  const bool fused_rope = attention_fusable(hd, m->n_heads / m->n_kv_heads) &&
                          ((uintptr_t)c->keys & 15) == 0 && ((uintptr_t)c->values & 15) == 0;
  RopeTable rt;
  if (fused_rope) {
    rt.cs = b.rope;
    rt.pos_dev = pos_dev;
    rt.pos = pos;
    rt.hd = hd;
    rt.theta = m->rope_theta;
  }
  NormInput ni;
  if (prenorm) {
    ni.norm = m->layers[0].attn_norm;
    ni.xn = b.xn;
    ni.parts = b.ssq;
  }
  if ((rc = hip(launch_embedding(m->token_embedding, m->vocab_size, dim, token_dev, token,
                                 b.x, s, rt, ni))) != MLQ_OK)
    return rc;
  for (int li = 0; li < m->n_layers; ++li) {
    const mlq_layer& l = m->layers[li];
    // attention sublayer (forwardLayerDevice, src/forward.cc:607-640)
    if (qkv_fused(l)) {
      if ((rc = any_norm_linear(l.wq, b.x, l.attn_norm, b.qkv, l.bq, MLQ_EPI_NONE)) != MLQ_OK)
        return rc;
    } else {
      if ((rc = any_norm_linear(l.wq, b.x, l.attn_norm, b.qkv, l.bq, MLQ_EPI_NONE)) != MLQ_OK)
        return rc;
      if ((rc = any_norm_linear(l.wk, b.x, l.attn_norm, b.qkv + qd, l.bk, MLQ_EPI_NONE)) !=
          MLQ_OK)
        return rc;
      if ((rc = any_norm_linear(l.wv, b.x, l.attn_norm, b.qkv + qd + kvd, l.bv,
                                MLQ_EPI_NONE)) != MLQ_OK)
        return rc;
    }
    if (!fused_rope) {
      RopeLaunch r;
      r.q = b.qkv;
      r.k = b.qkv + qd;
      r.v = b.qkv + qd + kvd;
      r.keys = c->keys;
      r.values = c->values;
      r.n_heads = m->n_heads;
      r.n_kv = m->n_kv_heads;
      r.hd = hd;
      r.neox = m->rope_type == MLQ_ROPE_NEOX;
      r.layer = li;
      r.max_seq = c->max_seq_len;
      r.pos_limit = m->max_seq_len;
      r.pos_dev = pos_dev;
      r.pos = pos;
      r.theta = m->rope_theta;
      if ((rc = hip(launch_rope(r, s))) != MLQ_OK) return rc;
    }
    AttnLaunch a;
    a.q = b.qkv;
    a.keys = c->keys;
    a.values = c->values;
    a.out = b.attn;
    a.ws = b.apart;
    a.layer = li;
    a.max_seq = c->max_seq_len;
    a.n_heads = m->n_heads;
    a.n_kv = m->n_kv_heads;
    a.hd = hd;
    a.max_len = pos_dev != nullptr ? m->max_seq_len : pos + 1;
    // the model's limit (the cache may be larger): forwardToken's
    // pos < max_seq_len rule (src/forward.cc:42) for device positions
    a.pos_limit = m->max_seq_len;
    a.pos_dev = pos_dev;
    a.pos = pos;
    if (fused_rope) {
      a.k_new = b.qkv + qd;
      a.v_new = b.qkv + qd + kvd;
      a.rope_cs = b.rope;
      a.neox = m->rope_type == MLQ_ROPE_NEOX;
    }
    if ((rc = hip(launch_attention(a, s))) != MLQ_OK) return rc;
    // x2 = x + wo . attn: the residual enters as the projection's bias
    if (prenorm)
      rc = produce(l.wo, b.attn, b.x2, b.x, l.ffn_norm);
    else
      rc = linear(l.wo, b.attn, b.x2, b.x, MLQ_EPI_NONE);
    if (rc != MLQ_OK) return rc;
    // FFN sublayer
    if (glu_fused(l)) {
      if ((rc = any_norm_linear(l.w_gate, b.x2, l.ffn_norm, b.ffn, nullptr, MLQ_EPI_SWIGLU)) !=
          MLQ_OK)
        return rc;
    } else {
      if ((rc = any_norm_linear(l.w_gate, b.x2, l.ffn_norm, b.gate, nullptr, MLQ_EPI_NONE)) !=
          MLQ_OK)
        return rc;
      if ((rc = any_norm_linear(l.w_up, b.x2, l.ffn_norm, b.up, nullptr, MLQ_EPI_NONE)) !=
          MLQ_OK)
        return rc;
      if ((rc = hip(launch_eltwise(kEltSwiGLU, b.gate, b.up, b.ffn, m->hidden_dim, s))) != MLQ_OK)
        return rc;
    }
    // x = x2 + w_down . ffn
    if (prenorm)
      rc = produce(l.w_down, b.ffn, b.x, b.x2,
                   li + 1 < m->n_layers ? m->layers[li + 1].attn_norm : m->final_norm);
    else
      rc = linear(l.w_down, b.ffn, b.x, b.x2, MLQ_EPI_NONE);
    if (rc != MLQ_OK) return rc;
  }
  // computeLogitsDevice (src/forward.cc:736-745)
  return any_norm_linear(m->lm_head, b.x, m->final_norm, logits, nullptr, MLQ_EPI_NONE);
}

int mlq_prefill_workspace(const mlq_model* m, int n_tokens, size_t* bytes) {
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  PrefillBuffers b;
  const int rc = plan_prefill(m, n_tokens, nullptr, &b);
  if (rc != MLQ_OK) return rc;
  *bytes = b.total;
  return MLQ_OK;
}

int mlq_prefill(const mlq_model* m, const mlq_kv_cache* c, const int32_t* tokens, int n_tokens,
                int start_pos, float* logits, void* ws, size_t ws_bytes, mlq_stream_t stream) {
  PrefillBuffers b;
  int rc = plan_prefill(m, n_tokens, (char*)ws, &b);
  if (rc != MLQ_OK) return rc;
  if ((rc = check_cache(c)) != MLQ_OK) return rc;
  if (tokens == nullptr || logits == nullptr || ws == nullptr) return MLQ_ERR_INVALID_ARG;
  if (((uintptr_t)ws & 255u) != 0) return MLQ_ERR_INVALID_ARG;
  if (ws_bytes < b.total) return MLQ_ERR_BUFFER_TOO_SMALL;
  if (c->n_layers != m->n_layers || c->n_kv_heads != m->n_kv_heads ||
      c->head_dim != m->head_dim || c->max_seq_len < m->max_seq_len)
    return MLQ_ERR_SHAPE;
  // forwardBatch / validateForwardInputs (src/batch.cc:32-55,
  // src/forward.cc:27-58) for every token of the batch
  if (start_pos < 0 || start_pos > m->max_seq_len - n_tokens) return MLQ_ERR_INVALID_ARG;
  for (int i = 0; i < n_tokens; ++i)
    if (tokens[i] < 0 || tokens[i] >= m->vocab_size) return MLQ_ERR_INVALID_ARG;

  const hipStream_t s = (hipStream_t)stream;
  const int n = n_tokens, dim = m->dim, hd = m->head_dim, hid = m->hidden_dim;
  const int qd = m->n_heads * hd, kvd = m->n_kv_heads * hd;
  auto hip = [](hipError_t e) { return record_hip(e); };
  auto linear = [&](const mlq_weight& w, const float* x, float* y, int rows, const float* bias,
                    int act) {
    return mlq_linear_epi(&w, x, y, rows, bias, act, b.lin, b.lin_bytes, stream);
  };
  // Prefill GEMM rows (n > 64, quantized weights): the RMSNorm producer
  // writes the q|k|v and gate|up GEMMs' fp16 input directly (rows scaled by
  // their power-of-two exponents), and the o / down projections add the
  // residual in their epilogue, which removes two fp16 copy passes and two
  // residual passes per layer with the same roundings and additions
  // (GemmOut). The attention output and the SwiGLU output go through the
  // GEMMs' own fp16 copy pass, which needs the whole row for its exponent.
  auto gemm_rows = [&](const mlq_weight& w) { return n > kSkinnyMaxRows && w.type != MLQ_F32; };
  auto f16_norm_ok = [&](const float* norm) {
    return dim % 4 == 0 && ((uintptr_t)norm & 15) == 0 && dim <= 16 * 4 * 256;
  };
  // (xh rows are f16_row_stride(w.k) halves: w.k is dim or hidden, checked
  // by plan())
  auto gemm_f16 = [&](const mlq_weight& w, float* y, const Epilogue& e, const GemmOut& o) {
    return hip(launch_gemm_f16(w, b.xh, b.xexp, y, n, b.lin, b.lin_bytes, s, e, o));
  };
  const int ldx = f16_row_stride(dim);
  if ((rc = hip(hipMemcpyAsync(b.tokens, tokens, (size_t)n * sizeof(int32_t),
                               hipMemcpyHostToDevice, s))) != MLQ_OK)
    return rc;
  if ((rc = hip(launch_embedding_rows(m->token_embedding, dim, b.tokens, n, b.x, s))) != MLQ_OK)
    return rc;
  // the prompt's RoPE angles, once for every layer
  if ((rc = hip(launch_rope_table(b.rope, n, start_pos, hd, m->rope_theta, s))) != MLQ_OK)
    return rc;
  for (int li = 0; li < m->n_layers; ++li) {
    const mlq_layer& l = m->layers[li];
    RopeRows rr;
    const bool qkv_f16 = gemm_rows(l.wq) && (qkv_fused(l) || (gemm_rows(l.wk) && gemm_rows(l.wv))) &&
                         f16_norm_ok(l.attn_norm);
    auto proj = [&](const mlq_weight& w, float* y, const float* bias) {
      if (!qkv_f16) return linear(w, b.h, y, n, bias, MLQ_EPI_NONE);
      Epilogue e;
      e.bias = bias;
      return gemm_f16(w, y, e, GemmOut());
    };
    if (qkv_f16)
      rc = hip(launch_rmsnorm_f16(b.x, l.attn_norm, b.xh, b.xexp, n, dim, ldx, m->rms_norm_eps,
                                  s));
    else
      rc = hip(launch_rmsnorm(b.x, l.attn_norm, b.h, n, dim, m->rms_norm_eps, s));
    if (rc != MLQ_OK) return rc;
    if (qkv_fused(l)) {
      if ((rc = proj(l.wq, b.qkv, l.bq)) != MLQ_OK) return rc;
      rr.q = b.qkv;
      rr.k = b.qkv + qd;
      rr.v = b.qkv + qd + kvd;
      rr.q_stride = rr.k_stride = rr.v_stride = qd + 2 * kvd;
    } else {
      if ((rc = proj(l.wq, b.qkv, l.bq)) != MLQ_OK) return rc;
      if ((rc = proj(l.wk, b.k, l.bk)) != MLQ_OK) return rc;
      if ((rc = proj(l.wv, b.v, l.bv)) != MLQ_OK) return rc;
      rr.q = b.qkv;
      rr.k = b.k;
      rr.v = b.v;
      rr.q_stride = qd;
      rr.k_stride = rr.v_stride = kvd;
    }
    rr.rows = n;
    rr.keys = c->keys;
    rr.values = c->values;
    rr.n_heads = m->n_heads;
    rr.n_kv = m->n_kv_heads;
    rr.hd = hd;
    rr.neox = m->rope_type == MLQ_ROPE_NEOX;
    rr.layer = li;
    rr.max_seq = c->max_seq_len;
    rr.pos0 = start_pos;
    rr.theta = m->rope_theta;
    rr.cs = b.rope;
    if ((rc = hip(launch_rope_rows(rr, s))) != MLQ_OK) return rc;
    // causal attention: query row r sees cache positions 0..start_pos + r;
    // MFMA tiles of query rows where the head dims allow, else the decode
    // kernel over blocks of query rows
    const bool mfma_attn = prefill_attention_supported(hd, m->n_heads / m->n_kv_heads) &&
                           ((uintptr_t)c->keys & 15) == 0 && ((uintptr_t)c->values & 15) == 0;
    if (mfma_attn) {
      AttnLaunch a;
      a.q = rr.q;
      a.keys = c->keys;
      a.values = c->values;
      a.out = b.attn;
      a.layer = li;
      a.max_seq = c->max_seq_len;
      a.n_heads = m->n_heads;
      a.n_kv = m->n_kv_heads;
      a.hd = hd;
      a.pos = start_pos;
      a.rows = n;
      a.q_stride = rr.q_stride;
      a.out_stride = qd;
      if ((rc = hip(launch_attention_prefill(a, s))) != MLQ_OK) return rc;
    }
    for (int r0 = 0; !mfma_attn && r0 < n; r0 += kPrefillAttnRows) {
      const int nr = std::min(kPrefillAttnRows, n - r0);
      AttnLaunch a;
      a.q = rr.q + (size_t)r0 * rr.q_stride;
      a.keys = c->keys;
      a.values = c->values;
      a.out = b.attn + (size_t)r0 * qd;
      a.ws = b.apart;
      a.layer = li;
      a.max_seq = c->max_seq_len;
      a.n_heads = m->n_heads;
      a.n_kv = m->n_kv_heads;
      a.hd = hd;
      a.pos = start_pos + r0;
      a.max_len = start_pos + r0 + nr;
      a.rows = nr;
      a.q_stride = rr.q_stride;
      a.out_stride = qd;
      if ((rc = hip(launch_attention(a, s))) != MLQ_OK) return rc;
    }
    // x2 = x + wo . attn (the GEMM adds the residual row by row)
    if (gemm_rows(l.wo)) {
      GemmOut o;
      o.residual = b.x;
      if ((rc = hip(launch_gemm_ws(l.wo, b.attn, b.x2, n, b.lin, b.lin_bytes, s, Epilogue(),
                                   o))) != MLQ_OK)
        return rc;
    } else {
      if ((rc = linear(l.wo, b.attn, b.x2, n, nullptr, MLQ_EPI_NONE)) != MLQ_OK) return rc;
      if ((rc = hip(launch_eltwise(kEltAdd, b.x, b.x2, b.x2, (int64_t)n * dim, s))) != MLQ_OK)
        return rc;
    }
    // x = x2 + w_down . swiglu(w_gate . h, w_up . h); with gate|up
    // interleaved and prefill GEMM rows: fp16 input from RMSNorm, the SwiGLU
    // epilogue in the gate|up GEMM, residual in the down GEMM
    if (glu_fused(l) && gemm_rows(l.w_gate) && gemm_rows(l.w_down) &&
        f16_norm_ok(l.ffn_norm)) {
      if ((rc = hip(launch_rmsnorm_f16(b.x2, l.ffn_norm, b.xh, b.xexp, n, dim, ldx,
                                       m->rms_norm_eps, s))) != MLQ_OK)
        return rc;
      Epilogue eg;
      eg.act = kEpiSwiGLU;
      if ((rc = gemm_f16(l.w_gate, b.ffn, eg, GemmOut())) != MLQ_OK) return rc;
      GemmOut od;
      od.residual = b.x2;
      if ((rc = hip(launch_gemm_ws(l.w_down, b.ffn, b.x, n, b.lin, b.lin_bytes, s, Epilogue(),
                                   od))) != MLQ_OK)
        return rc;
      continue;
    }
    if ((rc = hip(launch_rmsnorm(b.x2, l.ffn_norm, b.h, n, dim, m->rms_norm_eps, s))) != MLQ_OK)
      return rc;
    if (glu_fused(l)) {
      if ((rc = linear(l.w_gate, b.h, b.ffn, n, nullptr, MLQ_EPI_SWIGLU)) != MLQ_OK) return rc;
    } else {
      if ((rc = linear(l.w_gate, b.h, b.gate, n, nullptr, MLQ_EPI_NONE)) != MLQ_OK) return rc;
      if ((rc = linear(l.w_up, b.h, b.up, n, nullptr, MLQ_EPI_NONE)) != MLQ_OK) return rc;
      if ((rc = hip(launch_eltwise(kEltSwiGLU, b.gate, b.up, b.ffn, (int64_t)n * hid, s))) !=
          MLQ_OK)
        return rc;
    }
    // x = x2 + w_down . ffn
    if ((rc = linear(l.w_down, b.ffn, b.h, n, nullptr, MLQ_EPI_NONE)) != MLQ_OK) return rc;
    if ((rc = hip(launch_eltwise(kEltAdd, b.x2, b.h, b.x, (int64_t)n * dim, s))) != MLQ_OK)
      return rc;
  }
  // logits of the last token only (forwardBatch returns those)
  const float* last = b.x + (size_t)(n - 1) * dim;
  const mlq_weight& w = m->lm_head;
  if (w.type != MLQ_F32 && w.k <= gemv_max_k(w.type, 1) && gemv_norm_supported(w)) {
    Epilogue e;
    e.norm = m->final_norm;
    e.norm_eps = m->rms_norm_eps;
    return hip(launch_gemv(w, last, logits, 1, s, e));
  }
  if ((rc = hip(launch_rmsnorm(last, m->final_norm, b.h, 1, dim, m->rms_norm_eps, s))) != MLQ_OK)
    return rc;
  return linear(w, b.h, logits, 1, nullptr, MLQ_EPI_NONE);
}

}  // extern "C"
