// C ABI of the mlq library (declarations and contracts in include/mlq.h).
// Validates like the reference launch layer (src/cuda_quant.cu:188-227) but
// reports through return codes; launches are stream-ordered and never
// synchronize.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "kernels/launch.h"
#include "mlq.h"
#include "mlq_layout.h"

using namespace mlq;

namespace {

thread_local int g_last_hip_error = 0;

int hip_status(hipError_t e) {
  if (e == hipSuccess) return MLQ_OK;
  g_last_hip_error = (int)e;
  return MLQ_ERR_HIP;
}

bool quant_type(int type) {
  return type == MLQ_Q8_0 || type == MLQ_Q4_0 || type == MLQ_Q4_1;
}

// Shape / block-count checks shared by every entry point
// (validateQuantLinearShape, src/cuda_quant.cu:198-227).
int check_weight(int type, size_t block_count, int n, int k) {
  if (!quant_type(type)) return MLQ_ERR_INVALID_ARG;
  if (n <= 0 || k <= 0) return MLQ_ERR_SHAPE;
  const size_t nb = (size_t)((k + kQK - 1) / kQK);
  if (block_count != (size_t)n * nb) return MLQ_ERR_BLOCK_COUNT;
  return MLQ_OK;
}

int check_tiled(const mlq_weight* w);

// A Linear weight: tiled quantized, or plain fp32 rows (type MLQ_F32).
int check_linear_weight(const mlq_weight* w) {
  if (w == nullptr || w->base == nullptr) return MLQ_ERR_INVALID_ARG;
  if (w->type != MLQ_F32) return check_tiled(w);
  if (w->n <= 0 || w->k <= 0) return MLQ_ERR_SHAPE;
  if (w->bytes < (uint64_t)w->n * (uint64_t)w->k * sizeof(float)) return MLQ_ERR_INVALID_ARG;
  return MLQ_OK;
}

int check_tiled(const mlq_weight* w) {
  if (w == nullptr || w->base == nullptr) return MLQ_ERR_INVALID_ARG;
  if (!quant_type(w->type)) return MLQ_ERR_INVALID_ARG;
  if (w->n <= 0 || w->k <= 0) return MLQ_ERR_SHAPE;
  mlq_weight expect;
  mlq_weight_layout(w->type, w->n, w->k, &expect);
  if (w->nb != expect.nb || w->qs_off != expect.qs_off ||
      w->d_off != expect.d_off || w->m_off != expect.m_off ||
      w->bytes < expect.bytes)
    return MLQ_ERR_INVALID_ARG;
  return MLQ_OK;
}

// The automatic kernel choice: the decode GEMV for up to kGemvMaxRows rows
// when its activation staging fits LDS, the MFMA GEMM otherwise.
bool uses_gemv(const mlq_weight* w, int m) {
  return m <= kGemvMaxRows && w->k <= gemv_max_k(w->type, m);
}

}  // namespace

namespace mlq {
// MLQ status of a HIP result, recorded for mlq_last_hip_error (gguf.cpp).
int record_hip(hipError_t e) { return hip_status(e); }
}  // namespace mlq

extern "C" {

const char* mlq_status_string(int status) {
  switch (status) {
    case MLQ_OK: return "ok";
    case MLQ_ERR_INVALID_ARG: return "invalid argument";
    case MLQ_ERR_SHAPE: return "shape mismatch";
    case MLQ_ERR_BLOCK_COUNT: return "block count mismatch";
    case MLQ_ERR_BUFFER_TOO_SMALL: return "buffer too small";
    case MLQ_ERR_UNSUPPORTED: return "unsupported shape";
    case MLQ_ERR_NO_DEVICE: return "no HIP device";
    case MLQ_ERR_FORMAT: return "malformed GGUF file";
    case MLQ_ERR_SCRATCH_LIMIT: return "shape needs more than the fixed no-alloc scratch";
    case MLQ_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

int mlq_last_hip_error(void) { return g_last_hip_error; }

int mlq_device_count(int* count) {
  if (count == nullptr) return MLQ_ERR_INVALID_ARG;
  int c = 0;
  const hipError_t e = hipGetDeviceCount(&c);
  if (e != hipSuccess || c <= 0) {
    *count = 0;
    return MLQ_ERR_NO_DEVICE;
  }
  *count = c;
  return MLQ_OK;
}

size_t mlq_block_bytes(int type) {
  switch (type) {
    case MLQ_Q8_0: return 34;
    case MLQ_Q4_0: return 18;
    case MLQ_Q4_1: return 20;
    default: return 0;
  }
}

int mlq_weight_layout(int type, int n, int k, mlq_weight* out) {
  if (out == nullptr || !(quant_type(type) || type == MLQ_F32)) return MLQ_ERR_INVALID_ARG;
  if (n <= 0 || k <= 0) return MLQ_ERR_SHAPE;
  if (type == MLQ_F32) {
    mlq_weight w;
    std::memset(&w, 0, sizeof w);
    w.type = type;
    w.n = n;
    w.k = k;
    w.nb = (k + kQK - 1) / kQK;
    w.bytes = (uint64_t)n * (uint64_t)k * sizeof(float);
    *out = w;
    return MLQ_OK;
  }
  const Geometry geo = geometry(n, k);
  const uint64_t qbytes = unit_count(geo) * kLanes * quant_bytes_per_lane(type);
  const uint64_t sbytes = scale_count(geo) * 2;
  mlq_weight w;
  std::memset(&w, 0, sizeof w);
  w.type = type;
  w.n = n;
  w.k = k;
  w.nb = geo.nb;
  uint64_t off = 0;
  w.qs_off = off;
  off = align_up(off + qbytes, kRegionAlign);
  w.d_off = off;
  off = align_up(off + sbytes, kRegionAlign);
  if (type == MLQ_Q4_1) {
    w.m_off = off;
    off = align_up(off + sbytes, kRegionAlign);
  }
  w.bytes = off;
  *out = w;
  return MLQ_OK;
}

int mlq_repack_host(int type, const void* aos, size_t block_count, int n, int k,
                    void* dst, size_t dst_bytes) {
  int rc = check_weight(type, block_count, n, k);
  if (rc != MLQ_OK) return rc;
  if (aos == nullptr || dst == nullptr) return MLQ_ERR_INVALID_ARG;
  mlq_weight w;
  mlq_weight_layout(type, n, k, &w);
  if (dst_bytes < w.bytes) return MLQ_ERR_BUFFER_TOO_SMALL;
  const Geometry geo = geometry(n, k);
  const size_t bb = mlq_block_bytes(type);
  const uint8_t* src = (const uint8_t*)aos;
  uint8_t* base = (uint8_t*)dst;
  // Gaps between regions stay defined (zero); every slot is then written.
  std::memset(base, 0, w.bytes);
  uint8_t* qs = base + w.qs_off;
  uint16_t* d = (uint16_t*)(base + w.d_off);
  uint16_t* m = type == MLQ_Q4_1 ? (uint16_t*)(base + w.m_off) : nullptr;
  const int rows = geo.nt * kTileRows;
  const int bpr = geo.g * kGroupBlocks;
  for (int row = 0; row < rows; ++row) {
    for (int b = 0; b < bpr; ++b) {
      const bool real = row < n && b < geo.nb;
      const uint8_t* blk = real ? src + ((size_t)row * geo.nb + b) * bb : nullptr;
      repack_block(type, geo, row, b, blk, qs, d, m);
    }
  }
  return MLQ_OK;
}

int mlq_repack_device(int type, const void* aos_dev, size_t block_count, int n,
                      int k, void* dst_dev, size_t dst_bytes,
                      mlq_stream_t stream) {
  int rc = check_weight(type, block_count, n, k);
  if (rc != MLQ_OK) return rc;
  if (aos_dev == nullptr || dst_dev == nullptr) return MLQ_ERR_INVALID_ARG;
  mlq_weight w;
  mlq_weight_layout(type, n, k, &w);
  if (dst_bytes < w.bytes) return MLQ_ERR_BUFFER_TOO_SMALL;
  w.base = dst_dev;
  return hip_status(launch_repack(type, aos_dev, n, k, w, (hipStream_t)stream));
}

int mlq_dequantize(const mlq_weight* w, int row0, int rows, float* out,
                   mlq_stream_t stream) {
  int rc = check_tiled(w);
  if (rc != MLQ_OK) return rc;
  if (out == nullptr) return MLQ_ERR_INVALID_ARG;
  if (row0 < 0 || rows <= 0 || row0 + rows > w->n) return MLQ_ERR_SHAPE;
  return hip_status(launch_dequant(*w, row0, rows, out, (hipStream_t)stream));
}

int mlq_quantize_act_q8_0(const float* x, int rows, int row_size, void* out,
                          size_t out_bytes, mlq_stream_t stream) {
  if (x == nullptr || out == nullptr) return MLQ_ERR_INVALID_ARG;
  if (rows <= 0 || row_size <= 0) return MLQ_ERR_SHAPE;
  const size_t need = (size_t)rows * (size_t)((row_size + 31) / 32) * 34;
  if (out_bytes < need) return MLQ_ERR_BUFFER_TOO_SMALL;
  return hip_status(launch_quantize_act_q8_0(x, rows, row_size, out, (hipStream_t)stream));
}

int mlq_linear_path(const mlq_weight* w, const float* x, float* y, int m,
                    int path, mlq_stream_t stream) {
  int rc = check_linear_weight(w);
  if (rc != MLQ_OK) return rc;
  if (x == nullptr || y == nullptr) return MLQ_ERR_INVALID_ARG;
  if (m <= 0) return MLQ_ERR_SHAPE;
  if (w->type == MLQ_F32) {
    if (path != MLQ_PATH_AUTO && path != MLQ_PATH_GEMV)
      return path == MLQ_PATH_MFMA ? MLQ_ERR_UNSUPPORTED : MLQ_ERR_INVALID_ARG;
    return hip_status(
        launch_linear_f32((const float*)w->base, w->n, w->k, x, y, m, (hipStream_t)stream));
  }
  const bool gemv_fits = uses_gemv(w, m);
  bool use_gemv;
  switch (path) {
    case MLQ_PATH_AUTO: use_gemv = gemv_fits; break;
    case MLQ_PATH_GEMV:
      if (!gemv_fits) return MLQ_ERR_UNSUPPORTED;
      use_gemv = true;
      break;
    case MLQ_PATH_MFMA: use_gemv = false; break;
    default: return MLQ_ERR_INVALID_ARG;
  }
  const hipStream_t s = (hipStream_t)stream;
  return hip_status(use_gemv ? launch_gemv(*w, x, y, m, s)
                             : launch_gemm(*w, x, y, m, s));
}

int mlq_linear(const mlq_weight* w, const float* x, float* y, int m,
               mlq_stream_t stream) {
  return mlq_linear_path(w, x, y, m, MLQ_PATH_AUTO, stream);
}

int mlq_linear_workspace(const mlq_weight* w, int m, size_t* bytes) {
  int rc = check_linear_weight(w);
  if (rc != MLQ_OK) return rc;
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  if (m <= 0) return MLQ_ERR_SHAPE;
  *bytes = w->type == MLQ_F32 || uses_gemv(w, m) ? 0
           : m <= kSkinnyMaxRows ? skinny_workspace_bytes(w->type, m, w->n, w->k)
                                 : gemm_workspace_bytes(m, w->n, w->k);
  return MLQ_OK;
}

int mlq_linear_epi(const mlq_weight* w, const float* x, float* y, int m,
                   const float* bias, int act, void* workspace,
                   size_t workspace_bytes, mlq_stream_t stream) {
  int rc = check_linear_weight(w);
  if (rc != MLQ_OK) return rc;
  if (x == nullptr || y == nullptr) return MLQ_ERR_INVALID_ARG;
  if (m <= 0) return MLQ_ERR_SHAPE;
  if (act != MLQ_EPI_NONE && act != MLQ_EPI_SWIGLU) return MLQ_ERR_INVALID_ARG;
  if (act == MLQ_EPI_SWIGLU && w->n % 16 != 0) return MLQ_ERR_SHAPE;
  Epilogue epi;
  epi.bias = bias;
  epi.act = act == MLQ_EPI_SWIGLU ? kEpiSwiGLU : kEpiNone;
  const hipStream_t s = (hipStream_t)stream;
  if (w->type == MLQ_F32)
    return hip_status(launch_linear_f32((const float*)w->base, w->n, w->k, x, y, m, s, epi));
  if (uses_gemv(w, m)) return hip_status(launch_gemv(*w, x, y, m, s, epi));
  const size_t need = m <= kSkinnyMaxRows ? skinny_workspace_bytes(w->type, m, w->n, w->k)
                                           : gemm_workspace_bytes(m, w->n, w->k);
  if (need > 0) {
    if (workspace == nullptr || workspace_bytes < need) return MLQ_ERR_BUFFER_TOO_SMALL;
    if (((uintptr_t)workspace & 255u) != 0) return MLQ_ERR_INVALID_ARG;
  }
  if (m <= kSkinnyMaxRows)  // batched decode: skinny GEMM (+ split-K reduce)
    return hip_status(launch_skinny_ws(*w, x, y, m, workspace, workspace_bytes, s, epi));
  return hip_status(launch_gemm_ws(*w, x, y, m, workspace, workspace_bytes, s, epi));
}

int mlq_linear_ws(const mlq_weight* w, const float* x, float* y, int m,
                  void* workspace, size_t workspace_bytes,
                  mlq_stream_t stream) {
  return mlq_linear_epi(w, x, y, m, nullptr, MLQ_EPI_NONE, workspace,
                        workspace_bytes, stream);
}

int mlq_linear_q8act_workspace(const mlq_weight* w, int m, size_t* bytes) {
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  int rc = check_tiled(w);
  if (rc != MLQ_OK) return rc;
  if (w->type != MLQ_Q8_0) return MLQ_ERR_UNSUPPORTED;
  if (m <= 0) return MLQ_ERR_SHAPE;
  *bytes = gemm_i8_workspace_bytes(*w, m);
  return MLQ_OK;
}

int mlq_linear_q8act(const mlq_weight* w, const float* x, float* y, int m,
                     void* workspace, size_t workspace_bytes, mlq_stream_t stream) {
  size_t need = 0;
  int rc = mlq_linear_q8act_workspace(w, m, &need);
  if (rc != MLQ_OK) return rc;
  if (x == nullptr || y == nullptr || workspace == nullptr) return MLQ_ERR_INVALID_ARG;
  if (((uintptr_t)workspace & 255u) != 0) return MLQ_ERR_INVALID_ARG;
  if (workspace_bytes < need) return MLQ_ERR_BUFFER_TOO_SMALL;
  return hip_status(launch_gemm_i8(*w, x, y, m, workspace, (hipStream_t)stream));
}

int mlq_interleave_rows(const void* gate, const void* up, int rows,
                        size_t row_bytes, void* out) {
  if (gate == nullptr || up == nullptr || out == nullptr || row_bytes == 0)
    return MLQ_ERR_INVALID_ARG;
  if (rows <= 0 || rows % 8 != 0) return MLQ_ERR_SHAPE;
  const uint8_t* g = (const uint8_t*)gate;
  const uint8_t* u = (const uint8_t*)up;
  uint8_t* o = (uint8_t*)out;
  // output rows 16t + c = gate row 8t + c, 16t + 8 + c = up row 8t + c
  for (int t = 0; t < rows / 8; ++t) {
    std::memcpy(o + (size_t)16 * t * row_bytes, g + (size_t)8 * t * row_bytes, 8 * row_bytes);
    std::memcpy(o + (size_t)(16 * t + 8) * row_bytes, u + (size_t)8 * t * row_bytes,
                8 * row_bytes);
  }
  return MLQ_OK;
}

int mlq_linear_aos_workspace(int type, int n, int k, int m, size_t* bytes) {
  if (bytes == nullptr) return MLQ_ERR_INVALID_ARG;
  if (n <= 0 || k <= 0 || m <= 0) return MLQ_ERR_SHAPE;
  mlq_weight w;
  const int rc = mlq_weight_layout(type, n, k, &w);
  if (rc != MLQ_OK) return rc;
  *bytes = aos_gemv_supported(type, m, n, k) ? 0 : (size_t)w.bytes;
  return MLQ_OK;
}

int mlq_linear_aos(int type, const void* aos_dev, size_t block_count, int n,
                   int k, const float* x, float* y, int m, void* workspace,
                   size_t workspace_bytes, mlq_stream_t stream) {
  int rc = check_weight(type, block_count, n, k);
  if (rc != MLQ_OK) return rc;
  if (aos_dev == nullptr || x == nullptr || y == nullptr) return MLQ_ERR_INVALID_ARG;
  if (m <= 0) return MLQ_ERR_SHAPE;
  // up to 8 rows whose x fits in LDS: one pass over the blocks as they are
  if (aos_gemv_supported(type, m, n, k))
    return hip_status(launch_aos_gemv(type, aos_dev, n, k, x, y, m, (hipStream_t)stream));
  if (workspace == nullptr) return MLQ_ERR_INVALID_ARG;
  mlq_weight w;
  mlq_weight_layout(type, n, k, &w);
  if (workspace_bytes < w.bytes) return MLQ_ERR_BUFFER_TOO_SMALL;
  w.base = workspace;
  const hipStream_t s = (hipStream_t)stream;
  rc = hip_status(launch_repack(type, aos_dev, n, k, w, s));
  if (rc != MLQ_OK) return rc;
  return mlq_linear(&w, x, y, m, stream);
}

int mlq_set_gemm_split(int split) {
  if (split < 0 || split > 64) return MLQ_ERR_INVALID_ARG;
  set_gemm_split(split);
  return MLQ_OK;
}

int mlq_set_skinny_plan(int tiles, int splits) {
  const bool tiles_ok = tiles == 0 || tiles == 1 || tiles == 2 || tiles == 4;
  if (!tiles_ok || splits < 0 || splits > 8) return MLQ_ERR_INVALID_ARG;
  set_skinny_plan(tiles, splits);
  return MLQ_OK;
}

int mlq_set_gemv_split(int split) {
  const bool split_ok = split == 0 || split == 1 || split == 2 || split == 4 ||
                        split == 8 || split == 16;
  if (!split_ok) return MLQ_ERR_INVALID_ARG;
  set_gemv_split(split);
  return MLQ_OK;
}

int mlq_add_bias(float* y, const float* bias, int m, int n,
                 mlq_stream_t stream) {
  if (y == nullptr || bias == nullptr) return MLQ_ERR_INVALID_ARG;
  if (m <= 0 || n <= 0) return MLQ_ERR_SHAPE;
  return hip_status(launch_bias(y, bias, m, n, (hipStream_t)stream));
}

}  // extern "C"
