// Decode attention host layer (include/mini_llama/hip_attention.h): the
// reference's checks and messages (src/cuda_attention.cu:44-118) over
// mlq_attention_decode, with the partials in a grow-only per-device
// workspace (no allocation per call once it has grown).
#include "mini_llama/hip_attention.h"

#include <stdexcept>
#include <string>

#include "host_common.h"

namespace mini_llama {
namespace {

void validateCommon(const HipKvCache& kv, int layer, int pos, int n_heads, int n_kv_heads,
                    int head_dim, const std::string& caller) {
  if (kv.empty()) throw std::runtime_error(caller + ": KV cache is empty");
  if (layer < 0 || layer >= kv.nLayers()) throw std::out_of_range(caller + ": layer out of range");
  if (pos < 0 || pos >= kv.maxSeqLen()) throw std::out_of_range(caller + ": position out of range");
  if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0)
    throw std::runtime_error(caller + ": head counts and head_dim must be positive");
  if (n_heads % n_kv_heads != 0)
    throw std::runtime_error(caller + ": n_heads must be divisible by n_kv_heads");
}

void run(const float* q, float* out, const HipKvCache& kv, int layer, int pos, int n_heads,
         int device_id, const char* caller) {
  const mlq_kv_cache c = kv.view();
  size_t ws_bytes = 0;
  checkMlq(mlq_attention_workspace(&c, n_heads, &ws_bytes), "HIP attention error in", caller);
  Workspace ws = deviceWorkspace(kAttentionWorkspace, device_id, ws_bytes);
  checkMlq(mlq_attention_decode(&c, layer, pos, q, n_heads, out, ws.data, ws_bytes, nullptr),
           "HIP attention error in", caller);
}

}  // namespace

bool hipAttentionBuilt() { return true; }

Tensor hipAttentionDecode(const Tensor& q, const HipKvCache& kv_cache, int layer, int pos,
                          int n_heads, int n_kv_heads, int head_dim, int device_id) {
  if (q.shape != std::vector<int>{n_heads, head_dim})
    throw std::runtime_error("hipAttentionDecode: expected q shape [" + std::to_string(n_heads) +
                             ", " + std::to_string(head_dim) + "], got " + q.shapeString());
  validateCommon(kv_cache, layer, pos, n_heads, n_kv_heads, head_dim, "hipAttentionDecode");
  if (kv_cache.nKvHeads() != n_kv_heads || kv_cache.headDim() != head_dim)
    throw std::runtime_error(
        "hipAttentionDecode: KV cache shape does not match attention shape");
  hipSetDeviceId(device_id);
  HipTensor qd = hipTensorFromHost(q, device_id);
  HipTensor out({n_heads, head_dim}, device_id);
  run(static_cast<const float*>(qd.data()), static_cast<float*>(out.data()), kv_cache, layer, pos,
      n_heads, device_id, "hipAttentionDecode");
  return out.download();
}

HipTensor hipAttentionDecodeDeviceInput(const HipTensor& q, const HipKvCache& kv_cache,
                                        int layer, int pos, int n_heads, int n_kv_heads,
                                        int head_dim, int device_id) {
  static const std::string kCaller = "hipAttentionDecodeDeviceInput";
  if (q.deviceId() != device_id) throw std::runtime_error(kCaller + ": q on different HIP device");
  if (q.size() != (size_t)n_heads * (size_t)head_dim)
    throw std::runtime_error(kCaller + ": q shape mismatch");
  validateCommon(kv_cache, layer, pos, n_heads, n_kv_heads, head_dim, kCaller);
  if (kv_cache.nKvHeads() != n_kv_heads || kv_cache.headDim() != head_dim ||
      kv_cache.deviceId() != device_id)
    throw std::runtime_error(kCaller + ": KV cache shape or device mismatch");
  hipSetDeviceId(device_id);
  HipTensor out({n_heads * head_dim}, device_id);
  run(static_cast<const float*>(q.data()), static_cast<float*>(out.data()), kv_cache, layer, pos,
      n_heads, device_id, "hipAttentionDecodeDeviceInput");
  return out;
}

}  // namespace mini_llama
