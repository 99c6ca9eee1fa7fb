// Device-resident KV cache of the HIP backend: the CudaKvCache class of
// include/mini_llama/cuda_kv_cache.h:28-95 with a hip name. Layout (keys
// and values alike): [n_layers][max_seq_len][n_kv_heads][head_dim] fp32, so
// view() hands the same memory to the libmlq attention and decode-step
// entry points (mlq_kv_cache). Validation and messages follow
// src/cuda_kv_cache.cc.
#ifndef MINI_LLAMA_HIP_KV_CACHE_H_
#define MINI_LLAMA_HIP_KV_CACHE_H_

#include <cstddef>

#include "mini_llama/hip_runtime.h"
#include "mini_llama/hip_tensor.h"
#include "mini_llama/tensor.h"
#include "mlq.h"

namespace mini_llama {

bool hipKvCacheBuilt();

class HipKvCache {
 public:
  HipKvCache() = default;
  HipKvCache(int n_layers, int max_seq_len, int n_kv_heads, int head_dim, int device_id = 0);

  HipKvCache(const HipKvCache&) = delete;
  HipKvCache& operator=(const HipKvCache&) = delete;
  HipKvCache(HipKvCache&&) noexcept = default;
  HipKvCache& operator=(HipKvCache&&) noexcept = default;

  void reset();
  void reset(int n_layers, int max_seq_len, int n_kv_heads, int head_dim, int device_id = 0);

  // Fills both caches with zeros.
  void clear();

  // k, v: [n_kv_heads, head_dim] host tensors.
  void write(int layer, int pos, const Tensor& k, const Tensor& v);
  // k, v: device tensors of n_kv_heads * head_dim elements (device to device).
  void writeDevice(int layer, int pos, const HipTensor& k, const HipTensor& v);

  Tensor readKey(int layer, int pos) const;
  Tensor readValue(int layer, int pos) const;
  Tensor readKeyHead(int layer, int pos, int kv_head) const;
  Tensor readValueHead(int layer, int pos, int kv_head) const;

  const void* keysData() const;
  const void* valuesData() const;
  // The cache as the C ABI describes it (device pointers borrowed).
  mlq_kv_cache view() const;

  bool empty() const;
  size_t bytes() const;

  int nLayers() const { return n_layers_; }
  int maxSeqLen() const { return max_seq_len_; }
  int nKvHeads() const { return n_kv_heads_; }
  int headDim() const { return head_dim_; }
  int deviceId() const { return device_id_; }

 private:
  void validateIndices(int layer, int pos) const;
  void validateHeadIndex(int kv_head) const;
  size_t slotOffsetBytes(int layer, int pos) const;
  Tensor readSlice(const HipDeviceBuffer& buf, size_t offset, const std::vector<int>& shape) const;

  int n_layers_ = 0;
  int max_seq_len_ = 0;
  int n_kv_heads_ = 0;
  int head_dim_ = 0;
  int device_id_ = 0;
  HipDeviceBuffer keys_;
  HipDeviceBuffer values_;
};

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_KV_CACHE_H_
