// HipKvCache (include/mini_llama/hip_kv_cache.h): the reference cache's
// checks and messages (src/cuda_kv_cache.cc:16-335); writes from the device
// go through mlq_kv_write (stream-ordered on the null stream).
#include "mini_llama/hip_kv_cache.h"

#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "host_common.h"

namespace mini_llama {
namespace {

void requirePositive(int v, const char* name) {
  if (v <= 0) throw std::runtime_error(std::string("HipKvCache: ") + name + " must be positive");
}

size_t checkedMul(size_t a, size_t b, const char* label) {
  if (a != 0 && b > std::numeric_limits<size_t>::max() / a)
    throw std::runtime_error(std::string("HipKvCache: size overflow for ") + label);
  return a * b;
}

}  // namespace

bool hipKvCacheBuilt() { return true; }

HipKvCache::HipKvCache(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                       int device_id) {
  reset(n_layers, max_seq_len, n_kv_heads, head_dim, device_id);
}

void HipKvCache::reset() {
  keys_.reset();
  values_.reset();
  n_layers_ = max_seq_len_ = n_kv_heads_ = head_dim_ = device_id_ = 0;
}

void HipKvCache::reset(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                       int device_id) {
  requirePositive(n_layers, "n_layers");
  requirePositive(max_seq_len, "max_seq_len");
  requirePositive(n_kv_heads, "n_kv_heads");
  requirePositive(head_dim, "head_dim");
  size_t elems = checkedMul((size_t)n_layers, (size_t)max_seq_len, "layers * seq");
  elems = checkedMul(elems, (size_t)n_kv_heads, "layers * seq * heads");
  elems = checkedMul(elems, (size_t)head_dim, "layers * seq * heads * dim");
  const size_t bytes = checkedMul(elems, sizeof(float), "cache bytes");
  n_layers_ = n_layers;
  max_seq_len_ = max_seq_len;
  n_kv_heads_ = n_kv_heads;
  head_dim_ = head_dim;
  device_id_ = device_id;
  keys_.reset(bytes, device_id);
  values_.reset(bytes, device_id);
  clear();
}

void HipKvCache::clear() {
  if (empty()) return;
  hipSetDeviceId(device_id_);
  const std::vector<float> zeros(keys_.bytes() / sizeof(float), 0.0f);
  keys_.upload(zeros.data(), keys_.bytes());
  values_.upload(zeros.data(), values_.bytes());
}

void HipKvCache::write(int layer, int pos, const Tensor& k, const Tensor& v) {
  validateIndices(layer, pos);
  if (k.numDims() != 2 || v.numDims() != 2 || k.shape != v.shape)
    throw std::out_of_range("HipKvCache::write expected matching [n_kv_heads, head_dim] tensors");
  if (k.shape[0] != n_kv_heads_ || k.shape[1] != head_dim_)
    throw std::out_of_range("HipKvCache::write tensor shape does not match cache shape");
  const size_t off = slotOffsetBytes(layer, pos);
  hipSetDeviceId(device_id_);
  hipMemcpyBytes(static_cast<char*>(keys_.data()) + off, k.data.data(), k.size() * sizeof(float),
                 HipMemcpyKind::kHostToDevice);
  hipMemcpyBytes(static_cast<char*>(values_.data()) + off, v.data.data(),
                 v.size() * sizeof(float), HipMemcpyKind::kHostToDevice);
}

void HipKvCache::writeDevice(int layer, int pos, const HipTensor& k, const HipTensor& v) {
  validateIndices(layer, pos);
  if (k.deviceId() != device_id_ || v.deviceId() != device_id_)
    throw std::runtime_error("HipKvCache::writeDevice tensor is on a different HIP device");
  const size_t expected = (size_t)n_kv_heads_ * (size_t)head_dim_;
  if (k.size() != expected || v.size() != expected)
    throw std::out_of_range("HipKvCache::writeDevice tensor shape does not match cache shape");
  hipSetDeviceId(device_id_);
  const mlq_kv_cache c = view();
  checkMlq(mlq_kv_write(&c, layer, pos, static_cast<const float*>(k.data()),
                        static_cast<const float*>(v.data()), nullptr),
           "HIP KV cache error in", "HipKvCache::writeDevice");
}

Tensor HipKvCache::readSlice(const HipDeviceBuffer& buf, size_t offset,
                             const std::vector<int>& shape) const {
  Tensor out(shape, 0.0f);
  hipSetDeviceId(device_id_);
  hipMemcpyBytes(out.data.data(), static_cast<const char*>(buf.data()) + offset,
                 out.size() * sizeof(float), HipMemcpyKind::kDeviceToHost);
  return out;
}

Tensor HipKvCache::readKey(int layer, int pos) const {
  validateIndices(layer, pos);
  return readSlice(keys_, slotOffsetBytes(layer, pos), {n_kv_heads_, head_dim_});
}

Tensor HipKvCache::readValue(int layer, int pos) const {
  validateIndices(layer, pos);
  return readSlice(values_, slotOffsetBytes(layer, pos), {n_kv_heads_, head_dim_});
}

Tensor HipKvCache::readKeyHead(int layer, int pos, int kv_head) const {
  validateIndices(layer, pos);
  validateHeadIndex(kv_head);
  return readSlice(keys_, slotOffsetBytes(layer, pos) + (size_t)kv_head * head_dim_ * 4,
                   {head_dim_});
}

Tensor HipKvCache::readValueHead(int layer, int pos, int kv_head) const {
  validateIndices(layer, pos);
  validateHeadIndex(kv_head);
  return readSlice(values_, slotOffsetBytes(layer, pos) + (size_t)kv_head * head_dim_ * 4,
                   {head_dim_});
}

const void* HipKvCache::keysData() const {
  if (empty()) throw std::runtime_error("HipKvCache: cache is empty");
  return keys_.data();
}

const void* HipKvCache::valuesData() const {
  if (empty()) throw std::runtime_error("HipKvCache: cache is empty");
  return values_.data();
}

mlq_kv_cache HipKvCache::view() const {
  mlq_kv_cache c;
  c.keys = static_cast<float*>(const_cast<void*>(keysData()));
  c.values = static_cast<float*>(const_cast<void*>(valuesData()));
  c.n_layers = n_layers_;
  c.max_seq_len = max_seq_len_;
  c.n_kv_heads = n_kv_heads_;
  c.head_dim = head_dim_;
  return c;
}

bool HipKvCache::empty() const { return keys_.empty() || values_.empty(); }

size_t HipKvCache::bytes() const { return keys_.bytes() + values_.bytes(); }

void HipKvCache::validateIndices(int layer, int pos) const {
  if (empty()) throw std::runtime_error("HipKvCache: cache is empty");
  if (layer < 0 || layer >= n_layers_) throw std::out_of_range("HipKvCache layer out of range");
  if (pos < 0 || pos >= max_seq_len_) throw std::out_of_range("HipKvCache position out of range");
}

void HipKvCache::validateHeadIndex(int kv_head) const {
  if (kv_head < 0 || kv_head >= n_kv_heads_) throw std::out_of_range("HipKvCache head out of range");
}

size_t HipKvCache::slotOffsetBytes(int layer, int pos) const {
  return (((size_t)layer * max_seq_len_ + pos) * n_kv_heads_ * head_dim_) * sizeof(float);
}

}  // namespace mini_llama
