// Weight upload for the HIP backend (mirrors src/cuda_weight_upload.cc:21-325)
// with a host-side repack of GGUF AoS blocks into the tiled layout, and the
// registry that lets the raw-pointer Linear entry points recognise uploaded
// (tiled) buffers.
#include "mini_llama/hip_weight_upload.h"

#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace mini_llama {
namespace {

std::mutex& registryMutex() {
  static std::mutex m;
  return m;
}

std::unordered_map<const void*, mlq_weight>& registry() {
  static std::unordered_map<const void*, mlq_weight> r;
  return r;
}

void throwIfEmpty(const std::string& name, const std::string& format) {
  throw std::runtime_error("HIP weight upload: empty " + format +
                           " data for " + name);
}

int mlqType(QuantType t) {
  switch (t) {
    case QuantType::kQ80: return MLQ_Q8_0;
    case QuantType::kQ40: return MLQ_Q4_0;
    case QuantType::kQ41: return MLQ_Q4_1;
    default: return MLQ_F32;
  }
}

// Shape and block-count checks of uploadQ*LinearWeight
// (src/cuda_weight_upload.cc:118-139), then host repack + one H2D copy.
void uploadQuantized(HipModelWeights& storage, const QuantizedTensor& weight,
                     const std::string& name, int device_id, const void* blocks,
                     size_t block_count, const char* format) {
  if (weight.shape.size() != 2) {
    throw std::runtime_error("HIP weight upload: expected 2D " +
                             std::string(format) + " weight for " + name);
  }
  if (block_count == 0) throwIfEmpty(name, format);
  const int out_features = weight.shape[0];
  const int in_features = weight.shape[1];
  if (out_features <= 0 || in_features <= 0) {
    throw std::runtime_error("HIP weight upload: non-positive shape " +
                             weight.shapeString() + " for " + name);
  }
  const size_t blocks_per_row = (size_t)(in_features + 31) / 32;
  const size_t expected = (size_t)out_features * blocks_per_row;
  if (block_count != expected) {
    throw std::runtime_error("HIP weight upload: " + std::string(format) +
                             " block count mismatch for " + name +
                             ", expected " + std::to_string(expected) +
                             ", got " + std::to_string(block_count));
  }
  const int type = mlqType(weight.type);
  mlq_weight layout;
  int rc = mlq_weight_layout(type, out_features, in_features, &layout);
  if (rc != MLQ_OK)
    throw std::runtime_error("HIP weight upload: " +
                             std::string(mlq_status_string(rc)) + " for " + name);
  std::vector<unsigned char> staged(layout.bytes);
  rc = mlq_repack_host(type, blocks, block_count, out_features, in_features,
                       staged.data(), staged.size());
  if (rc != MLQ_OK)
    throw std::runtime_error("HIP weight upload: repack failed (" +
                             std::string(mlq_status_string(rc)) + ") for " +
                             name);
  HipUploadedWeight uploaded;
  uploaded.name = name;
  uploaded.type = weight.type;
  uploaded.linear = true;
  uploaded.shape = weight.shape;
  uploaded.block_count = block_count;
  uploaded.buffer.reset(layout.bytes, device_id);
  uploaded.buffer.upload(staged.data(), layout.bytes);
  layout.base = uploaded.buffer.data();
  uploaded.layout = layout;
  registerTiledWeight(layout.base, layout);

  storage.uploaded_weight_count += 1;
  storage.uploaded_bytes += layout.bytes;
  storage.weights.push_back(std::move(uploaded));
}

}  // namespace

void registerTiledWeight(const void* device_base, const mlq_weight& layout) {
  std::lock_guard<std::mutex> lock(registryMutex());
  registry()[device_base] = layout;
}

void unregisterTiledWeight(const void* device_base) {
  std::lock_guard<std::mutex> lock(registryMutex());
  registry().erase(device_base);
}

bool lookupTiledWeight(const void* device_base, mlq_weight* layout) {
  std::lock_guard<std::mutex> lock(registryMutex());
  auto it = registry().find(device_base);
  if (it == registry().end()) return false;
  if (layout) *layout = it->second;
  return true;
}

void uploadF32LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id) {
  if (weight.type != QuantType::kF32) return;
  if (weight.f32_data.empty()) throwIfEmpty(name, "F32");
  const size_t expected = weight.num_elements();
  if (weight.f32_data.size() != expected) {
    throw std::runtime_error("HIP weight upload: data size mismatch for " +
                             name + ", expected " + std::to_string(expected) +
                             ", got " + std::to_string(weight.f32_data.size()));
  }
  const size_t bytes = weight.f32_data.size() * sizeof(float);
  HipUploadedWeight uploaded;
  uploaded.name = name;
  uploaded.type = QuantType::kF32;
  uploaded.linear = true;
  uploaded.shape = weight.shape;
  uploaded.buffer.reset(bytes, device_id);
  uploaded.buffer.upload(weight.f32_data.data(), bytes);
  storage.uploaded_weight_count += 1;
  storage.uploaded_bytes += bytes;
  storage.weights.push_back(std::move(uploaded));
}

void uploadF32TensorWeight(HipModelWeights& storage, const Tensor& weight,
                           const std::string& name, int device_id) {
  if (weight.data.empty()) return;
  // data must hold the shape's element count (the reference's message,
  // src/cuda_weight_upload.cc:75-81, whose comparison of data.size() with
  // size() == data.size() cannot fail; the shape product is what it names)
  size_t expected = weight.shape.empty() ? weight.data.size() : 1;
  for (const int d : weight.shape) expected *= (size_t)(d > 0 ? d : 0);
  if (weight.data.size() != expected) {
    throw std::runtime_error("HIP weight upload: tensor data size mismatch for " + name +
                             ", expected " + std::to_string(expected) + ", got " +
                             std::to_string(weight.data.size()));
  }
  const size_t bytes = weight.data.size() * sizeof(float);
  HipUploadedWeight uploaded;
  uploaded.name = name;
  uploaded.type = QuantType::kF32;
  uploaded.linear = false;
  uploaded.shape = weight.shape;
  uploaded.buffer.reset(bytes, device_id);
  uploaded.buffer.upload(weight.data.data(), bytes);
  storage.uploaded_weight_count += 1;
  storage.uploaded_bytes += bytes;
  storage.weights.push_back(std::move(uploaded));
}

void uploadQ80LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id) {
  if (weight.type != QuantType::kQ80) return;
  uploadQuantized(storage, weight, name, device_id, weight.q8_0_data.data(),
                  weight.q8_0_data.size(), "Q8_0");
}

void uploadQ40LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id) {
  if (weight.type != QuantType::kQ40) return;
  uploadQuantized(storage, weight, name, device_id, weight.q4_0_data.data(),
                  weight.q4_0_data.size(), "Q4_0");
}

void uploadQ41LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id) {
  if (weight.type != QuantType::kQ41) return;
  uploadQuantized(storage, weight, name, device_id, weight.q4_1_data.data(),
                  weight.q4_1_data.size(), "Q4_1");
}

void uploadLinearWeight(HipModelWeights& storage, const QuantizedTensor& weight,
                        const std::string& name, int device_id) {
  uploadF32LinearWeight(storage, weight, name, device_id);
  uploadQ80LinearWeight(storage, weight, name, device_id);
  uploadQ40LinearWeight(storage, weight, name, device_id);
  uploadQ41LinearWeight(storage, weight, name, device_id);
}

const HipUploadedWeight* findHipWeight(const HipModelWeights& storage,
                                       const std::string& name,
                                       QuantType type) {
  for (const auto& w : storage.weights)
    if (w.name == name && w.type == type) return &w;
  return nullptr;
}

void recordHipLinearCall(HipModelWeights& storage) { storage.linear_calls += 1; }

void recordHipLinearCopy(HipModelWeights& storage, size_t h2d_bytes,
                         size_t d2h_bytes) {
  storage.linear_calls += 1;
  storage.host_to_device_copies += 1;
  storage.device_to_host_copies += 1;
  storage.host_to_device_bytes += h2d_bytes;
  storage.device_to_host_bytes += d2h_bytes;
}

void recordHipHostToDeviceCopy(HipModelWeights& storage, size_t bytes) {
  storage.host_to_device_copies += 1;
  storage.host_to_device_bytes += bytes;
}

void resetHipRuntimeStats(HipModelWeights& storage) {
  storage.linear_calls = 0;
  storage.activation_calls = 0;
  storage.attention_calls = 0;
  storage.attention_cpu_fallbacks = 0;
  storage.kv_cache_write_bytes = 0;
  storage.kv_cache_read_bytes = 0;
  storage.host_to_device_copies = 0;
  storage.device_to_host_copies = 0;
  storage.host_to_device_bytes = 0;
  storage.device_to_host_bytes = 0;
}

}  // namespace mini_llama
