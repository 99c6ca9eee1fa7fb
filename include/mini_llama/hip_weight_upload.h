// Weight upload for the HIP backend (mirrors
// include/mini_llama/cuda_weight_upload.h:18-111).
//
// Difference from the reference: quantized Linear weights are REPACKED on
// upload (host side, then one copy) from GGUF AoS blocks into the tiled
// layout of mlq.h (16-row tiles, 1 KiB wave lines, split scale/min arrays).
// The uploaded buffer is registered, so passing `buffer.data()` to the
// hipQ*LinearDevice* functions takes the repacked fast path while raw AoS
// device pointers keep the reference meaning (see hip_quant.h).
#ifndef MINI_LLAMA_HIP_WEIGHT_UPLOAD_H_
#define MINI_LLAMA_HIP_WEIGHT_UPLOAD_H_

#include <cstddef>
#include <string>
#include <vector>

#include "mini_llama/hip_runtime.h"
#include "mini_llama/quantized_tensor.h"
#include "mini_llama/tensor.h"
#include "mlq.h"

namespace mini_llama {

struct HipUploadedWeight {
  std::string name;
  QuantType type = QuantType::kF32;
  bool linear = true;
  std::vector<int> shape;
  size_t block_count = 0;  // GGUF blocks of the source (0 for F32)
  HipDeviceBuffer buffer;  // F32: raw floats; quantized: tiled layout
  mlq_weight layout{};     // quantized only: region offsets inside buffer
};

struct HipModelWeights {
  int device_id = 0;

  size_t uploaded_weight_count = 0;
  size_t uploaded_bytes = 0;

  size_t linear_calls = 0;
  size_t activation_calls = 0;
  size_t attention_calls = 0;
  size_t attention_cpu_fallbacks = 0;
  size_t kv_cache_write_bytes = 0;
  size_t kv_cache_read_bytes = 0;
  size_t host_to_device_copies = 0;
  size_t device_to_host_copies = 0;
  size_t host_to_device_bytes = 0;
  size_t device_to_host_bytes = 0;

  std::vector<HipUploadedWeight> weights;
};

void uploadF32LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id);
void uploadF32TensorWeight(HipModelWeights& storage, const Tensor& weight,
                           const std::string& name, int device_id);
void uploadQ80LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id);
void uploadQ40LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id);
void uploadQ41LinearWeight(HipModelWeights& storage,
                           const QuantizedTensor& weight,
                           const std::string& name, int device_id);
void uploadLinearWeight(HipModelWeights& storage, const QuantizedTensor& weight,
                        const std::string& name, int device_id);

// Name + type lookup (the reference's findCudaWeight, src/forward.cc:64-73).
const HipUploadedWeight* findHipWeight(const HipModelWeights& storage,
                                       const std::string& name, QuantType type);

void recordHipLinearCall(HipModelWeights& storage);
void recordHipLinearCopy(HipModelWeights& storage, size_t h2d_bytes,
                         size_t d2h_bytes);
void recordHipHostToDeviceCopy(HipModelWeights& storage, size_t bytes);
void resetHipRuntimeStats(HipModelWeights& storage);

// Registry of device buffers that hold tiled weights (keyed by base pointer;
// entries are removed when the owning HipDeviceBuffer frees the memory).
void registerTiledWeight(const void* device_base, const mlq_weight& layout);
void unregisterTiledWeight(const void* device_base);
bool lookupTiledWeight(const void* device_base, mlq_weight* layout);

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_WEIGHT_UPLOAD_H_
