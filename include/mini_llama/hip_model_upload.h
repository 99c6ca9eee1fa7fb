// Model-level weight upload for the HIP backend: the twin of
// uploadModelWeightsToCuda and its helpers (include/mini_llama/model.h:78-99,
// src/model.cc:151-219).
//
// The reference's MiniLlamaModel (model.h:52-61) lives with its loader and
// CPU engine, which are not part of this backend, so these are templates
// over the model type. Any type with MiniLlamaModel's weight fields works:
//   bool loaded; Tensor token_embedding, final_norm; QuantizedTensor lm_head;
//   layers: a sequence of LayerWeights (model.h:37-50: attention_norm, wq,
//   wk, wv, bq, bk, bv, wo, ffn_norm, w_gate, w_up, w_down);
//   std::shared_ptr<HipModelWeights> hip_weights (the member the drop-in adds
//   beside cuda_weights, model.h:60).
// Weights are uploaded under the reference's names and in its order
// ("token_embedding", "final_norm", "lm_head", "layers.<i>.wq", ...), so the
// name lookups of the device forward pass (findHipWeight, the twin of
// findCudaWeight, src/forward.cc:64-73) find them. Quantized Linear weights
// are repacked into the tiled layout on upload (hip_weight_upload.h); empty
// optional biases are skipped, as the reference skips them.
#ifndef MINI_LLAMA_HIP_MODEL_UPLOAD_H_
#define MINI_LLAMA_HIP_MODEL_UPLOAD_H_

#include <cstddef>
#include <memory>
#include <stdexcept>
#include <string>

#include "mini_llama/hip_runtime.h"
#include "mini_llama/hip_weight_upload.h"

namespace mini_llama {

// Uploads every weight of a loaded model to `device_id`; afterwards
// model.hip_weights != nullptr. Throws like uploadModelWeightsToCuda when
// the model is not loaded, and propagates the per-weight upload errors.
template <class Model>
void uploadModelWeightsToHip(Model& model, int device_id = 0) {
  if (!model.loaded) {
    throw std::runtime_error("HIP weight upload requires a loaded model");
  }
  hipSetDeviceId(device_id);
  auto storage = std::make_shared<HipModelWeights>();
  storage->device_id = device_id;

  // global weights
  uploadF32TensorWeight(*storage, model.token_embedding, "token_embedding", device_id);
  uploadF32TensorWeight(*storage, model.final_norm, "final_norm", device_id);
  uploadLinearWeight(*storage, model.lm_head, "lm_head", device_id);

  // per-layer weights: attention, then FFN
  for (size_t layer = 0; layer < model.layers.size(); ++layer) {
    const auto& lw = model.layers[layer];
    const std::string prefix = "layers." + std::to_string(layer) + ".";
    uploadF32TensorWeight(*storage, lw.attention_norm, prefix + "attention_norm", device_id);
    uploadLinearWeight(*storage, lw.wq, prefix + "wq", device_id);
    uploadLinearWeight(*storage, lw.wk, prefix + "wk", device_id);
    uploadLinearWeight(*storage, lw.wv, prefix + "wv", device_id);
    uploadF32TensorWeight(*storage, lw.bq, prefix + "bq", device_id);
    uploadF32TensorWeight(*storage, lw.bk, prefix + "bk", device_id);
    uploadF32TensorWeight(*storage, lw.bv, prefix + "bv", device_id);
    uploadLinearWeight(*storage, lw.wo, prefix + "wo", device_id);
    uploadF32TensorWeight(*storage, lw.ffn_norm, prefix + "ffn_norm", device_id);
    uploadLinearWeight(*storage, lw.w_gate, prefix + "w_gate", device_id);
    uploadLinearWeight(*storage, lw.w_up, prefix + "w_up", device_id);
    uploadLinearWeight(*storage, lw.w_down, prefix + "w_down", device_id);
  }
  model.hip_weights = std::move(storage);
}

// Releases the model's device weights (clearModelCudaWeights).
template <class Model>
void clearModelHipWeights(Model& model) {
  model.hip_weights.reset();
}

// True once uploadModelWeightsToHip has run (modelHasCudaWeights).
template <class Model>
bool modelHasHipWeights(const Model& model) {
  return model.hip_weights != nullptr;
}

// Uploaded weight count and device bytes (modelCudaUploadedWeightCount,
// modelCudaMemoryBytes); 0 before the upload.
template <class Model>
size_t modelHipUploadedWeightCount(const Model& model) {
  return model.hip_weights ? model.hip_weights->uploaded_weight_count : 0;
}

template <class Model>
size_t modelHipMemoryBytes(const Model& model) {
  return model.hip_weights ? model.hip_weights->uploaded_bytes : 0;
}

// Zeroes the runtime counters between inference runs: model.h:97 declares
// resetModelCudaRuntimeStats (the reference defines only the storage-level
// resetCudaRuntimeStats, src/cuda_weight_upload.cc:314); this one calls its
// twin resetHipRuntimeStats on the model's storage.
template <class Model>
void resetModelHipRuntimeStats(Model& model) {
  if (model.hip_weights) resetHipRuntimeStats(*model.hip_weights);
}

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_MODEL_UPLOAD_H_
