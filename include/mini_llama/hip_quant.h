// Quantized Linear on the HIP backend: y = x @ W^T (+ bias).
//
// Drop-in for include/mini_llama/cuda_quant.h:13-76: the same nine entry
// points (cuda -> hip), same argument meaning, same validation and
// std::runtime_error messages (src/cuda_quant.cu:188-227), same output rank
// rule (x [K] -> y [N], x [M, K] -> y [M, N]).
//
// Weight pointer meaning for the DeviceWeight / DeviceInput variants:
//  - a buffer produced by the HIP upload path (hip_weight_upload.h) is
//    recognised through the tiled-weight registry and used directly;
//  - any other pointer is taken, like the reference, as raw GGUF AoS blocks
//    in device memory; it is repacked into a per-device workspace first.
// All device work runs on the null stream. *Linear and *DeviceWeight return
// after the result is on the host; *DeviceInput returns without waiting.
#ifndef MINI_LLAMA_HIP_QUANT_H_
#define MINI_LLAMA_HIP_QUANT_H_

#include <cstddef>
#include <vector>

#include "mini_llama/hip_tensor.h"
#include "mini_llama/hip_weight_upload.h"
#include "mini_llama/quantized_tensor.h"
#include "mini_llama/tensor.h"

namespace mini_llama {

bool hipQuantBuilt();

// ---- Q8_0 ------------------------------------------------------------------
Tensor hipQ80Linear(const Tensor& x, const std::vector<BlockQ80>& weight,
                    const std::vector<int>& weight_shape,
                    const Tensor* bias = nullptr, int device_id = 0);
Tensor hipQ80LinearDeviceWeight(const Tensor& x, const void* q8_0_device,
                                size_t q8_0_block_count,
                                const std::vector<int>& weight_shape,
                                const Tensor* bias = nullptr,
                                int device_id = 0);
HipTensor hipQ80LinearDeviceInput(const HipTensor& x, const void* q8_0_device,
                                  size_t q8_0_block_count,
                                  const std::vector<int>& weight_shape,
                                  int device_id = 0);

// ---- Q4_0 ------------------------------------------------------------------
Tensor hipQ40Linear(const Tensor& x, const std::vector<BlockQ40>& weight,
                    const std::vector<int>& weight_shape,
                    const Tensor* bias = nullptr, int device_id = 0);
Tensor hipQ40LinearDeviceWeight(const Tensor& x, const void* q4_0_device,
                                size_t q4_0_block_count,
                                const std::vector<int>& weight_shape,
                                const Tensor* bias = nullptr,
                                int device_id = 0);
HipTensor hipQ40LinearDeviceInput(const HipTensor& x, const void* q4_0_device,
                                  size_t q4_0_block_count,
                                  const std::vector<int>& weight_shape,
                                  int device_id = 0);

// ---- Q4_1 ------------------------------------------------------------------
Tensor hipQ41Linear(const Tensor& x, const std::vector<BlockQ41>& weight,
                    const std::vector<int>& weight_shape,
                    const Tensor* bias = nullptr, int device_id = 0);
Tensor hipQ41LinearDeviceWeight(const Tensor& x, const void* q4_1_device,
                                size_t q4_1_block_count,
                                const std::vector<int>& weight_shape,
                                const Tensor* bias = nullptr,
                                int device_id = 0);
HipTensor hipQ41LinearDeviceInput(const HipTensor& x, const void* q4_1_device,
                                  size_t q4_1_block_count,
                                  const std::vector<int>& weight_shape,
                                  int device_id = 0);

// ---- Uploaded-weight entry (forwardLinearDevice-style callers) -------------
// Runs the tiled fast path for a quantized weight from uploadLinearWeight,
// and an F32 weight through the fp32 GEMV (hipLinearDeviceInput), as
// forwardLinearDevice sends F32 projections to cudaLinearDeviceInput
// (src/forward.cc:206-209).
HipTensor hipLinearUploaded(const HipTensor& x, const HipUploadedWeight& weight,
                            int device_id = 0);

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_QUANT_H_
