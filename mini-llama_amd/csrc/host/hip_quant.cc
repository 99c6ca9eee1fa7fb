// Quantized Linear host layer of the HIP backend: the nine entry points of
// include/mini_llama/cuda_quant.h with the reference's validation, output
// shapes and error messages (src/cuda_quant.cu:188-517), calling the C ABI
// launchers of libmlq (include/mlq.h).
#include "mini_llama/hip_quant.h"

#include <hip/hip_runtime_api.h>

#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "host_common.h"
#include "mini_llama/hip_matmul.h"
#include "mlq.h"

namespace mini_llama {
namespace {

// Status -> exception in the style of checkCudaQuant (src/cuda_quant.cu:20-29).
void checkStatus(int rc, const char* what) { checkMlq(rc, "HIP quant error in", what); }

int quantInFeatures(const std::vector<int>& x_shape, const std::string& x_str,
                    const char* caller) {
  if (x_shape.size() == 1) return x_shape[0];
  if (x_shape.size() == 2) return x_shape[1];
  throw std::runtime_error(
      std::string(caller) +
      ": expected x shape [in_features] or [batch, in_features], got " + x_str);
}

// validateQuantLinearShape (src/cuda_quant.cu:198-227).
void validateQuantLinearShape(const std::vector<int>& x_shape,
                              const std::string& x_str,
                              const std::vector<int>& w_shape,
                              size_t block_count, int block_size,
                              const char* caller) {
  if (w_shape.size() != 2) {
    throw std::runtime_error(std::string(caller) +
                             ": expected weight shape [out_features, in_features]");
  }
  const int in_feat = quantInFeatures(x_shape, x_str, caller);
  if (in_feat <= 0 || w_shape[0] <= 0 || w_shape[1] <= 0 ||
      (x_shape.size() == 2 && x_shape[0] <= 0)) {
    throw std::runtime_error(std::string(caller) +
                             ": empty tensors are not supported");
  }
  if (w_shape[1] != in_feat) {
    throw std::runtime_error(std::string(caller) + ": dimension mismatch x=" +
                             x_str + " weight=[" + std::to_string(w_shape[0]) +
                             ", " + std::to_string(w_shape[1]) + "]");
  }
  const int blocks_per_row = (in_feat + block_size - 1) / block_size;
  const size_t expected = static_cast<size_t>(w_shape[0]) * blocks_per_row;
  if (block_count != expected) {
    throw std::runtime_error(std::string(caller) +
                             ": block count mismatch: expected " +
                             std::to_string(expected) + ", got " +
                             std::to_string(block_count));
  }
}

struct LinearParams {
  bool input_is_1d;
  int rows;
  int in_features;
  int out_features;
};

LinearParams computeLinearParams(const std::vector<int>& x_shape,
                                 const std::vector<int>& w_shape) {
  LinearParams p;
  p.input_is_1d = x_shape.size() == 1;
  p.rows = p.input_is_1d ? 1 : x_shape[0];
  p.in_features = p.input_is_1d ? x_shape[0] : x_shape[1];
  p.out_features = w_shape[0];
  return p;
}

std::vector<int> outputShape(const LinearParams& p) {
  return p.input_is_1d ? std::vector<int>{p.out_features}
                       : std::vector<int>{p.rows, p.out_features};
}

void addBiasInPlace(Tensor& y, const Tensor& bias, int rows, int cols) {
  if (static_cast<int>(bias.size()) != cols) {
    throw std::runtime_error("hipQuantLinear: bias size " +
                             std::to_string(bias.size()) +
                             " does not match out_features " +
                             std::to_string(cols));
  }
  for (int row = 0; row < rows; ++row)
    for (int col = 0; col < cols; ++col)
      y.data[static_cast<size_t>(row) * cols + col] += bias.data[col];
}

// Runs y = x W^T for a device weight pointer: a registered tiled buffer goes
// straight to the kernels, anything else is taken as GGUF AoS blocks.
void runLinear(int type, const void* w_dev, size_t block_count,
               const LinearParams& p, const float* x, float* y, int device_id,
               const char* caller) {
  mlq_weight layout;
  int rc;
  if (lookupTiledWeight(w_dev, &layout)) {
    if (layout.type != type || layout.n != p.out_features ||
        layout.k != p.in_features) {
      throw std::runtime_error(std::string(caller) +
                               ": uploaded weight has a different type or shape");
    }
    size_t ws_bytes = 0;
    rc = mlq_linear_workspace(&layout, p.rows, &ws_bytes);
    checkStatus(rc, caller);
    Workspace ws;
    if (ws_bytes) ws = deviceWorkspace(kActivationWorkspace, device_id, ws_bytes);
    rc = mlq_linear_ws(&layout, x, y, p.rows, ws.data, ws_bytes, nullptr);
  } else {
    // GGUF blocks as they are: up to 8 rows read them directly (no
    // workspace), more are repacked into the per-device workspace first
    size_t need = 0;
    rc = mlq_linear_aos_workspace(type, p.out_features, p.in_features, p.rows, &need);
    checkStatus(rc, caller);
    Workspace ws;
    if (need) ws = deviceWorkspace(kAosWorkspace, device_id, need);
    rc = mlq_linear_aos(type, w_dev, block_count, p.out_features, p.in_features,
                        x, y, p.rows, ws.data, need, nullptr);
  }
  checkStatus(rc, "mlq_linear");
}

Tensor linearDeviceWeight(int type, int block_size, const Tensor& x,
                          const void* w_dev, size_t block_count,
                          const std::vector<int>& weight_shape,
                          const Tensor* bias, int device_id,
                          const char* caller) {
  if (w_dev == nullptr)
    throw std::runtime_error(std::string(caller) + ": null weight pointer");
  validateQuantLinearShape(x.shape, x.shapeString(), weight_shape, block_count,
                           block_size, caller);
  hipSetDeviceId(device_id);
  const LinearParams p = computeLinearParams(x.shape, weight_shape);
  Tensor y(outputShape(p), 0.0f);
  HipDeviceBuffer x_dev(x.size() * sizeof(float), device_id);
  HipDeviceBuffer y_dev(y.size() * sizeof(float), device_id);
  x_dev.upload(x.data.data(), x.size() * sizeof(float));
  runLinear(type, w_dev, block_count, p, static_cast<const float*>(x_dev.data()),
            static_cast<float*>(y_dev.data()), device_id, caller);
  y_dev.download(y.data.data(), y.size() * sizeof(float));
  if (bias != nullptr) addBiasInPlace(y, *bias, p.rows, p.out_features);
  return y;
}

HipTensor linearDeviceInput(int type, int block_size, const HipTensor& x,
                            const void* w_dev, size_t block_count,
                            const std::vector<int>& weight_shape, int device_id,
                            const char* caller) {
  if (w_dev == nullptr)
    throw std::runtime_error(std::string(caller) + ": null weight pointer");
  if (x.deviceId() != device_id)
    throw std::runtime_error(std::string(caller) +
                             ": input tensor on different HIP device");
  validateQuantLinearShape(x.shape(), x.shapeString(), weight_shape,
                           block_count, block_size, caller);
  hipSetDeviceId(device_id);
  const LinearParams p = computeLinearParams(x.shape(), weight_shape);
  HipTensor y(outputShape(p), device_id);
  runLinear(type, w_dev, block_count, p, static_cast<const float*>(x.data()),
            static_cast<float*>(y.data()), device_id, caller);
  return y;
}

template <typename Block>
Tensor linearHostWeight(int type, int block_size, const Tensor& x,
                        const std::vector<Block>& weight,
                        const std::vector<int>& weight_shape, const Tensor* bias,
                        int device_id, const char* caller) {
  validateQuantLinearShape(x.shape, x.shapeString(), weight_shape,
                           weight.size(), block_size, caller);
  HipDeviceBuffer w_dev(weight.size() * sizeof(Block), device_id);
  w_dev.upload(weight.data(), weight.size() * sizeof(Block));
  return linearDeviceWeight(type, block_size, x, w_dev.data(), weight.size(),
                            weight_shape, bias, device_id, caller);
}

}  // namespace

bool hipQuantBuilt() { return true; }

// ---- Q8_0 -------------------------------------------------------------------
Tensor hipQ80Linear(const Tensor& x, const std::vector<BlockQ80>& weight,
                    const std::vector<int>& weight_shape, const Tensor* bias,
                    int device_id) {
  return linearHostWeight(MLQ_Q8_0, kQ80BlockSize, x, weight, weight_shape,
                          bias, device_id, "hipQ80Linear");
}

Tensor hipQ80LinearDeviceWeight(const Tensor& x, const void* q8_0_device,
                                size_t q8_0_block_count,
                                const std::vector<int>& weight_shape,
                                const Tensor* bias, int device_id) {
  return linearDeviceWeight(MLQ_Q8_0, kQ80BlockSize, x, q8_0_device,
                            q8_0_block_count, weight_shape, bias, device_id,
                            "hipQ80Linear");
}

HipTensor hipQ80LinearDeviceInput(const HipTensor& x, const void* q8_0_device,
                                  size_t q8_0_block_count,
                                  const std::vector<int>& weight_shape,
                                  int device_id) {
  return linearDeviceInput(MLQ_Q8_0, kQ80BlockSize, x, q8_0_device,
                           q8_0_block_count, weight_shape, device_id,
                           "hipQ80LinearDeviceInput");
}

// ---- Q4_0 -------------------------------------------------------------------
Tensor hipQ40Linear(const Tensor& x, const std::vector<BlockQ40>& weight,
                    const std::vector<int>& weight_shape, const Tensor* bias,
                    int device_id) {
  return linearHostWeight(MLQ_Q4_0, kQ40BlockSize, x, weight, weight_shape,
                          bias, device_id, "hipQ40Linear");
}

Tensor hipQ40LinearDeviceWeight(const Tensor& x, const void* q4_0_device,
                                size_t q4_0_block_count,
                                const std::vector<int>& weight_shape,
                                const Tensor* bias, int device_id) {
  return linearDeviceWeight(MLQ_Q4_0, kQ40BlockSize, x, q4_0_device,
                            q4_0_block_count, weight_shape, bias, device_id,
                            "hipQ40Linear");
}

HipTensor hipQ40LinearDeviceInput(const HipTensor& x, const void* q4_0_device,
                                  size_t q4_0_block_count,
                                  const std::vector<int>& weight_shape,
                                  int device_id) {
  return linearDeviceInput(MLQ_Q4_0, kQ40BlockSize, x, q4_0_device,
                           q4_0_block_count, weight_shape, device_id,
                           "hipQ40LinearDeviceInput");
}

// ---- Q4_1 -------------------------------------------------------------------
Tensor hipQ41Linear(const Tensor& x, const std::vector<BlockQ41>& weight,
                    const std::vector<int>& weight_shape, const Tensor* bias,
                    int device_id) {
  return linearHostWeight(MLQ_Q4_1, kQ41BlockSize, x, weight, weight_shape,
                          bias, device_id, "hipQ41Linear");
}

Tensor hipQ41LinearDeviceWeight(const Tensor& x, const void* q4_1_device,
                                size_t q4_1_block_count,
                                const std::vector<int>& weight_shape,
                                const Tensor* bias, int device_id) {
  return linearDeviceWeight(MLQ_Q4_1, kQ41BlockSize, x, q4_1_device,
                            q4_1_block_count, weight_shape, bias, device_id,
                            "hipQ41Linear");
}

HipTensor hipQ41LinearDeviceInput(const HipTensor& x, const void* q4_1_device,
                                  size_t q4_1_block_count,
                                  const std::vector<int>& weight_shape,
                                  int device_id) {
  return linearDeviceInput(MLQ_Q4_1, kQ41BlockSize, x, q4_1_device,
                           q4_1_block_count, weight_shape, device_id,
                           "hipQ41LinearDeviceInput");
}

// ---- uploaded weights ---------------------------------------------------------
HipTensor hipLinearUploaded(const HipTensor& x, const HipUploadedWeight& weight,
                            int device_id) {
  static constexpr const char* kCaller = "hipLinearUploaded";
  if (x.deviceId() != device_id || weight.buffer.device_id() != device_id)
    throw std::runtime_error(std::string(kCaller) +
                             ": tensors on different HIP devices");
  if (weight.type == QuantType::kF32) {
    // F32 projections: the fp32 GEMV over the raw rows, as forwardLinearDevice
    // sends them to cudaLinearDeviceInput (src/forward.cc:206-209)
    return hipLinearDeviceInput(x, weight.buffer.data(), weight.shape, device_id);
  }
  validateQuantLinearShape(x.shape(), x.shapeString(), weight.shape,
                           weight.block_count, 32, kCaller);
  hipSetDeviceId(device_id);
  const LinearParams p = computeLinearParams(x.shape(), weight.shape);
  HipTensor y(outputShape(p), device_id);
  size_t ws_bytes = 0;
  checkStatus(mlq_linear_workspace(&weight.layout, p.rows, &ws_bytes), kCaller);
  Workspace ws;
  if (ws_bytes) ws = deviceWorkspace(kActivationWorkspace, device_id, ws_bytes);
  checkStatus(mlq_linear_ws(&weight.layout, static_cast<const float*>(x.data()),
                            static_cast<float*>(y.data()), p.rows, ws.data, ws_bytes,
                            nullptr),
              "mlq_linear_ws");
  return y;
}

}  // namespace mini_llama
