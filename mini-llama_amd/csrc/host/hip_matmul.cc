// F32 Linear / matmul host layer (include/mini_llama/hip_matmul.h): the
// reference's validation and messages (src/cuda_matmul.cc:93-241) over the
// fp32 GEMV of libmlq.
#include "mini_llama/hip_matmul.h"

#include <stdexcept>
#include <string>

#include "host_common.h"
#include "mlq.h"

namespace mini_llama {
namespace {

int linearInFeatures(const std::vector<int>& x_shape, const std::string& x_str,
                     const char* caller) {
  if (x_shape.size() == 1) return x_shape[0];
  if (x_shape.size() == 2) return x_shape[1];
  throw std::runtime_error(std::string(caller) +
                           ": expected x shape [in_features] or [batch, in_features], got " +
                           x_str);
}

// validateLinearShape (src/cuda_matmul.cc:120-136), plus the empty-shape
// check the fp32 GEMV needs (cuBLAS would reject such a call too).
void validateLinearShape(const std::vector<int>& x_shape, const std::string& x_str,
                         const std::vector<int>& w_shape, const char* caller) {
  if (w_shape.size() != 2)
    throw std::runtime_error(std::string(caller) +
                             ": expected weight shape [out_features, in_features]");
  const int in_features = linearInFeatures(x_shape, x_str, caller);
  if (w_shape[1] != in_features)
    throw std::runtime_error(std::string(caller) + ": dimension mismatch x=" + x_str +
                             " weight=[" + std::to_string(w_shape[0]) + ", " +
                             std::to_string(w_shape[1]) + "]");
  if (in_features <= 0 || w_shape[0] <= 0 || (x_shape.size() == 2 && x_shape[0] <= 0))
    throw std::runtime_error(std::string(caller) + ": empty tensors are not supported");
}

std::vector<int> outputShape(const std::vector<int>& x_shape, int out_features) {
  return x_shape.size() == 1 ? std::vector<int>{out_features}
                             : std::vector<int>{x_shape[0], out_features};
}

// y[rows, out] = x[rows, in] W^T on the device.
void runF32(const float* x, const void* w_device, int rows, int out_features, int in_features,
            float* y, const char* caller) {
  mlq_weight w;
  checkMlq(mlq_weight_layout(MLQ_F32, out_features, in_features, &w), "HIP matmul error in",
           caller);
  w.base = const_cast<void*>(w_device);
  checkMlq(mlq_linear(&w, x, y, rows, nullptr), "HIP matmul error in", caller);
}

// addBiasInPlace (src/cuda_matmul.cc:140-150).
void addBiasInPlace(Tensor& y, const Tensor& bias, int rows, int cols) {
  if (bias.numDims() != 1 || bias.shape[0] != cols)
    throw std::runtime_error("hipLinear: expected bias shape [out_features]");
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) y.data[(size_t)r * cols + c] += bias.data[c];
}

}  // namespace

bool hipMatmulBuilt() { return true; }

Tensor hipMatmul(const Tensor& a, const Tensor& b, int device_id) {
  // validateMatmulShapes (src/cuda_matmul.cc:93-103)
  if (a.numDims() != 2 || b.numDims() != 2)
    throw std::runtime_error("hipMatmul: expected a and b to be 2D tensors");
  if (a.shape[1] != b.shape[0])
    throw std::runtime_error("hipMatmul: dimension mismatch " + a.shapeString() + " vs " +
                             b.shapeString());
  const int m = a.shape[0], k = a.shape[1], n = b.shape[1];
  if (m <= 0 || k <= 0 || n <= 0)
    throw std::runtime_error("hipMatmul: empty tensors are not supported");
  // a @ b = a @ (b^T)^T: b^T [n, k] is the Linear weight
  std::vector<float> bt((size_t)n * k);
  for (int i = 0; i < k; ++i)
    for (int j = 0; j < n; ++j) bt[(size_t)j * k + i] = b.data[(size_t)i * n + j];
  hipSetDeviceId(device_id);
  HipDeviceBuffer a_dev(a.size() * sizeof(float), device_id);
  HipDeviceBuffer b_dev(bt.size() * sizeof(float), device_id);
  HipDeviceBuffer c_dev((size_t)m * n * sizeof(float), device_id);
  a_dev.upload(a.data.data(), a.size() * sizeof(float));
  b_dev.upload(bt.data(), bt.size() * sizeof(float));
  runF32(static_cast<const float*>(a_dev.data()), b_dev.data(), m, n, k,
         static_cast<float*>(c_dev.data()), "hipMatmul");
  Tensor c({m, n}, 0.0f);
  c_dev.download(c.data.data(), c.size() * sizeof(float));
  return c;
}

Tensor hipLinearDeviceWeight(const Tensor& x, const void* w_device,
                             const std::vector<int>& w_shape, const Tensor* bias,
                             int device_id) {
  if (w_device == nullptr) throw std::runtime_error("hipLinear: device weight pointer is null");
  validateLinearShape(x.shape, x.shapeString(), w_shape, "hipLinear");
  const int rows = x.numDims() == 1 ? 1 : x.shape[0];
  const int in_features = x.shape.back(), out_features = w_shape[0];
  hipSetDeviceId(device_id);
  Tensor y(outputShape(x.shape, out_features), 0.0f);
  HipDeviceBuffer x_dev(x.size() * sizeof(float), device_id);
  HipDeviceBuffer y_dev(y.size() * sizeof(float), device_id);
  x_dev.upload(x.data.data(), x.size() * sizeof(float));
  runF32(static_cast<const float*>(x_dev.data()), w_device, rows, out_features, in_features,
         static_cast<float*>(y_dev.data()), "hipLinear");
  y_dev.download(y.data.data(), y.size() * sizeof(float));
  if (bias != nullptr) addBiasInPlace(y, *bias, rows, out_features);
  return y;
}

Tensor hipLinear(const Tensor& x, const Tensor& weight, const Tensor* bias, int device_id) {
  if (weight.numDims() != 2)
    throw std::runtime_error("hipLinear: expected weight shape [out_features, in_features]");
  validateLinearShape(x.shape, x.shapeString(), weight.shape, "hipLinear");
  hipSetDeviceId(device_id);
  HipDeviceBuffer w_dev(weight.size() * sizeof(float), device_id);
  w_dev.upload(weight.data.data(), weight.size() * sizeof(float));
  return hipLinearDeviceWeight(x, w_dev.data(), weight.shape, bias, device_id);
}

HipTensor hipLinearDeviceInput(const HipTensor& x, const void* w_device,
                               const std::vector<int>& w_shape, int device_id) {
  if (w_device == nullptr)
    throw std::runtime_error("hipLinearDeviceInput: device weight pointer is null");
  if (x.deviceId() != device_id)
    throw std::runtime_error("hipLinearDeviceInput: input tensor is on a different HIP device");
  validateLinearShape(x.shape(), x.shapeString(), w_shape, "hipLinearDeviceInput");
  const int rows = x.numDims() == 1 ? 1 : x.shape()[0];
  const int in_features = x.shape().back(), out_features = w_shape[0];
  hipSetDeviceId(device_id);
  HipTensor y(outputShape(x.shape(), out_features), device_id);
  runF32(static_cast<const float*>(x.data()), w_device, rows, out_features, in_features,
         static_cast<float*>(y.data()), "hipLinearDeviceInput");
  return y;
}

}  // namespace mini_llama
