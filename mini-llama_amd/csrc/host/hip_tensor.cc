// Device-resident F32 tensor (mirrors src/cuda_tensor.cc:51-107).
#include "mini_llama/hip_tensor.h"

#include <stdexcept>

namespace mini_llama {
namespace {

size_t numelChecked(const std::vector<int>& shape, const char* caller) {
  size_t n = 1;
  for (int d : shape) {
    if (d <= 0)
      throw std::runtime_error(std::string(caller) +
                               ": dimensions must be positive, got " +
                               shapeToString(shape));
    n *= static_cast<size_t>(d);
  }
  return n;
}

}  // namespace

HipTensor::HipTensor(const std::vector<int>& shape, int device_id) {
  reset(shape, device_id);
}

void HipTensor::reset() {
  buffer_.reset();
  shape_.clear();
  numel_ = 0;
}

void HipTensor::reset(const std::vector<int>& shape, int device_id) {
  const size_t n = numelChecked(shape, "HipTensor");
  buffer_.reset(n * sizeof(float), device_id);
  shape_ = shape;
  numel_ = n;
  device_id_ = device_id;
}

void HipTensor::uploadFrom(const Tensor& src) {
  if (src.shape != shape_)
    throw std::runtime_error("HipTensor::uploadFrom: shape mismatch " +
                             src.shapeString() + " vs " + shapeString());
  buffer_.upload(src.data.data(), src.size() * sizeof(float));
}

Tensor HipTensor::download() const {
  if (shape_.empty()) return Tensor();
  Tensor out(shape_, 0.0f);
  downloadTo(out);
  return out;
}

// A host tensor of another shape is an error, as CudaTensor::downloadTo
// (src/cuda_tensor.cc:88-95): nothing is reallocated behind the caller.
void HipTensor::downloadTo(Tensor& dst) const {
  if (dst.shape != shape_)
    throw std::runtime_error("HipTensor::downloadTo shape mismatch: device=" + shapeString() +
                             " host=" + dst.shapeString());
  buffer_.download(dst.data.data(), numel_ * sizeof(float));
}

void* HipTensor::data() { return buffer_.data(); }
const void* HipTensor::data() const { return buffer_.data(); }

std::string HipTensor::shapeString() const { return shapeToString(shape_); }

HipTensor hipTensorFromHost(const Tensor& src, int device_id) {
  HipTensor t(src.shape, device_id);
  t.uploadFrom(src);
  return t;
}

}  // namespace mini_llama
