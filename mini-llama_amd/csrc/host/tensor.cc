// Minimal F32 Tensor of the HIP backend's host interface.
#include "mini_llama/tensor.h"

#include <stdexcept>

namespace mini_llama {

std::string shapeToString(const std::vector<int>& shape) {
  std::string s = "[";
  for (size_t i = 0; i < shape.size(); ++i) {
    s += std::to_string(shape[i]);
    if (i + 1 < shape.size()) s += ", ";
  }
  return s + "]";
}

Tensor::Tensor(const std::vector<int>& input_shape, float fill)
    : shape(input_shape) {
  size_t total = 1;
  for (int d : input_shape) {
    if (d <= 0)
      throw std::runtime_error("Tensor: dimensions must be positive, got " +
                               shapeToString(input_shape));
    total *= static_cast<size_t>(d);
  }
  data.assign(total, fill);
}

float& Tensor::at2(int i, int j) {
  return data[static_cast<size_t>(i) * shape[1] + j];
}

float Tensor::at2(int i, int j) const {
  return data[static_cast<size_t>(i) * shape[1] + j];
}

std::string Tensor::shapeString() const { return shapeToString(shape); }

}  // namespace mini_llama
