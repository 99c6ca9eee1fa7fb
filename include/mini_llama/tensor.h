// Minimal dense F32 tensor for the HIP backend's host interface.
// Same data model and accessor names as the reference Tensor
// (include/mini_llama/tensor.h:15-60): row-major std::vector<float> data plus
// an int shape. Invalid dimensions throw std::runtime_error here (the
// reference only logs them).
#ifndef MINI_LLAMA_HIP_TENSOR_BASE_H_
#define MINI_LLAMA_HIP_TENSOR_BASE_H_

#include <cstddef>
#include <string>
#include <vector>

namespace mini_llama {

struct Tensor {
  std::vector<float> data;
  std::vector<int> shape;

  Tensor() = default;
  explicit Tensor(const std::vector<int>& input_shape, float fill = 0.0f);

  size_t size() const { return data.size(); }
  size_t numElements() const { return data.size(); }
  int numDims() const { return static_cast<int>(shape.size()); }
  bool empty() const { return size() == 0; }

  float& at2(int i, int j);
  float at2(int i, int j) const;

  float& operator[](size_t i) { return data[i]; }
  float operator[](size_t i) const { return data[i]; }

  std::string shapeString() const;
};

std::string shapeToString(const std::vector<int>& shape);

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_TENSOR_BASE_H_
