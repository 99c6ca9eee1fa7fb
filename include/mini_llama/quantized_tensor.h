// Block-quantized weight types: byte-identical to the reference's GGUF
// compatible structs (include/mini_llama/quantized_tensor.h:23-133) so that
// blocks produced by the reference loader/quantizer can be handed over as-is.
#ifndef MINI_LLAMA_HIP_QUANTIZED_TENSOR_H_
#define MINI_LLAMA_HIP_QUANTIZED_TENSOR_H_

#include <cstdint>
#include <vector>

#include "mini_llama/tensor.h"

namespace mini_llama {

// Enumerator order matches the reference (and enum mlq_type in mlq.h).
enum class QuantType {
  kF32,
  kQ80,
  kQ40,
  kQ41,
};

constexpr int kQ80BlockSize = 32;
constexpr int kQ40BlockSize = 32;
constexpr int kQ41BlockSize = 32;

struct BlockQ80 {
  uint16_t d;     // fp16 scale
  int8_t qs[32];  // value = d * qs[i]
};
static_assert(sizeof(BlockQ80) == 34, "wrong Q8_0 block size");

struct BlockQ40 {
  uint16_t d;      // fp16 scale
  uint8_t qs[16];  // element i<16: low nibble of qs[i]; i>=16: high of qs[i-16]
};
static_assert(sizeof(BlockQ40) == 18, "wrong Q4_0 block size");

struct BlockQ41 {
  uint16_t d;      // fp16 scale
  uint16_t m;      // fp16 min: value = d * nibble + m
  uint8_t qs[16];
};
static_assert(sizeof(BlockQ41) == 20, "wrong Q4_1 block size");

struct QuantizedTensor {
  QuantType type = QuantType::kF32;
  std::vector<int> shape;
  std::vector<float> f32_data;
  std::vector<BlockQ80> q8_0_data;
  std::vector<BlockQ40> q4_0_data;
  std::vector<BlockQ41> q4_1_data;

  size_t num_elements() const {
    size_t n = 1;
    for (int d : shape) n *= static_cast<size_t>(d);
    return n;
  }
  int num_dims() const { return static_cast<int>(shape.size()); }
  std::string shapeString() const { return shapeToString(shape); }
};

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_QUANTIZED_TENSOR_H_
