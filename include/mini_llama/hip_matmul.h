// F32 Linear / matmul of the HIP backend: the interface of
// include/mini_llama/cuda_matmul.h:14-38 with hip names. The reference runs
// cuBLAS Sgemm (src/cuda_matmul.cc:150-241); here every call is the fp32
// HBM-streaming GEMV of libmlq (mlq_linear on an MLQ_F32 weight, y = x W^T
// with W [out_features, in_features] fp32 row-major), with the reference's
// validation and messages.
#ifndef MINI_LLAMA_HIP_MATMUL_H_
#define MINI_LLAMA_HIP_MATMUL_H_

#include <vector>

#include "mini_llama/hip_tensor.h"
#include "mini_llama/tensor.h"

namespace mini_llama {

bool hipMatmulBuilt();

// c = a @ b, a [m, k], b [k, n] -> [m, n] (cudaMatmul, cuda_matmul.h:18).
Tensor hipMatmul(const Tensor& a, const Tensor& b, int device_id = 0);

// y = x @ weight^T + bias; x [in] or [batch, in], weight [out, in]
// (cudaLinear, cuda_matmul.h:25).
Tensor hipLinear(const Tensor& x, const Tensor& weight, const Tensor* bias = nullptr,
                 int device_id = 0);

// weight already on the device (cudaLinearDeviceWeight, cuda_matmul.h:29).
Tensor hipLinearDeviceWeight(const Tensor& x, const void* w_device,
                             const std::vector<int>& w_shape, const Tensor* bias = nullptr,
                             int device_id = 0);

// input and output on the device (cudaLinearDeviceInput, cuda_matmul.h:36).
HipTensor hipLinearDeviceInput(const HipTensor& x, const void* w_device,
                               const std::vector<int>& w_shape, int device_id = 0);

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_MATMUL_H_
