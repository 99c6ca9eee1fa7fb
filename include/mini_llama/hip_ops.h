// Decode-step operators of the HIP backend: the interface of
// include/mini_llama/cuda_ops.h:14-85 with hip names, over the operator
// entry points of libmlq (mlq_rmsnorm, mlq_silu, mlq_mul, mlq_add,
// mlq_softmax, mlq_embedding, mlq_rope). Validation and messages follow
// src/cuda_ops.cu. Host-interface calls upload, run and download; device
// interfaces return HipTensor results on the null stream.
#ifndef MINI_LLAMA_HIP_OPS_H_
#define MINI_LLAMA_HIP_OPS_H_

#include <vector>

#include "mini_llama/hip_tensor.h"
#include "mini_llama/model_config.h"
#include "mini_llama/tensor.h"

namespace mini_llama {

bool hipOpsBuilt();

// ---- host interface (cuda_ops.h:22-34) ----
Tensor hipRmsNorm(const Tensor& x, const Tensor& weight, float eps, int device_id = 0);
Tensor hipSilu(const Tensor& x, int device_id = 0);
Tensor hipElementwiseMul(const Tensor& a, const Tensor& b, int device_id = 0);
Tensor hipElementwiseAdd(const Tensor& a, const Tensor& b, int device_id = 0);

// ---- device interface (cuda_ops.h:40-81) ----
HipTensor hipRmsNormDeviceWeight(const HipTensor& x, const void* weight_data,
                                 const std::vector<int>& weight_shape, float eps,
                                 int device_id = 0);
HipTensor hipRmsNormDeviceInput(const HipTensor& x, const Tensor& weight, float eps,
                                int device_id = 0);
HipTensor hipSiluDeviceInput(const HipTensor& x, int device_id = 0);
HipTensor hipElementwiseMulDeviceInput(const HipTensor& a, const HipTensor& b,
                                       int device_id = 0);
HipTensor hipElementwiseAddDeviceInput(const HipTensor& a, const HipTensor& b,
                                       int device_id = 0);
HipTensor hipElementwiseAddDeviceWeight(const HipTensor& a, const void* b_data,
                                        const std::vector<int>& b_shape, int device_id = 0);
Tensor hipSoftmax(const Tensor& x, int device_id = 0);
HipTensor hipEmbeddingLookupDeviceWeight(const void* embedding_data,
                                         const std::vector<int>& embedding_shape, int token_id,
                                         int device_id = 0);
// q [n_heads, head_dim], k [n_kv_heads, head_dim], rotated in place.
void hipRope(Tensor& q, Tensor& k, int pos, float theta, RopeType rope_type = RopeType::kNormal,
             int device_id = 0);
void hipRopeDeviceInput(HipTensor& q, HipTensor& k, int n_heads, int n_kv_heads, int head_dim,
                        int pos, float theta, RopeType rope_type = RopeType::kNormal,
                        int device_id = 0);

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_OPS_H_
