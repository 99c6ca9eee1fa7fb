// Decode attention of the HIP backend: the interface of
// include/mini_llama/cuda_attention.h:11-26 with hip names, over
// mlq_attention_decode (GQA: query head h reads kv head h / (n_heads /
// n_kv_heads), softmax(q.K^T / sqrt(head_dim)).V over positions 0..pos).
#ifndef MINI_LLAMA_HIP_ATTENTION_H_
#define MINI_LLAMA_HIP_ATTENTION_H_

#include "mini_llama/hip_kv_cache.h"
#include "mini_llama/hip_tensor.h"
#include "mini_llama/tensor.h"

namespace mini_llama {

bool hipAttentionBuilt();

// q [n_heads, head_dim] on the host -> [n_heads, head_dim] on the host.
Tensor hipAttentionDecode(const Tensor& q, const HipKvCache& kv_cache, int layer, int pos,
                          int n_heads, int n_kv_heads, int head_dim, int device_id = 0);

// q: n_heads * head_dim floats on the device -> [n_heads * head_dim].
HipTensor hipAttentionDecodeDeviceInput(const HipTensor& q, const HipKvCache& kv_cache,
                                        int layer, int pos, int n_heads, int n_kv_heads,
                                        int head_dim, int device_id = 0);

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_ATTENTION_H_
