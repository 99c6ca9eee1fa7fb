// Model hyper-parameters shared by the HIP backend's host interfaces: the
// RopeType and ModelConfig of include/mini_llama/model.h:17-34 (same
// enumerators, fields and defaults, so a reference ModelConfig maps over
// field by field). The reference's MiniLlamaModel, loader and CPU forward
// pass are not part of this backend.
#ifndef MINI_LLAMA_HIP_MODEL_CONFIG_H_
#define MINI_LLAMA_HIP_MODEL_CONFIG_H_

namespace mini_llama {

enum class RopeType {
  kNormal,
  kNeoX,
};

struct ModelConfig {
  int vocab_size = 128;
  int dim = 32;
  int hidden_dim = 86;
  int n_layers = 2;
  int n_heads = 4;
  int n_kv_heads = 4;
  int head_dim = 8;
  int max_seq_len = 128;
  float rope_theta = 10000.0f;
  float rms_norm_eps = 1e-5f;
  RopeType rope_type = RopeType::kNormal;
};

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_MODEL_CONFIG_H_
