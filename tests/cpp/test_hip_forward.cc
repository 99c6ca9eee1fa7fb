// The reference's device forward pass (forwardToken's CUDA branch,
// src/forward.cc:607-640, 736-784) written against the HIP backend's C++
// interfaces only: hipEmbeddingLookupDeviceWeight, hipRmsNormDeviceWeight,
// hipLinearUploaded (F32 and quantized projections, as forwardLinearDevice
// dispatches them), hipRopeDeviceInput, HipKvCache::writeDevice,
// hipAttentionDecodeDeviceInput, hipSiluDeviceInput,
// hipElementwiseMulDeviceInput / AddDeviceInput / AddDeviceWeight (biases).
// This is the caller side a `--backend hip` build runs; the checker is the
// Python test that launches this program (tests/test_gpu_cpp_forward.py)
// and compares what it writes with the CPU oracle.
//
// Usage: test_hip_forward <model.json> <model.bin> <f32|q8_0|q4_0> <out> <token>...
// Loads a model in the reference's manifest format (model.json + raw fp32
// model.bin, as loadModel reads it, src/loader.cc:805-1000), quantizes the
// Linear weights with the oracle quantizer when asked (quantizeModelToQ80's
// role), runs every token at positions 0, 1, ... and writes to <out>, as
// raw fp32: the logits of every step ([tokens][vocab]), then the K and V
// cache rows of every layer and position ([layers][tokens][n_kv][hd] keys,
// then values). Exit status 0 on success, 2 when no HIP device is visible.
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "mini_llama/hip_attention.h"
#include "mini_llama/hip_kv_cache.h"
#include "mini_llama/hip_matmul.h"
#include "mini_llama/hip_ops.h"
#include "mini_llama/hip_quant.h"
#include "mini_llama/hip_runtime.h"
#include "mini_llama/hip_tensor.h"
#include "mini_llama/hip_model_upload.h"
#include "mini_llama/hip_weight_upload.h"
#include "mini_llama/model_config.h"
#include "quant_ref.h"

using namespace mini_llama;

namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ----
struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  double number = 0.0;
  bool boolean = false;
  std::string text;
  std::vector<Json> items;
  std::map<std::string, Json> fields;
  const Json& at(const std::string& key) const {
    auto it = fields.find(key);
    if (kind != kObject || it == fields.end()) throw std::runtime_error("json: missing " + key);
    return it->second;
  }
  bool has(const std::string& key) const { return kind == kObject && fields.count(key) > 0; }
};

class JsonReader {
 public:
  explicit JsonReader(const std::string& s) : s_(s) {}
  Json parse() {
    Json v = value();
    space();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* what) {
    throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(i_));
  }
  void space() {
    while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
  }
  bool take(char c) {
    space();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  std::string str() {
    if (!take('"')) fail("expected string");
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      if (s_[i_] == '\\') {
        if (++i_ >= s_.size()) fail("bad escape");
        const char e = s_[i_];
        out += e == 'n' ? '\n' : e == 't' ? '\t' : e;  // (\u escapes do not occur)
      } else {
        out += s_[i_];
      }
      ++i_;
    }
    if (i_ >= s_.size()) fail("unterminated string");
    ++i_;
    return out;
  }
  Json value() {
    space();
    if (i_ >= s_.size()) fail("unexpected end");
    Json v;
    const char c = s_[i_];
    if (c == '{') {
      ++i_;
      v.kind = Json::kObject;
      if (take('}')) return v;
      do {
        const std::string key = str();
        if (!take(':')) fail("expected ':'");
        v.fields[key] = value();
      } while (take(','));
      if (!take('}')) fail("expected '}'");
    } else if (c == '[') {
      ++i_;
      v.kind = Json::kArray;
      if (take(']')) return v;
      do v.items.push_back(value());
      while (take(','));
      if (!take(']')) fail("expected ']'");
    } else if (c == '"') {
      v.kind = Json::kString;
      v.text = str();
    } else if (s_.compare(i_, 4, "true") == 0 || s_.compare(i_, 5, "false") == 0) {
      v.kind = Json::kBool;
      v.boolean = s_[i_] == 't';
      i_ += v.boolean ? 4 : 5;
    } else if (s_.compare(i_, 4, "null") == 0) {
      i_ += 4;
    } else {
      size_t used = 0;
      v.kind = Json::kNumber;
      v.number = std::stod(s_.substr(i_, 64), &used);
      if (used == 0) fail("bad number");
      i_ += used;
    }
    return v;
  }
  const std::string& s_;
  size_t i_ = 0;
};

std::string readFile(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot open " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

// ---- the model --------------------------------------------------------------
struct Layer {
  Tensor bq, bk, bv;  // optional biases (empty when absent)
};

struct Model {
  ModelConfig c;
  std::map<std::string, Tensor> tensors;
  std::vector<Layer> layers;
};

Model loadManifest(const std::string& json_path, const std::string& bin_path) {
  const Json m = JsonReader(readFile(json_path)).parse();
  const std::string bin = readFile(bin_path);
  Model model;
  const Json& cfg = m.at("config");
  model.c.vocab_size = (int)cfg.at("vocab_size").number;
  model.c.dim = (int)cfg.at("dim").number;
  model.c.hidden_dim = (int)cfg.at("hidden_dim").number;
  model.c.n_layers = (int)cfg.at("n_layers").number;
  model.c.n_heads = (int)cfg.at("n_heads").number;
  model.c.n_kv_heads = (int)cfg.at("n_kv_heads").number;
  model.c.max_seq_len = (int)cfg.at("max_seq_len").number;
  model.c.rope_theta = (float)cfg.at("rope_theta").number;
  model.c.rms_norm_eps = (float)cfg.at("rms_norm_eps").number;
  model.c.head_dim = model.c.dim / model.c.n_heads;  // parseConfig's rule
  for (const Json& t : m.at("tensors").items) {
    std::vector<int> shape;
    size_t n = 1;
    for (const Json& d : t.at("shape").items) {
      shape.push_back((int)d.number);
      n *= (size_t)d.number;
    }
    const size_t off = (size_t)t.at("offset").number, bytes = (size_t)t.at("byte_size").number;
    if (bytes != 4 * n || off + bytes > bin.size())
      throw std::runtime_error("bad tensor extent: " + t.at("name").text);
    Tensor x(shape, 0.0f);
    std::memcpy(x.data.data(), bin.data() + off, bytes);
    model.tensors[t.at("name").text] = std::move(x);
  }
  model.layers.resize(model.c.n_layers);
  for (int i = 0; i < model.c.n_layers; ++i) {
    const std::string p = "layers." + std::to_string(i) + ".";
    for (auto [name, dst] : {std::pair<const char*, Tensor*>{"bq", &model.layers[i].bq},
                             {"bk", &model.layers[i].bk},
                             {"bv", &model.layers[i].bv}})
      if (model.tensors.count(p + name)) *dst = model.tensors[p + name];
  }
  return model;
}

QuantizedTensor linearWeight(const Tensor& w, const std::string& quant) {
  QuantizedTensor q;
  q.shape = w.shape;
  const int rows = w.shape[0], k = w.shape[1];
  const size_t nb = (size_t)rows * ((k + 31) / 32);
  if (quant == "f32") {
    q.type = QuantType::kF32;
    q.f32_data = w.data;
  } else if (quant == "q8_0") {
    q.type = QuantType::kQ80;
    q.q8_0_data.resize(nb);
    ref_quantize_q8_0(w.data.data(), rows, k, reinterpret_cast<ref_block_q8_0*>(q.q8_0_data.data()));
  } else if (quant == "q4_0") {
    q.type = QuantType::kQ40;
    q.q4_0_data.resize(nb);
    ref_quantize_q4_0(w.data.data(), rows, k, reinterpret_cast<ref_block_q4_0*>(q.q4_0_data.data()));
  } else {
    throw std::runtime_error("unknown quant " + quant);
  }
  return q;
}

// The reference's MiniLlamaModel weight fields (include/mini_llama/model.h:
// 37-61), with the hip_weights member a --backend hip build adds: what
// uploadModelWeightsToHip takes.
struct HostLayerWeights {
  Tensor attention_norm;
  QuantizedTensor wq, wk, wv;
  Tensor bq, bk, bv;
  QuantizedTensor wo;
  Tensor ffn_norm;
  QuantizedTensor w_gate, w_up, w_down;
};

struct HostModel {
  bool loaded = false;
  Tensor token_embedding;
  std::vector<HostLayerWeights> layers;
  Tensor final_norm;
  QuantizedTensor lm_head;
  std::shared_ptr<HipModelWeights> hip_weights;
};

// The manifest model with its Linear weights quantized as asked
// (quantizeModelToQ80 / Q40's role, src/model.cc:107-148).
HostModel hostModel(const Model& m, const std::string& quant) {
  HostModel h;
  auto get = [&](const std::string& name) {
    const auto it = m.tensors.find(name);
    return it == m.tensors.end() ? Tensor() : it->second;
  };
  h.token_embedding = get("token_embedding");
  h.final_norm = get("final_norm");
  h.lm_head = linearWeight(get("lm_head"), quant);
  for (int i = 0; i < m.c.n_layers; ++i) {
    const std::string p = "layers." + std::to_string(i) + ".";
    HostLayerWeights lw;
    lw.attention_norm = get(p + "attention_norm");
    lw.wq = linearWeight(get(p + "wq"), quant);
    lw.wk = linearWeight(get(p + "wk"), quant);
    lw.wv = linearWeight(get(p + "wv"), quant);
    lw.bq = get(p + "bq");
    lw.bk = get(p + "bk");
    lw.bv = get(p + "bv");
    lw.wo = linearWeight(get(p + "wo"), quant);
    lw.ffn_norm = get(p + "ffn_norm");
    lw.w_gate = linearWeight(get(p + "w_gate"), quant);
    lw.w_up = linearWeight(get(p + "w_up"), quant);
    lw.w_down = linearWeight(get(p + "w_down"), quant);
    h.layers.push_back(std::move(lw));
  }
  h.loaded = true;
  return h;
}

// ---- forwardToken's device branch ---------------------------------------------
struct Engine {
  Engine(const Model& m, const HipModelWeights& uploaded) : model(m), weights(uploaded) {}
  const Model& model;
  const HipModelWeights& weights;
  HipKvCache cache;
  int dev = 0;

  const HipUploadedWeight& w(const std::string& name, QuantType type) const {
    const HipUploadedWeight* cw = findHipWeight(weights, name, type);
    if (cw == nullptr) throw std::runtime_error("missing uploaded weight: " + name);
    return *cw;
  }
  QuantType linearType = QuantType::kF32;

  HipTensor rmsNorm(const std::string& name, const HipTensor& x) const {
    const HipUploadedWeight& n = w(name, QuantType::kF32);
    return hipRmsNormDeviceWeight(x, n.buffer.data(), n.shape, model.c.rms_norm_eps, dev);
  }
  // forwardLinearDevice (src/forward.cc:190-225): F32 or quantized
  HipTensor linear(const std::string& name, const HipTensor& x) const {
    return hipLinearUploaded(x, w(name, linearType), dev);
  }
  HipTensor bias(const std::string& name, HipTensor x, const Tensor& b) const {
    if (b.data.empty()) return x;
    const HipUploadedWeight& bw = w(name, QuantType::kF32);
    return hipElementwiseAddDeviceWeight(x, bw.buffer.data(), bw.shape, dev);
  }

  HipTensor layer(const HipTensor& x, int li, int pos) {
    const ModelConfig& c = model.c;
    const std::string p = "layers." + std::to_string(li) + ".";
    const HipTensor h = rmsNorm(p + "attention_norm", x);
    HipTensor q = bias(p + "bq", linear(p + "wq", h), model.layers[li].bq);
    HipTensor k = bias(p + "bk", linear(p + "wk", h), model.layers[li].bk);
    HipTensor v = bias(p + "bv", linear(p + "wv", h), model.layers[li].bv);
    hipRopeDeviceInput(q, k, c.n_heads, c.n_kv_heads, c.head_dim, pos, c.rope_theta, c.rope_type,
                       dev);
    cache.writeDevice(li, pos, k, v);
    const HipTensor attn = hipAttentionDecodeDeviceInput(q, cache, li, pos, c.n_heads,
                                                         c.n_kv_heads, c.head_dim, dev);
    const HipTensor x_attn = hipElementwiseAddDeviceInput(x, linear(p + "wo", attn), dev);
    const HipTensor h2 = rmsNorm(p + "ffn_norm", x_attn);
    const HipTensor gate = linear(p + "w_gate", h2);
    const HipTensor up = linear(p + "w_up", h2);
    const HipTensor act = hipElementwiseMulDeviceInput(hipSiluDeviceInput(gate, dev), up, dev);
    return hipElementwiseAddDeviceInput(x_attn, linear(p + "w_down", act), dev);
  }

  Tensor forwardToken(int token, int pos) {
    const HipUploadedWeight& e = w("token_embedding", QuantType::kF32);
    HipTensor x = hipEmbeddingLookupDeviceWeight(e.buffer.data(), e.shape, token, dev);
    for (int li = 0; li < model.c.n_layers; ++li) x = layer(x, li, pos);
    return linear("lm_head", rmsNorm("final_norm", x)).download();
  }
};

}  // namespace

int main(int argc, char** argv) {
  if (argc < 6) {
    std::cerr << "usage: test_hip_forward <model.json> <model.bin> <f32|q8_0|q4_0> <out> <token>...\n";
    return 1;
  }
  if (hipDeviceCount() == 0) {
    std::cerr << "no HIP device\n";
    return 2;
  }
  try {
    const Model model = loadManifest(argv[1], argv[2]);
    const std::string quant = argv[3];
    std::vector<int> tokens;
    for (int i = 5; i < argc; ++i) tokens.push_back(std::atoi(argv[i]));
    const ModelConfig& c = model.c;
    // uploadModelWeightsToCuda's twin (src/model.cc:151-199): every Linear,
    // plus the embedding, norms and biases as plain F32 tensors
    HostModel host = hostModel(model, quant);
    HostModel unloaded;
    bool threw = false;
    try {
      uploadModelWeightsToHip(unloaded, 0);
    } catch (const std::runtime_error&) {
      threw = true;
    }
    if (!threw || modelHasHipWeights(unloaded))
      throw std::runtime_error("upload of an unloaded model did not throw");
    uploadModelWeightsToHip(host, 0);
    // 3 global weights + per layer 2 norms, 7 Linear weights and the biases
    // the manifest holds
    size_t expected = 3;
    for (const HostLayerWeights& lw : host.layers)
      expected += 9 + !lw.bq.data.empty() + !lw.bk.data.empty() + !lw.bv.data.empty();
    if (!modelHasHipWeights(host) || modelHipUploadedWeightCount(host) != expected ||
        modelHipMemoryBytes(host) == 0)
      throw std::runtime_error("uploadModelWeightsToHip: " +
                               std::to_string(modelHipUploadedWeightCount(host)) +
                               " weights uploaded, expected " + std::to_string(expected));
    Engine eng(model, *host.hip_weights);
    eng.linearType = host.lm_head.type;
    eng.cache.reset(c.n_layers, c.max_seq_len, c.n_kv_heads, c.head_dim, 0);
    std::ofstream out(argv[4], std::ios::binary);
    for (size_t i = 0; i < tokens.size(); ++i) {
      const Tensor logits = eng.forwardToken(tokens[i], (int)i);
      if ((int)logits.size() != c.vocab_size) throw std::runtime_error("logits size");
      out.write(reinterpret_cast<const char*>(logits.data.data()), logits.size() * 4);
    }
    for (int kind = 0; kind < 2; ++kind)
      for (int li = 0; li < c.n_layers; ++li)
        for (int p = 0; p < (int)tokens.size(); ++p) {
          const Tensor row = kind == 0 ? eng.cache.readKey(li, p) : eng.cache.readValue(li, p);
          out.write(reinterpret_cast<const char*>(row.data.data()), row.size() * 4);
        }
    std::cout << "test_hip_forward: " << tokens.size() << " tokens, " << quant << ", "
              << eng.weights.uploaded_weight_count << " weights uploaded\n";
  } catch (const std::exception& e) {
    std::cerr << "test_hip_forward: " << e.what() << "\n";
    return 1;
  }
  return 0;
}
