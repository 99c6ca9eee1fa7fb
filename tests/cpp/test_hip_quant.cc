// GPU tests of the HIP backend's quantized Linear host interface, written
// like the reference's CUDA tests (tests/test_cuda.cc:679-808: same inputs,
// same 1e-4 / 1e-5 tolerances, same validation cases) with cuda* -> hip*.
// The CPU side is the oracle restatement of linearQ80/Q40/Q41
// (oracle/quant_ref.c), linked here as the checker only.
//
// Usage: test_hip_quant [filter]   (exit 0 = all passed; prints one line per
// test). Every test returns early with "skip" when no HIP device is visible.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <iostream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "mini_llama/backend.h"
#include "mini_llama/hip_attention.h"
#include "mini_llama/hip_kv_cache.h"
#include "mini_llama/hip_matmul.h"
#include "mini_llama/hip_ops.h"
#include "mini_llama/hip_quant.h"
#include "mini_llama/hip_runtime.h"
#include "mini_llama/hip_tensor.h"
#include "mini_llama/hip_weight_upload.h"
#include "forward_ref.h"
#include "quant_ref.h"

using namespace mini_llama;

namespace {

struct TestCase {
  const char* name;
  std::function<bool()> fn;
};

std::vector<TestCase>& registry() {
  static std::vector<TestCase> r;
  return r;
}

struct Registrar {
  Registrar(const char* name, std::function<bool()> fn) {
    registry().push_back({name, std::move(fn)});
  }
};

#define TEST(name)                                   \
  static bool name();                                \
  static Registrar name##_registrar(#name, name);    \
  static bool name()

#define CHECK(cond)                                                        \
  do {                                                                     \
    if (!(cond)) {                                                         \
      std::cerr << "  check failed: " #cond " (" << __FILE__ << ":"        \
                << __LINE__ << ")\n";                                      \
      return false;                                                        \
    }                                                                      \
  } while (0)

bool hipAvailable() { return hipDeviceCount() > 0; }

template <typename Ex>
bool throwsAs(const std::function<void()>& fn) {
  try {
    fn();
  } catch (const Ex&) {
    return true;
  } catch (...) {
    return false;
  }
  return false;
}

void fillLinear(Tensor& t, float scale, float offset) {
  for (size_t i = 0; i < t.size(); ++i)
    t.data[i] = offset + scale * static_cast<float>(i);
}

bool expectNear(const Tensor& actual, const Tensor& expected, float tol,
                const char* what) {
  if (actual.shape != expected.shape) {
    std::cerr << "  shape mismatch for " << what << ": " << actual.shapeString()
              << " vs " << expected.shapeString() << "\n";
    return false;
  }
  float max_diff = 0.0f;
  size_t arg = 0;
  for (size_t i = 0; i < actual.size(); ++i) {
    const float diff = std::fabs(actual.data[i] - expected.data[i]);
    if (!(diff <= max_diff)) {
      max_diff = diff;
      arg = i;
    }
  }
  if (!(max_diff <= tol)) {
    std::cerr << "  " << what << ": max diff " << max_diff << " at " << arg
              << " (actual=" << actual.data[arg]
              << ", expected=" << expected.data[arg] << ", tol=" << tol << ")\n";
    return false;
  }
  return true;
}

// Oracle wrappers (CPU reference path: quantizeToQ80/Q40, linearQ80/Q40/Q41).
std::vector<BlockQ80> quantizeQ80(const Tensor& t) {
  const int row = t.numDims() >= 2 ? t.shape.back() : (int)t.size();
  const int rows = (int)t.size() / row;
  std::vector<BlockQ80> out((size_t)rows * ((row + 31) / 32));
  ref_quantize_q8_0(t.data.data(), rows, row, (ref_block_q8_0*)out.data());
  return out;
}

std::vector<BlockQ40> quantizeQ40(const Tensor& t) {
  const int row = t.numDims() >= 2 ? t.shape.back() : (int)t.size();
  const int rows = (int)t.size() / row;
  std::vector<BlockQ40> out((size_t)rows * ((row + 31) / 32));
  ref_quantize_q4_0(t.data.data(), rows, row, (ref_block_q4_0*)out.data());
  return out;
}

template <typename Block>
Tensor cpuLinear(const Tensor& x, const std::vector<Block>& w,
                 const std::vector<int>& shape) {
  const int rows = x.numDims() == 1 ? 1 : x.shape[0];
  const int k = x.numDims() == 1 ? x.shape[0] : x.shape[1];
  Tensor y(x.numDims() == 1 ? std::vector<int>{shape[0]}
                            : std::vector<int>{rows, shape[0]});
  int rc;
  if (sizeof(Block) == 34)
    rc = ref_linear_q8_0(x.data.data(), rows, k, (const ref_block_q8_0*)w.data(),
                         w.size(), shape[0], shape[1], y.data.data(), 1);
  else if (sizeof(Block) == 18)
    rc = ref_linear_q4_0(x.data.data(), rows, k, (const ref_block_q4_0*)w.data(),
                         w.size(), shape[0], shape[1], y.data.data(), 1);
  else
    rc = ref_linear_q4_1(x.data.data(), rows, k, (const ref_block_q4_1*)w.data(),
                         w.size(), shape[0], shape[1], y.data.data(), 1);
  if (rc != 0) throw std::runtime_error("oracle linear failed");
  return y;
}

// tests/test_cuda.cc:116-132: deterministic Q4_1 blocks (d=0.5, m=0).
std::vector<BlockQ41> makeQ41Blocks(int out_features, int in_features) {
  const int bpr = (in_features + 31) / 32;
  std::vector<BlockQ41> blocks((size_t)out_features * bpr);
  for (auto& b : blocks) {
    b.d = 0x3800;
    b.m = 0x0000;
    for (int i = 0; i < 16; ++i) {
      const int lo = (i * 3 + 1) & 0x0F;
      const int hi = (i * 5 + 2) & 0x0F;
      b.qs[i] = static_cast<uint8_t>(lo | (hi << 4));
    }
  }
  return blocks;
}

#define SKIP_WITHOUT_HIP()                               \
  do {                                                   \
    if (!hipAvailable()) {                               \
      std::cout << "  (skip: no HIP device)\n";          \
      return true;                                       \
    }                                                    \
  } while (0)

}  // namespace

// ---- mirrors tests/test_cuda.cc:679-710 ------------------------------------
TEST(hip_q80_linear_matches_cpu) {
  SKIP_WITHOUT_HIP();
  Tensor weight({4, 32});
  fillLinear(weight, 0.05f, -1.0f);
  Tensor x({32});
  fillLinear(x, 0.1f, -0.4f);
  auto blocks = quantizeQ80(weight);
  Tensor cpu = cpuLinear(x, blocks, weight.shape);
  Tensor gpu = hipQ80Linear(x, blocks, weight.shape);
  CHECK(expectNear(gpu, cpu, 1e-4f, "hipQ80Linear"));

  Tensor x2({2, 32});
  fillLinear(x2, 0.07f, -0.3f);
  Tensor bias({4});
  fillLinear(bias, 0.2f, -0.1f);
  Tensor cpu2 = cpuLinear(x2, blocks, weight.shape);
  for (int r = 0; r < 2; ++r)
    for (int c = 0; c < 4; ++c) cpu2.at2(r, c) += bias[c];
  CHECK(expectNear(hipQ80Linear(x2, blocks, weight.shape, &bias), cpu2, 1e-4f,
                   "hipQ80Linear 2D+bias"));
  return true;
}

// ---- mirrors tests/test_cuda.cc:712-727 ------------------------------------
TEST(hip_q40_linear_matches_cpu) {
  SKIP_WITHOUT_HIP();
  Tensor weight({4, 32});
  fillLinear(weight, 0.05f, -1.0f);
  Tensor x({32});
  fillLinear(x, 0.1f, -0.4f);
  auto blocks = quantizeQ40(weight);
  Tensor cpu = cpuLinear(x, blocks, weight.shape);
  Tensor gpu = hipQ40Linear(x, blocks, weight.shape);
  CHECK(expectNear(gpu, cpu, 1e-4f, "hipQ40Linear"));
  return true;
}

// ---- mirrors tests/test_cuda.cc:729-743 ------------------------------------
TEST(hip_q41_linear_matches_cpu) {
  SKIP_WITHOUT_HIP();
  Tensor x({32});
  fillLinear(x, 0.1f, -0.4f);
  auto blocks = makeQ41Blocks(4, 32);
  std::vector<int> shape = {4, 32};
  Tensor cpu = cpuLinear(x, blocks, shape);
  Tensor gpu = hipQ41Linear(x, blocks, shape);
  CHECK(expectNear(gpu, cpu, 1e-4f, "hipQ41Linear"));
  return true;
}

// ---- mirrors tests/test_cuda.cc:745-774 ------------------------------------
TEST(hip_quant_device_variants) {
  SKIP_WITHOUT_HIP();
  Tensor weight({4, 32});
  fillLinear(weight, 0.05f, -1.0f);
  Tensor x({32});
  fillLinear(x, 0.1f, -0.4f);
  auto blocks = quantizeQ80(weight);
  Tensor host = hipQ80Linear(x, blocks, weight.shape);

  HipDeviceBuffer w_dev(blocks.size() * sizeof(BlockQ80), 0);
  w_dev.upload(blocks.data(), blocks.size() * sizeof(BlockQ80));
  Tensor dev_weight = hipQ80LinearDeviceWeight(x, w_dev.data(), blocks.size(),
                                               weight.shape, nullptr);
  CHECK(expectNear(dev_weight, host, 1e-5f, "hipQ80LinearDeviceWeight"));

  HipTensor x_dev = hipTensorFromHost(x, 0);
  HipTensor dev_input = hipQ80LinearDeviceInput(x_dev, w_dev.data(),
                                                blocks.size(), weight.shape, 0);
  Tensor dev_input_host = dev_input.download();
  CHECK(dev_input_host.shape == std::vector<int>({4}));
  CHECK(expectNear(dev_input_host, host, 1e-5f, "hipQ80LinearDeviceInput"));
  return true;
}

// ---- mirrors tests/test_cuda.cc:776-808 ------------------------------------
TEST(hip_quant_validation) {
  SKIP_WITHOUT_HIP();
  Tensor weight({4, 32});
  fillLinear(weight, 0.05f, -1.0f);
  auto blocks = quantizeQ80(weight);

  Tensor x_bad({16});
  CHECK(throwsAs<std::runtime_error>(
      [&] { (void)hipQ80Linear(x_bad, blocks, weight.shape); }));

  auto short_blocks = blocks;
  short_blocks.pop_back();
  Tensor x({32});
  CHECK(throwsAs<std::runtime_error>(
      [&] { (void)hipQ80Linear(x, short_blocks, weight.shape); }));

  CHECK(throwsAs<std::runtime_error>([&] {
    (void)hipQ80LinearDeviceWeight(x, nullptr, blocks.size(), weight.shape,
                                   nullptr);
  }));

  Tensor x_3d({1, 1, 32});
  CHECK(throwsAs<std::runtime_error>(
      [&] { (void)hipQ80Linear(x_3d, blocks, weight.shape); }));

  // non-2D weight shape and a device id that does not exist
  CHECK(throwsAs<std::runtime_error>(
      [&] { (void)hipQ80Linear(x, blocks, std::vector<int>{128}); }));
  HipTensor xd = hipTensorFromHost(x, 0);
  CHECK(throwsAs<std::runtime_error>([&] {
    (void)hipQ80LinearDeviceInput(xd, blocks.data(), blocks.size(), weight.shape,
                                  hipDeviceCount());
  }));
  return true;
}

// ---- uploaded (tiled) weights take the same result as raw AoS pointers ----
TEST(hip_uploaded_weight_matches_aos_pointer) {
  SKIP_WITHOUT_HIP();
  std::mt19937 rng(1234);
  std::uniform_real_distribution<float> u(-1.0f, 1.0f);
  const int n = 40, k = 200;  // partial row tile and partial last block
  Tensor w({n, k});
  for (auto& v : w.data) v = u(rng);
  Tensor x({3, k});
  for (auto& v : x.data) v = u(rng);

  QuantizedTensor qt;
  qt.type = QuantType::kQ40;
  qt.shape = {n, k};
  qt.q4_0_data = quantizeQ40(w);
  HipModelWeights storage;
  uploadLinearWeight(storage, qt, "layers.0.wq", 0);
  CHECK(storage.weights.size() == 1);
  const HipUploadedWeight* up = findHipWeight(storage, "layers.0.wq", QuantType::kQ40);
  CHECK(up != nullptr);

  HipTensor xd = hipTensorFromHost(x, 0);
  Tensor via_registry =
      hipQ40LinearDeviceInput(xd, up->buffer.data(), qt.q4_0_data.size(), qt.shape, 0)
          .download();
  Tensor via_uploaded = hipLinearUploaded(xd, *up, 0).download();
  HipDeviceBuffer aos(qt.q4_0_data.size() * sizeof(BlockQ40), 0);
  aos.upload(qt.q4_0_data.data(), aos.bytes());
  Tensor via_aos =
      hipQ40LinearDeviceInput(xd, aos.data(), qt.q4_0_data.size(), qt.shape, 0)
          .download();
  Tensor cpu = cpuLinear(x, qt.q4_0_data, qt.shape);
  // a registered buffer runs the tiled kernels; a raw AoS pointer (3 rows)
  // runs the GEMV that reads the blocks as they are, in fp32 like the CPU
  // loop but in another summation order
  CHECK(expectNear(via_registry, via_uploaded, 0.0f, "registry vs uploaded (bit-exact)"));
  CHECK(expectNear(via_registry, via_aos, 1e-5f, "registry vs aos"));
  CHECK(expectNear(via_aos, cpu, 1e-5f, "aos vs cpu"));
  CHECK(expectNear(via_registry, cpu, 1e-4f, "registry vs cpu"));
  return true;
}

// ---- F32 projections: hipLinearUploaded runs them as forwardLinearDevice does
// (src/forward.cc:206-209, cudaLinearDeviceInput) ------------------------------
TEST(hip_uploaded_f32_weight_matches_cpu) {
  SKIP_WITHOUT_HIP();
  std::mt19937 rng(77);
  std::uniform_real_distribution<float> u(-1.0f, 1.0f);
  const int n = 37, k = 70;
  Tensor w({n, k});
  for (auto& v : w.data) v = u(rng);
  QuantizedTensor qt;
  qt.type = QuantType::kF32;
  qt.shape = {n, k};
  qt.f32_data = w.data;
  HipModelWeights storage;
  uploadLinearWeight(storage, qt, "layers.0.wo", 0);
  const HipUploadedWeight* up = findHipWeight(storage, "layers.0.wo", QuantType::kF32);
  CHECK(up != nullptr);
  for (int rows : {1, 3, 9}) {
    Tensor x({rows, k});
    for (auto& v : x.data) v = u(rng);
    Tensor got = hipLinearUploaded(hipTensorFromHost(x, 0), *up, 0).download();
    Tensor want({rows, n});
    for (int r = 0; r < rows; ++r)
      ref_linear_f32(x.data.data() + (size_t)r * k, w.data.data(), want.data.data() + (size_t)r * n,
                     n, k);
    CHECK(expectNear(got, want, 1e-4f, "uploaded F32 vs linearNaive"));
    // the host and device F32 entry points agree with it
    CHECK(expectNear(hipLinear(x, w), want, 1e-4f, "hipLinear"));
    CHECK(expectNear(hipLinearDeviceWeight(x, up->buffer.data(), qt.shape), want, 1e-4f,
                     "hipLinearDeviceWeight"));
  }
  // 1-D input keeps a 1-D output (cuda_matmul.cc:223-226)
  Tensor x1({k});
  for (auto& v : x1.data) v = u(rng);
  HipTensor y1 = hipLinearDeviceInput(hipTensorFromHost(x1, 0), up->buffer.data(), qt.shape, 0);
  CHECK(y1.shape() == std::vector<int>{n});
  CHECK(throwsAs<std::runtime_error>([&] {
    (void)hipLinearDeviceInput(hipTensorFromHost(x1, 0), up->buffer.data(), {n, k + 1}, 0);
  }));
  CHECK(throwsAs<std::runtime_error>(
      [&] { (void)hipLinearDeviceInput(hipTensorFromHost(x1, 0), nullptr, qt.shape, 0); }));
  return true;
}

// ---- cudaMatmul's contract: c = a @ b (tests/test_cuda.cc matmul cases) ----
TEST(hip_matmul_matches_cpu) {
  SKIP_WITHOUT_HIP();
  Tensor a({3, 5}), b({5, 4});
  fillLinear(a, 0.1f, -0.7f);
  fillLinear(b, 0.05f, -0.5f);
  Tensor c = hipMatmul(a, b);
  Tensor want({3, 4});
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 4; ++j) {
      double s = 0.0;
      for (int t = 0; t < 5; ++t) s += (double)a.at2(i, t) * b.at2(t, j);
      want.at2(i, j) = (float)s;
    }
  CHECK(expectNear(c, want, 1e-5f, "hipMatmul"));
  CHECK(throwsAs<std::runtime_error>([&] { (void)hipMatmul(a, a); }));
  return true;
}

// ---- the operators against the oracle (ops.cc restatements) ----------------
TEST(hip_ops_match_cpu) {
  SKIP_WITHOUT_HIP();
  Tensor x({33}), w({33}), b({33});
  fillLinear(x, 0.11f, -1.7f);
  fillLinear(w, 0.03f, 0.4f);
  fillLinear(b, -0.07f, 0.9f);
  Tensor want(x.shape);
  ref_rmsnorm(x.data.data(), w.data.data(), want.data.data(), 33, 1e-5f);
  CHECK(expectNear(hipRmsNorm(x, w, 1e-5f), want, 1e-5f, "hipRmsNorm"));
  HipTensor xd = hipTensorFromHost(x, 0), bd = hipTensorFromHost(b, 0);
  CHECK(expectNear(hipRmsNormDeviceInput(xd, w, 1e-5f).download(), want, 1e-5f,
                   "hipRmsNormDeviceInput"));
  ref_softmax(x.data.data(), want.data.data(), 33);
  CHECK(expectNear(hipSoftmax(x), want, 1e-6f, "hipSoftmax"));
  for (size_t i = 0; i < x.size(); ++i) want.data[i] = x.data[i] / (1.0f + std::exp(-x.data[i]));
  CHECK(expectNear(hipSilu(x), want, 1e-6f, "hipSilu"));
  CHECK(expectNear(hipSiluDeviceInput(xd).download(), want, 1e-6f, "hipSiluDeviceInput"));
  for (size_t i = 0; i < x.size(); ++i) want.data[i] = x.data[i] * b.data[i];
  CHECK(expectNear(hipElementwiseMul(x, b), want, 0.0f, "hipElementwiseMul"));
  CHECK(expectNear(hipElementwiseMulDeviceInput(xd, bd).download(), want, 0.0f, "mul device"));
  for (size_t i = 0; i < x.size(); ++i) want.data[i] = x.data[i] + b.data[i];
  CHECK(expectNear(hipElementwiseAdd(x, b), want, 0.0f, "hipElementwiseAdd"));
  CHECK(expectNear(hipElementwiseAddDeviceInput(xd, bd).download(), want, 0.0f, "add device"));
  CHECK(expectNear(hipElementwiseAddDeviceWeight(xd, bd.data(), b.shape).download(), want, 0.0f,
                   "add device weight"));
  CHECK(throwsAs<std::runtime_error>([&] { (void)hipRmsNorm(x, w, 0.0f); }));
  CHECK(throwsAs<std::runtime_error>([&] { (void)hipElementwiseAdd(x, Tensor({32})); }));
  // embedding row and its range check
  Tensor table({5, 33});
  fillLinear(table, 0.01f, -0.2f);
  HipTensor td = hipTensorFromHost(table, 0);
  Tensor row = hipEmbeddingLookupDeviceWeight(td.data(), table.shape, 3).download();
  for (int i = 0; i < 33; ++i) CHECK(row.data[i] == table.at2(3, i));
  CHECK(throwsAs<std::out_of_range>(
      [&] { (void)hipEmbeddingLookupDeviceWeight(td.data(), table.shape, 5); }));
  // RoPE host and device forms against the oracle, both pairings
  for (RopeType rt : {RopeType::kNormal, RopeType::kNeoX}) {
    Tensor q({4, 8}), k({2, 8});
    fillLinear(q, 0.05f, -0.8f);
    fillLinear(k, -0.04f, 0.6f);
    Tensor qw = q, kw = k;
    CHECK(ref_rope(qw.data.data(), kw.data.data(), 4, 2, 8, 7, 10000.0f,
                   rt == RopeType::kNeoX ? 1 : 0) == 0);
    Tensor qh = q, kh = k;
    hipRope(qh, kh, 7, 10000.0f, rt);
    CHECK(expectNear(qh, qw, 2e-6f, "hipRope q"));
    CHECK(expectNear(kh, kw, 2e-6f, "hipRope k"));
    HipTensor qd = hipTensorFromHost(q, 0), kd = hipTensorFromHost(k, 0);
    hipRopeDeviceInput(qd, kd, 4, 2, 8, 7, 10000.0f, rt);
    CHECK(expectNear(qd.download(), qw, 2e-6f, "hipRopeDeviceInput q"));
  }
  return true;
}

// ---- KV cache + decode attention (tests/test_cuda.cc:962-1141 style) --------
TEST(hip_kv_cache_and_attention_match_cpu) {
  SKIP_WITHOUT_HIP();
  const int layers = 2, seq = 16, nkv = 2, hd = 8, nh = 4;
  HipKvCache cache(layers, seq, nkv, hd, 0);
  CHECK(!cache.empty());
  CHECK(cache.bytes() == (size_t)2 * layers * seq * nkv * hd * 4);
  std::vector<float> keys((size_t)layers * seq * nkv * hd, 0.0f), values(keys.size(), 0.0f);
  std::mt19937 rng(5);
  std::uniform_real_distribution<float> u(-1.0f, 1.0f);
  for (int p = 0; p < 5; ++p) {
    Tensor k({nkv, hd}), v({nkv, hd});
    for (auto& e : k.data) e = u(rng);
    for (auto& e : v.data) e = u(rng);
    if (p % 2 == 0) {
      cache.write(1, p, k, v);
    } else {
      HipTensor kd = hipTensorFromHost(k, 0), vd = hipTensorFromHost(v, 0);
      cache.writeDevice(1, p, kd, vd);
    }
    std::copy(k.data.begin(), k.data.end(), keys.begin() + ((size_t)(seq + p) * nkv * hd));
    std::copy(v.data.begin(), v.data.end(), values.begin() + ((size_t)(seq + p) * nkv * hd));
    CHECK(expectNear(cache.readKey(1, p), k, 0.0f, "readKey"));
    Tensor vh({hd});
    std::copy(v.data.begin() + hd, v.data.end(), vh.data.begin());
    CHECK(expectNear(cache.readValueHead(1, p, 1), vh, 0.0f, "readValueHead"));
  }
  Tensor q({nh, hd});
  for (auto& e : q.data) e = u(rng);
  Tensor want({nh, hd});
  ref_attention(q.data.data(), keys.data(), values.data(), 1, 4, nh, nkv, hd, seq,
                want.data.data());
  CHECK(expectNear(hipAttentionDecode(q, cache, 1, 4, nh, nkv, hd), want, 1e-5f,
                   "hipAttentionDecode"));
  HipTensor qd = hipTensorFromHost(q, 0);
  Tensor got = hipAttentionDecodeDeviceInput(qd, cache, 1, 4, nh, nkv, hd).download();
  got.shape = {nh, hd};
  CHECK(expectNear(got, want, 1e-5f, "hipAttentionDecodeDeviceInput"));
  CHECK(throwsAs<std::out_of_range>([&] { (void)cache.readKey(2, 0); }));
  CHECK(throwsAs<std::out_of_range>([&] { (void)cache.readKey(0, seq); }));
  CHECK(throwsAs<std::out_of_range>([&] { (void)hipAttentionDecode(q, cache, 1, seq, nh, nkv, hd); }));
  CHECK(throwsAs<std::runtime_error>([&] { (void)hipAttentionDecode(q, cache, 1, 4, 3, nkv, hd); }));
  // downloadTo into a host tensor of another shape throws
  // (CudaTensor::downloadTo, src/cuda_tensor.cc:88-95)
  Tensor wrong({3});
  CHECK(throwsAs<std::runtime_error>([&] { qd.downloadTo(wrong); }));
  CHECK(wrong.shape == std::vector<int>{3});
  cache.clear();
  CHECK(expectNear(cache.readKey(1, 0), Tensor({nkv, hd}), 0.0f, "cleared"));
  return true;
}

// ---- larger shapes through every host entry point, all three types --------
TEST(hip_all_types_random_shapes) {
  SKIP_WITHOUT_HIP();
  std::mt19937 rng(99);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  const int shapes[][3] = {{1, 64, 96}, {2, 33, 257}, {5, 100, 512}, {8, 16, 4096},
                           {17, 48, 300}, {130, 130, 160}};
  for (const auto& s : shapes) {
    const int m = s[0], n = s[1], k = s[2];
    Tensor w({n, k});
    for (auto& v : w.data) v = 0.05f * nd(rng);
    Tensor x({m, k});
    for (auto& v : x.data) v = nd(rng);
    auto b8 = quantizeQ80(w);
    auto b4 = quantizeQ40(w);
    std::vector<BlockQ41> b41(b4.size());
    for (size_t i = 0; i < b4.size(); ++i) {
      b41[i].d = b4[i].d;
      b41[i].m = b8[i].d;  // any fp16 value
      std::memcpy(b41[i].qs, b4[i].qs, 16);
    }
    // GEMV rows (m <= 8) are fp32-class; the MFMA GEMM rounds operands to
    // fp16: stated tolerance = allclose(rtol 2e-3, atol 1e-3*|x|*sqrt(k/4096))
    auto check = [&](const Tensor& got, const Tensor& ref, const char* what) {
      for (int r = 0; r < m; ++r) {
        double xn = 0;
        for (int kk = 0; kk < k; ++kk) xn += (double)x.at2(r, kk) * x.at2(r, kk);
        const double atol = 1e-3 * std::sqrt(xn) * std::sqrt(k / 4096.0);
        for (int c = 0; c < n; ++c) {
          const double a = got.at2(r, c), e = ref.at2(r, c);
          const double err = std::fabs(a - e);
          if (!(err <= atol || err <= 2e-3 * std::fabs(e))) {
            std::cerr << "  " << what << " m=" << m << " n=" << n << " k=" << k
                      << " at (" << r << "," << c << "): " << a << " vs " << e
                      << "\n";
            return false;
          }
        }
      }
      return true;
    };
    CHECK(check(hipQ80Linear(x, b8, {n, k}), cpuLinear(x, b8, {n, k}), "q8_0"));
    CHECK(check(hipQ40Linear(x, b4, {n, k}), cpuLinear(x, b4, {n, k}), "q4_0"));
    CHECK(check(hipQ41Linear(x, b41, {n, k}), cpuLinear(x, b41, {n, k}), "q4_1"));
  }
  return true;
}

TEST(backend_hip_parses) {
  BackendKind kind = BackendKind::kCpu;
  CHECK(parseBackendKind("hip", kind) && kind == BackendKind::kHip);
  CHECK(backendKindName(BackendKind::kHip) == "hip");
  CHECK(parseBackendKind("cuda", kind) && kind == BackendKind::kCuda);
  CHECK(!parseBackendKind("rocm", kind));
  BackendConfig cfg;
  cfg.kind = BackendKind::kCuda;
  CHECK(throwsAs<std::runtime_error>([&] { validateBackend(cfg); }));
  if (hipAvailable()) {
    cfg.kind = BackendKind::kHip;
    validateBackend(cfg);
    std::cout << "  " << hipDeviceSummary(0) << "\n";
  }
  return true;
}

int main(int argc, char** argv) {
  const char* filter = argc > 1 ? argv[1] : nullptr;
  int failed = 0, run = 0;
  for (const auto& t : registry()) {
    if (filter && std::strstr(t.name, filter) == nullptr) continue;
    ++run;
    std::cout << "[ RUN  ] " << t.name << std::endl;
    bool ok = false;
    try {
      ok = t.fn();
    } catch (const std::exception& e) {
      std::cerr << "  exception: " << e.what() << "\n";
    }
    std::cout << (ok ? "[  OK  ] " : "[ FAIL ] ") << t.name << std::endl;
    if (!ok) ++failed;
  }
  std::cout << run - failed << "/" << run << " passed" << std::endl;
  return failed == 0 ? 0 : 1;
}
