// Decode-step operators, host layer (include/mini_llama/hip_ops.h): the
// reference's validation and messages (src/cuda_ops.cu:40-733) over the
// operator entry points of libmlq.
#include "mini_llama/hip_ops.h"

#include <cmath>
#include <stdexcept>
#include <string>

#include "host_common.h"
#include "mlq.h"

namespace mini_llama {
namespace {

constexpr const char* kErr = "HIP ops error in";

void requireSameShape(const Tensor& a, const Tensor& b, const char* caller) {
  if (a.shape != b.shape)
    throw std::runtime_error(std::string(caller) + ": shape mismatch " + a.shapeString() +
                             " vs " + b.shapeString());
  if (a.size() == 0) throw std::runtime_error(std::string(caller) + ": empty tensor");
}

void requireSameShape(const HipTensor& a, const HipTensor& b, const char* caller) {
  if (a.shape() != b.shape())
    throw std::runtime_error(std::string(caller) + ": shape mismatch " + a.shapeString() +
                             " vs " + b.shapeString());
  if (a.deviceId() != b.deviceId())
    throw std::runtime_error(std::string(caller) + ": tensors are on different HIP devices");
  if (a.size() == 0) throw std::runtime_error(std::string(caller) + ": empty tensor");
}

void require1D(const std::string& shape_str, int dims, size_t size, const char* caller) {
  if (dims != 1)
    throw std::runtime_error(std::string(caller) + ": expected 1D tensor, got " + shape_str);
  if (size == 0) throw std::runtime_error(std::string(caller) + ": empty tensor");
}
void require1D(const Tensor& x, const char* caller) {
  require1D(x.shapeString(), x.numDims(), x.size(), caller);
}
void require1D(const HipTensor& x, const char* caller) {
  require1D(x.shapeString(), x.numDims(), x.size(), caller);
}

void requireEps(float eps, const char* caller) {
  if (!std::isfinite(eps) || eps <= 0.0f)
    throw std::runtime_error(std::string(caller) + ": eps must be finite and positive");
}

const float* cf(const HipTensor& t) { return static_cast<const float*>(t.data()); }
float* f(HipTensor& t) { return static_cast<float*>(t.data()); }

// Host interface: upload the inputs, run, download (src/cuda_ops.cu:180-280).
template <typename Launch>
Tensor hostCall(const std::vector<const Tensor*>& inputs, const std::vector<int>& out_shape,
                int device_id, Launch launch) {
  hipSetDeviceId(device_id);
  std::vector<HipTensor> dev;
  for (const Tensor* t : inputs) dev.push_back(hipTensorFromHost(*t, device_id));
  HipTensor y(out_shape, device_id);
  launch(dev, y);
  return y.download();
}

HipTensor rmsNormDevice(const HipTensor& x, const float* w, float eps, int device_id,
                        const char* caller) {
  hipSetDeviceId(device_id);
  HipTensor y(x.shape(), device_id);
  checkMlq(mlq_rmsnorm(cf(x), w, f(y), 1, static_cast<int>(x.size()), eps, nullptr), kErr,
           caller);
  return y;
}

int eltwise(int op, const float* a, const float* b, float* y, int64_t n) {
  switch (op) {
    case 0: return mlq_add(a, b, y, n, nullptr);
    case 1: return mlq_mul(a, b, y, n, nullptr);
    default: return mlq_silu(a, y, n, nullptr);
  }
}

int ropeType(RopeType t) { return t == RopeType::kNeoX ? MLQ_ROPE_NEOX : MLQ_ROPE_NORMAL; }

}  // namespace

bool hipOpsBuilt() { return true; }

Tensor hipRmsNorm(const Tensor& x, const Tensor& weight, float eps, int device_id) {
  require1D(x, "hipRmsNorm");
  require1D(weight, "hipRmsNorm");
  if (x.shape != weight.shape) throw std::runtime_error("hipRmsNorm: x and weight shape mismatch");
  requireEps(eps, "hipRmsNorm");
  return hostCall({&x, &weight}, x.shape, device_id, [&](std::vector<HipTensor>& d, HipTensor& y) {
    checkMlq(mlq_rmsnorm(cf(d[0]), cf(d[1]), f(y), 1, static_cast<int>(x.size()), eps, nullptr),
             kErr, "hipRmsNorm");
  });
}

Tensor hipSilu(const Tensor& x, int device_id) {
  if (x.size() == 0) throw std::runtime_error("hipSilu: empty tensor");
  return hostCall({&x}, x.shape, device_id, [&](std::vector<HipTensor>& d, HipTensor& y) {
    checkMlq(eltwise(2, cf(d[0]), nullptr, f(y), (int64_t)x.size()), kErr, "hipSilu");
  });
}

Tensor hipElementwiseMul(const Tensor& a, const Tensor& b, int device_id) {
  requireSameShape(a, b, "hipElementwiseMul");
  return hostCall({&a, &b}, a.shape, device_id, [&](std::vector<HipTensor>& d, HipTensor& y) {
    checkMlq(eltwise(1, cf(d[0]), cf(d[1]), f(y), (int64_t)a.size()), kErr, "hipElementwiseMul");
  });
}

Tensor hipElementwiseAdd(const Tensor& a, const Tensor& b, int device_id) {
  requireSameShape(a, b, "hipElementwiseAdd");
  return hostCall({&a, &b}, a.shape, device_id, [&](std::vector<HipTensor>& d, HipTensor& y) {
    checkMlq(eltwise(0, cf(d[0]), cf(d[1]), f(y), (int64_t)a.size()), kErr, "hipElementwiseAdd");
  });
}

HipTensor hipRmsNormDeviceWeight(const HipTensor& x, const void* weight_data,
                                 const std::vector<int>& weight_shape, float eps, int device_id) {
  // validateRmsNormDeviceWeight (src/cuda_ops.cu:83-103)
  require1D(x, "hipRmsNormDeviceWeight");
  if (weight_data == nullptr)
    throw std::runtime_error("hipRmsNormDeviceWeight: weight data is null");
  if (weight_shape != x.shape())
    throw std::runtime_error("hipRmsNormDeviceWeight: x and weight shape mismatch");
  if (x.deviceId() != device_id)
    throw std::runtime_error(
        "hipRmsNormDeviceWeight: input tensor is on a different HIP device");
  requireEps(eps, "hipRmsNormDeviceWeight");
  return rmsNormDevice(x, static_cast<const float*>(weight_data), eps, device_id,
                       "hipRmsNormDeviceWeight");
}

HipTensor hipRmsNormDeviceInput(const HipTensor& x, const Tensor& weight, float eps,
                                int device_id) {
  require1D(x, "hipRmsNormDeviceInput");
  require1D(weight, "hipRmsNormDeviceInput");
  if (weight.shape != x.shape())
    throw std::runtime_error("hipRmsNormDeviceInput: x and weight shape mismatch");
  if (x.deviceId() != device_id)
    throw std::runtime_error("hipRmsNormDeviceInput: input tensor is on a different HIP device");
  requireEps(eps, "hipRmsNormDeviceInput");
  HipTensor w = hipTensorFromHost(weight, device_id);
  return rmsNormDevice(x, cf(w), eps, device_id, "hipRmsNormDeviceInput");
}

HipTensor hipSiluDeviceInput(const HipTensor& x, int device_id) {
  if (x.deviceId() != device_id)
    throw std::runtime_error("hipSiluDeviceInput: input tensor is on a different HIP device");
  if (x.size() == 0) throw std::runtime_error("hipSiluDeviceInput: empty tensor");
  hipSetDeviceId(device_id);
  HipTensor y(x.shape(), device_id);
  checkMlq(eltwise(2, cf(x), nullptr, f(y), (int64_t)x.size()), kErr, "hipSiluDeviceInput");
  return y;
}

HipTensor hipElementwiseMulDeviceInput(const HipTensor& a, const HipTensor& b, int device_id) {
  requireSameShape(a, b, "hipElementwiseMulDeviceInput");
  if (a.deviceId() != device_id)
    throw std::runtime_error(
        "hipElementwiseMulDeviceInput: input tensor is on a different HIP device");
  hipSetDeviceId(device_id);
  HipTensor y(a.shape(), device_id);
  checkMlq(eltwise(1, cf(a), cf(b), f(y), (int64_t)a.size()), kErr,
           "hipElementwiseMulDeviceInput");
  return y;
}

HipTensor hipElementwiseAddDeviceInput(const HipTensor& a, const HipTensor& b, int device_id) {
  requireSameShape(a, b, "hipElementwiseAddDeviceInput");
  if (a.deviceId() != device_id)
    throw std::runtime_error(
        "hipElementwiseAddDeviceInput: input tensor is on a different HIP device");
  hipSetDeviceId(device_id);
  HipTensor y(a.shape(), device_id);
  checkMlq(eltwise(0, cf(a), cf(b), f(y), (int64_t)a.size()), kErr,
           "hipElementwiseAddDeviceInput");
  return y;
}

HipTensor hipElementwiseAddDeviceWeight(const HipTensor& a, const void* b_data,
                                        const std::vector<int>& b_shape, int device_id) {
  // validateAddDeviceWeight (src/cuda_ops.cu:105-121)
  if (a.deviceId() != device_id)
    throw std::runtime_error(
        "hipElementwiseAddDeviceWeight: input tensor is on a different HIP device");
  if (b_data == nullptr)
    throw std::runtime_error("hipElementwiseAddDeviceWeight: weight data is null");
  if (a.shape() != b_shape)
    throw std::runtime_error("hipElementwiseAddDeviceWeight: input and weight shape mismatch");
  if (a.size() == 0) throw std::runtime_error("hipElementwiseAddDeviceWeight: empty tensor");
  hipSetDeviceId(device_id);
  HipTensor y(a.shape(), device_id);
  checkMlq(eltwise(0, cf(a), static_cast<const float*>(b_data), f(y), (int64_t)a.size()), kErr,
           "hipElementwiseAddDeviceWeight");
  return y;
}

Tensor hipSoftmax(const Tensor& x, int device_id) {
  require1D(x, "hipSoftmax");
  return hostCall({&x}, x.shape, device_id, [&](std::vector<HipTensor>& d, HipTensor& y) {
    checkMlq(mlq_softmax(cf(d[0]), f(y), (int64_t)x.size(), nullptr), kErr, "hipSoftmax");
  });
}

HipTensor hipEmbeddingLookupDeviceWeight(const void* embedding_data,
                                         const std::vector<int>& embedding_shape, int token_id,
                                         int device_id) {
  // src/cuda_ops.cu:608-628
  if (embedding_data == nullptr)
    throw std::runtime_error("hipEmbeddingLookupDeviceWeight: embedding data is null");
  if (embedding_shape.size() != 2)
    throw std::runtime_error("hipEmbeddingLookupDeviceWeight: expected 2D embedding weight");
  const int vocab = embedding_shape[0], dim = embedding_shape[1];
  if (vocab <= 0 || dim <= 0)
    throw std::runtime_error("hipEmbeddingLookupDeviceWeight: embedding shape must be positive");
  if (token_id < 0 || token_id >= vocab)
    throw std::out_of_range("hipEmbeddingLookupDeviceWeight: token id out of range");
  hipSetDeviceId(device_id);
  HipTensor y({dim}, device_id);
  checkMlq(mlq_embedding(static_cast<const float*>(embedding_data), vocab, dim, token_id, f(y),
                         nullptr),
           kErr, "hipEmbeddingLookupDeviceWeight");
  return y;
}

void hipRope(Tensor& q, Tensor& k, int pos, float theta, RopeType rope_type, int device_id) {
  // src/cuda_ops.cu:643-660
  if (q.numDims() != 2 || k.numDims() != 2)
    throw std::runtime_error("hipRope: expected 2D tensors");
  if (pos < 0) throw std::out_of_range("hipRope: position must be non-negative");
  if (!std::isfinite(theta) || theta <= 0.0f)
    throw std::runtime_error("hipRope: theta must be finite and positive");
  if (q.shape[1] != k.shape[1]) throw std::runtime_error("hipRope: q and k head_dim mismatch");
  const int hd = q.shape[1];
  if (hd <= 0 || hd % 2 != 0)
    throw std::runtime_error("hipRope: head_dim must be positive and even");
  if (q.shape[0] <= 0 || k.shape[0] <= 0) throw std::runtime_error("hipRope: empty tensor");
  hipSetDeviceId(device_id);
  HipTensor qd = hipTensorFromHost(q, device_id);
  HipTensor kd = hipTensorFromHost(k, device_id);
  checkMlq(mlq_rope(f(qd), f(kd), q.shape[0], k.shape[0], hd, pos, theta, ropeType(rope_type),
                    nullptr),
           kErr, "hipRope");
  qd.downloadTo(q);
  kd.downloadTo(k);
}

void hipRopeDeviceInput(HipTensor& q, HipTensor& k, int n_heads, int n_kv_heads, int head_dim,
                        int pos, float theta, RopeType rope_type, int device_id) {
  // src/cuda_ops.cu:694-716
  if (q.deviceId() != device_id || k.deviceId() != device_id)
    throw std::runtime_error("hipRopeDeviceInput: input tensor on different HIP device");
  if (n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0)
    throw std::runtime_error("hipRopeDeviceInput: invalid head shape");
  if (q.size() != (size_t)n_heads * (size_t)head_dim)
    throw std::runtime_error("hipRopeDeviceInput: q shape mismatch");
  if (k.size() != (size_t)n_kv_heads * (size_t)head_dim)
    throw std::runtime_error("hipRopeDeviceInput: k shape mismatch");
  if (pos < 0) throw std::out_of_range("hipRopeDeviceInput: position must be non-negative");
  if (!std::isfinite(theta) || theta <= 0.0f)
    throw std::runtime_error("hipRopeDeviceInput: theta must be finite and positive");
  hipSetDeviceId(device_id);
  checkMlq(mlq_rope(f(q), f(k), n_heads, n_kv_heads, head_dim, pos, theta, ropeType(rope_type),
                    nullptr),
           kErr, "hipRopeDeviceInput");
}

}  // namespace mini_llama
