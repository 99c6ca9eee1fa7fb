// HIP device runtime: queries, device selection, synchronous copies and the
// RAII device buffer (mirrors src/cuda_runtime.cc:50-238).
#include "mini_llama/hip_runtime.h"

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>
#include <utility>

#include "mini_llama/hip_weight_upload.h"

namespace mini_llama {
namespace {

void checkHip(hipError_t err, const char* expr) {
  if (err != hipSuccess) {
    throw std::runtime_error("HIP runtime error in " + std::string(expr) +
                             ": " + hipGetErrorString(err));
  }
}

hipMemcpyKind toHipKind(HipMemcpyKind kind) {
  switch (kind) {
    case HipMemcpyKind::kHostToDevice: return hipMemcpyHostToDevice;
    case HipMemcpyKind::kDeviceToHost: return hipMemcpyDeviceToHost;
    case HipMemcpyKind::kDeviceToDevice: return hipMemcpyDeviceToDevice;
  }
  return hipMemcpyDefault;
}

}  // namespace

bool hipRuntimeBuilt() { return true; }

int hipDeviceCount() {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return 0;
  return count;
}

void hipSetDeviceId(int device_id) {
  const int count = hipDeviceCount();
  if (device_id < 0 || device_id >= count) {
    throw std::runtime_error("HIP device id " + std::to_string(device_id) +
                             " out of range (" + std::to_string(count) +
                             " device(s) visible)");
  }
  checkHip(hipSetDevice(device_id), "hipSetDevice");
}

HipDeviceInfo hipGetDeviceInfo(int device_id) {
  hipSetDeviceId(device_id);
  hipDeviceProp_t prop;
  checkHip(hipGetDeviceProperties(&prop, device_id), "hipGetDeviceProperties");
  HipDeviceInfo info;
  info.id = device_id;
  info.name = prop.name;
  info.gcn_arch = prop.gcnArchName;
  info.compute_units = prop.multiProcessorCount;
  info.total_memory_bytes = prop.totalGlobalMem;
  checkHip(hipDriverGetVersion(&info.driver_version), "hipDriverGetVersion");
  checkHip(hipRuntimeGetVersion(&info.runtime_version), "hipRuntimeGetVersion");
  return info;
}

std::string hipFormatDeviceInfo(const HipDeviceInfo& info) {
  return "HIP device " + std::to_string(info.id) + ": " + info.name + " (" +
         info.gcn_arch + ", " + std::to_string(info.compute_units) + " CUs, " +
         std::to_string(info.total_memory_bytes >> 20) + " MiB, runtime " +
         std::to_string(info.runtime_version) + ")";
}

void* hipMallocBytes(size_t bytes) {
  if (bytes == 0) return nullptr;
  void* p = nullptr;
  checkHip(hipMalloc(&p, bytes), "hipMalloc");
  return p;
}

void hipFreeBytes(void* ptr) {
  if (ptr == nullptr) return;
  unregisterTiledWeight(ptr);
  checkHip(hipFree(ptr), "hipFree");
}

void hipMemcpyBytes(void* dst, const void* src, size_t bytes,
                    HipMemcpyKind kind) {
  if (bytes == 0) return;
  if (dst == nullptr || src == nullptr)
    throw std::runtime_error("hipMemcpyBytes: null pointer");
  checkHip(hipMemcpy(dst, src, bytes, toHipKind(kind)), "hipMemcpy");
}

void hipSynchronizeDevice(int device_id) {
  hipSetDeviceId(device_id);
  checkHip(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

HipDeviceBuffer::HipDeviceBuffer(size_t bytes, int device_id) {
  reset(bytes, device_id);
}

HipDeviceBuffer::~HipDeviceBuffer() { releaseNoexcept(); }

HipDeviceBuffer::HipDeviceBuffer(HipDeviceBuffer&& other) noexcept
    : data_(std::exchange(other.data_, nullptr)),
      bytes_(std::exchange(other.bytes_, 0)),
      device_id_(other.device_id_) {}

HipDeviceBuffer& HipDeviceBuffer::operator=(HipDeviceBuffer&& other) noexcept {
  if (this != &other) {
    releaseNoexcept();
    data_ = std::exchange(other.data_, nullptr);
    bytes_ = std::exchange(other.bytes_, 0);
    device_id_ = other.device_id_;
  }
  return *this;
}

void HipDeviceBuffer::reset() { releaseNoexcept(); }

void HipDeviceBuffer::reset(size_t bytes, int device_id) {
  releaseNoexcept();
  hipSetDeviceId(device_id);
  data_ = hipMallocBytes(bytes);
  bytes_ = bytes;
  device_id_ = device_id;
}

void HipDeviceBuffer::upload(const void* src, size_t bytes) {
  if (bytes > bytes_)
    throw std::runtime_error("HipDeviceBuffer::upload: " +
                             std::to_string(bytes) + " bytes exceed buffer of " +
                             std::to_string(bytes_));
  hipSetDeviceId(device_id_);
  hipMemcpyBytes(data_, src, bytes, HipMemcpyKind::kHostToDevice);
}

void HipDeviceBuffer::download(void* dst, size_t bytes) const {
  if (bytes > bytes_)
    throw std::runtime_error("HipDeviceBuffer::download: " +
                             std::to_string(bytes) + " bytes exceed buffer of " +
                             std::to_string(bytes_));
  hipSetDeviceId(device_id_);
  hipMemcpyBytes(dst, data_, bytes, HipMemcpyKind::kDeviceToHost);
}

void HipDeviceBuffer::releaseNoexcept() noexcept {
  if (data_ != nullptr) {
    unregisterTiledWeight(data_);
    (void)hipSetDevice(device_id_);
    (void)hipFree(data_);
  }
  data_ = nullptr;
  bytes_ = 0;
}

}  // namespace mini_llama
