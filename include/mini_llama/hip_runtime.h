// HIP device runtime for the mini-llama HIP backend: device queries, device
// selection, copies and an RAII device buffer.
// Mirrors include/mini_llama/cuda_runtime.h:12-69 with hip* names. All
// failures throw std::runtime_error("HIP runtime error in <expr>: <msg>").
#ifndef MINI_LLAMA_HIP_RUNTIME_H_
#define MINI_LLAMA_HIP_RUNTIME_H_

#include <cstddef>
#include <string>

namespace mini_llama {

struct HipDeviceInfo {
  int id = 0;
  std::string name;
  std::string gcn_arch;  // e.g. "gfx950:sramecc+:xnack-"
  int compute_units = 0;
  size_t total_memory_bytes = 0;
  int driver_version = 0;
  int runtime_version = 0;
};

enum class HipMemcpyKind {
  kHostToDevice,
  kDeviceToHost,
  kDeviceToDevice,
};

bool hipRuntimeBuilt();
int hipDeviceCount();  // 0 when no device is visible (never throws)
void hipSetDeviceId(int device_id);
HipDeviceInfo hipGetDeviceInfo(int device_id);
std::string hipFormatDeviceInfo(const HipDeviceInfo& info);

void* hipMallocBytes(size_t bytes);
void hipFreeBytes(void* ptr);
// Synchronous copy (like cudaMemcpyBytes, src/cuda_runtime.cc:145-164).
void hipMemcpyBytes(void* dst, const void* src, size_t bytes,
                    HipMemcpyKind kind);
// Blocks until all work on the device's null stream is done.
void hipSynchronizeDevice(int device_id);

class HipDeviceBuffer {
 public:
  HipDeviceBuffer() = default;
  explicit HipDeviceBuffer(size_t bytes, int device_id = 0);
  ~HipDeviceBuffer();

  HipDeviceBuffer(const HipDeviceBuffer&) = delete;
  HipDeviceBuffer& operator=(const HipDeviceBuffer&) = delete;

  HipDeviceBuffer(HipDeviceBuffer&& other) noexcept;
  HipDeviceBuffer& operator=(HipDeviceBuffer&& other) noexcept;

  void reset();
  void reset(size_t bytes, int device_id = 0);

  void upload(const void* src, size_t bytes);
  void download(void* dst, size_t bytes) const;

  void* data() { return data_; }
  const void* data() const { return data_; }
  size_t bytes() const { return bytes_; }
  int device_id() const { return device_id_; }
  bool empty() const { return data_ == nullptr; }

 private:
  void releaseNoexcept() noexcept;

  void* data_ = nullptr;
  size_t bytes_ = 0;
  int device_id_ = 0;
};

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_RUNTIME_H_
