// Backend selection with `hip` (mirrors src/backdend.cc:12-85).
#include "mini_llama/backend.h"

#include <stdexcept>
#include <string>

#include "mini_llama/hip_runtime.h"

namespace mini_llama {

bool parseBackendKind(const std::string& text, BackendKind& kind) {
  if (text == "cpu") {
    kind = BackendKind::kCpu;
    return true;
  }
  if (text == "cuda") {
    kind = BackendKind::kCuda;
    return true;
  }
  if (text == "hip") {
    kind = BackendKind::kHip;
    return true;
  }
  return false;
}

std::string backendKindName(BackendKind kind) {
  switch (kind) {
    case BackendKind::kCpu: return "cpu";
    case BackendKind::kCuda: return "cuda";
    case BackendKind::kHip: return "hip";
  }
  return "unknown";
}

bool cudaBackendBuilt() { return false; }

bool hipBackendBuilt() { return hipRuntimeBuilt(); }

bool hipBackendAvailable(int device_id) {
  const int count = hipDeviceCount();
  return device_id >= 0 && device_id < count;
}

std::string hipDeviceSummary(int device_id) {
  try {
    return hipFormatDeviceInfo(hipGetDeviceInfo(device_id));
  } catch (const std::exception& e) {
    return e.what();
  }
}

void validateBackend(const BackendConfig& config) {
  switch (config.kind) {
    case BackendKind::kCpu:
      if (config.device_id_set)
        throw std::runtime_error(
            "--device can only be used with --backend cuda or --backend hip.");
      return;
    case BackendKind::kCuda:
      throw std::runtime_error(
          "CUDA backend was not built. This build provides --backend hip.");
    case BackendKind::kHip:
      if (!hipBackendBuilt())
        throw std::runtime_error("HIP backend was not built.");
      if (!hipBackendAvailable(config.device_id))
        throw std::runtime_error("HIP device " +
                                 std::to_string(config.device_id) +
                                 " is not available: " +
                                 hipDeviceSummary(config.device_id));
      return;
  }
  throw std::runtime_error("unknown backend");
}

std::string backendExecutionNote(const BackendConfig& config) {
  if (config.kind == BackendKind::kCpu) return "compute: cpu";
  if (config.kind == BackendKind::kHip)
    return "compute: hip quantized Linear (Q8_0/Q4_0/Q4_1, tiled weights, "
           "gfx950 GEMV/MFMA kernels)";
  return "compute: cuda (not built)";
}

}  // namespace mini_llama
