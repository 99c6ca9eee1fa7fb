// Backend selection with the new `hip` backend
// (reference: include/mini_llama/backend.h:11-33, src/backdend.cc:12-85).
// `--backend hip` parses to BackendKind::kHip; kCuda stays a known name so a
// mixed build can still report it, but this build does not provide it.
#ifndef MINI_LLAMA_HIP_BACKEND_H_
#define MINI_LLAMA_HIP_BACKEND_H_

#include <string>

namespace mini_llama {

enum class BackendKind {
  kCpu,
  kCuda,
  kHip,
};

struct BackendConfig {
  BackendKind kind = BackendKind::kCpu;
  int device_id = 0;
  bool device_id_set = false;
};

bool parseBackendKind(const std::string& text, BackendKind& kind);
std::string backendKindName(BackendKind kind);

bool cudaBackendBuilt();  // always false in this build
bool hipBackendBuilt();
bool hipBackendAvailable(int device_id = 0);
std::string hipDeviceSummary(int device_id = 0);

// Throws std::runtime_error when the requested backend cannot run here.
void validateBackend(const BackendConfig& config);

// Explains which execution path is active.
std::string backendExecutionNote(const BackendConfig& config);

}  // namespace mini_llama

#endif  // MINI_LLAMA_HIP_BACKEND_H_
