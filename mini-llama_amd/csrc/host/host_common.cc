#include "host_common.h"

#include <hip/hip_runtime_api.h>

#include <map>
#include <stdexcept>

#include "mini_llama/hip_runtime.h"
#include "mlq.h"

namespace mini_llama {

void checkMlq(int rc, const char* prefix, const std::string& what) {
  if (rc == MLQ_OK) return;
  const std::string detail =
      rc == MLQ_ERR_HIP ? hipGetErrorString(static_cast<hipError_t>(mlq_last_hip_error()))
                        : mlq_status_string(rc);
  throw std::runtime_error(std::string(prefix) + " " + what + ": " + detail);
}

Workspace deviceWorkspace(WorkspaceSlot slot, int device_id, size_t bytes) {
  static std::mutex mu[kWorkspaceSlots];
  static std::map<int, HipDeviceBuffer> buffers[kWorkspaceSlots];
  Workspace w;
  w.lock = std::unique_lock<std::mutex>(mu[slot]);
  HipDeviceBuffer& buf = buffers[slot][device_id];
  if (buf.bytes() < bytes) buf.reset(bytes, device_id);
  w.data = buf.data();
  return w;
}

}  // namespace mini_llama
