// Helpers shared by the C++ host layer of the HIP backend (library-private).
#pragma once

#include <cstddef>
#include <mutex>
#include <string>

namespace mini_llama {

// mlq status -> std::runtime_error "<prefix> <what>: <text>" (the HIP error
// string for MLQ_ERR_HIP), in the style of the reference's checkCuda*
// helpers (src/cuda_quant.cu:20-29, src/cuda_ops.cu:25-30).
void checkMlq(int rc, const char* prefix, const std::string& what);

// A grow-only per-device device buffer, held locked from the moment it is
// handed out until the caller drops it (after enqueuing the launches that
// use it), so another host thread cannot grow (free and reallocate) it in
// between. hipFree of an old buffer waits for the device, so work already
// enqueued on it completes first; launches go to the null stream, which
// orders the calls that reuse it.
struct Workspace {
  std::unique_lock<std::mutex> lock;
  void* data = nullptr;
};
enum WorkspaceSlot {
  kAosWorkspace = 0,         // raw AoS weights repacked per call
  kActivationWorkspace = 1,  // fp16 copy of x and split-K partials
  kAttentionWorkspace = 2,   // decode attention partials
  kWorkspaceSlots = 3
};
Workspace deviceWorkspace(WorkspaceSlot slot, int device_id, size_t bytes);

}  // namespace mini_llama
