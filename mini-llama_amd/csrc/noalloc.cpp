// mlq_linear_epi_noalloc: the quantized Linear with its scratch memory taken
// from a fixed device array instead of a caller workspace, for callers that
// cannot allocate (code under HIP graph capture, serving loops, harnesses
// that forbid hipMalloc). It runs exactly the kernels of mlq_linear_epi.
//
// The array lives in this translation unit's code object, so every device
// the library runs on holds its own copy, at its own address, until the
// process ends. In host code `scratch` is only a host-side stand-in for that
// symbol; the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, and only that address is ever handed
// to a kernel.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "kernels/launch.h"
#include "mlq.h"

namespace {

constexpr size_t kScratchBytes = (size_t)MLQ_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch must keep 256-byte alignment");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};

DeviceScratch g_scratch[kMaxDevices];

// Device address of `scratch` on `device` (looked up on the first call for
// that device, with the device made current for the lookup).
hipError_t scratch_for(int device, void** out) {
  DeviceScratch& s = g_scratch[device];
  std::call_once(s.once, [&] {
    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess && prev != device) e = hipSetDevice(device);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev >= 0 && prev != device) {
      const hipError_t r = hipSetDevice(prev);
      if (e == hipSuccess) e = r;
    }
    s.err = e;
    s.ptr = e == hipSuccess ? p : nullptr;
  });
  *out = s.ptr;
  return s.err;
}

}  // namespace

extern "C" {

int mlq_linear_epi_noalloc(const mlq_weight* w, const float* x, float* y, int m,
                           const float* bias, int act, mlq_stream_t stream) {
  size_t need = 0;
  int rc = mlq_linear_workspace(w, m, &need);  // also validates w and m
  if (rc != MLQ_OK) return rc;
  if (x == nullptr || y == nullptr) return MLQ_ERR_INVALID_ARG;
  if (need > kScratchBytes) return MLQ_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  if (need > 0) {
    // the device the launches go to: the stream's, else the current one
    int device = 0;
    hipError_t e = stream != nullptr ? hipStreamGetDevice((hipStream_t)stream, &device)
                                     : hipGetDevice(&device);
    if (e != hipSuccess) return mlq::record_hip(e);
    if (device < 0 || device >= kMaxDevices) return MLQ_ERR_NO_DEVICE;
    e = scratch_for(device, &ws);
    if (e != hipSuccess) return mlq::record_hip(e);
  }
  return mlq_linear_epi(w, x, y, m, bias, act, ws, need > 0 ? kScratchBytes : 0, stream);
}

}  // extern "C"
