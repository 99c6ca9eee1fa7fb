// Streaming-read probe: the time a plain read of `bytes` from HBM takes in
// one launch, the ceiling that the GEMV rooflines are compared against
// (mlq_read_probe, a measurement aid with no counterpart in the reference).
// Each wave reads whole contiguous 8 KiB chunks (dwordx4, non-temporal like
// the GEMV's weight lines), the grid sized to the chunk count; the data are
// folded into one word so the loads cannot be removed, and the word is
// stored only when it equals a value no input produces in practice.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "device_common.h"
#include "launch.h"

namespace mlq {
namespace {

constexpr int kProbeUnroll = 8;  // 16 B x 64 lanes x 8 = 8 KiB per wave

__global__ __launch_bounds__(256) void read_probe_kernel(const uint8_t* p, uint64_t bytes,
                                                         uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const uint64_t base = wave * (uint64_t)(kProbeUnroll * 64 * 16);
  const uint64_t left = base < bytes ? bytes - base : 0;
  const rsrc_t r = make_rsrc(p + (base < bytes ? base : 0),
                             (uint32_t)(left < (1u << 30) ? left : (1u << 30)));
  uint4 v[kProbeUnroll];
#pragma unroll
  for (int i = 0; i < kProbeUnroll; ++i)
    v[i] = buf_load16_stream(r, (uint32_t)((i * 64 + lane) * 16), 0);
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < kProbeUnroll; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace

hipError_t launch_read_probe(const void* p, size_t bytes, uint32_t* sink, hipStream_t stream) {
  const uint64_t chunk = (uint64_t)kProbeUnroll * 64 * 16;
  const uint64_t waves = (bytes + chunk - 1) / chunk;
  const uint64_t blocks = (waves + 3) / 4;
  if (blocks == 0 || blocks > 0x7fffffffull) return hipErrorInvalidValue;
  read_probe_kernel<<<(unsigned)blocks, 256, 0, stream>>>((const uint8_t*)p, bytes, sink);
  return hipGetLastError();
}

}  // namespace mlq
