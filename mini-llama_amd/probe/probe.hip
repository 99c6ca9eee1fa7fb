// Bench-only measurement library (libmlq_probe.so, not part of libmlq.so's
// C ABI): a streaming-read probe, the time a plain read of `bytes` from HBM
// takes in one launch (the ceiling that the GEMV rooflines are compared
// against), and a shared-read probe for the skinny GEMM's load pattern.
// Neither has a counterpart in the reference; bench.py and the probe tests
// are the only callers.
// Each wave reads whole contiguous 8 KiB chunks (dwordx4, non-temporal like
// the GEMV's weight lines), the grid sized to the chunk count; the data are
// folded into one word so the loads cannot be removed, and the word is
// stored only when it equals a value no input produces in practice.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "kernels/device_common.h"
#include "probe.h"

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

// Shared-read probe (the skinny GEMM's access pattern without its math):
// every workgroup's 8 waves read the SAME region (wave w its 1/8 slice,
// NS contiguous 1 KiB loads), plus a distinct range of `own` per wave (NO
// 1 KiB loads; the range check zeroes the tail past own_per_wave); every
// load is issued before any is used.
template <int NS, int NO>
__global__ __launch_bounds__(512) void shared_probe_kernel(const uint8_t* shared,
                                                           const uint8_t* own,
                                                           uint32_t own_per_wave,
                                                           uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t acc = 0;
  if constexpr (NO > 0) {
    const rsrc_t ro =
        make_rsrc(own + ((size_t)blockIdx.x * 8 + wave) * own_per_wave, own_per_wave);
    uint4 o[NO];
#pragma unroll
    for (int i = 0; i < NO; ++i) o[i] = buf_load16_stream(ro, (uint32_t)((i * 64 + lane) * 16), 0);
    if constexpr (NS > 0) {
      const rsrc_t rs = make_rsrc(shared + (size_t)wave * NS * 1024, NS * 1024);
      uint4 v[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i) v[i] = buf_load16(rs, (uint32_t)((i * 64 + lane) * 16), 0);
#pragma unroll
      for (int i = 0; i < NS; ++i) acc ^= v[i].x ^ v[i].w;
    }
#pragma unroll
    for (int i = 0; i < NO; ++i) acc ^= o[i].x ^ o[i].w;
  } else {
    const rsrc_t rs = make_rsrc(shared + (size_t)wave * NS * 1024, NS * 1024);
    uint4 v[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) v[i] = buf_load16(rs, (uint32_t)((i * 64 + lane) * 16), 0);
#pragma unroll
    for (int i = 0; i < NS; ++i) acc ^= v[i].x ^ v[i].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

template <int NS>
hipError_t launch_shared_ns(const void* shared, const void* own, size_t own_per_wave,
                            int workgroups, uint32_t* sink, hipStream_t stream) {
  const int no = (int)((own_per_wave + 1023) / 1024);
  const auto* sh = (const uint8_t*)shared;
  const auto* ow = (const uint8_t*)own;
  const uint32_t opw = (uint32_t)own_per_wave;
  switch (no) {
#define MLQ_PROBE_NO(N)                                                            \
  case N:                                                                          \
    if constexpr (NS > 0 || N > 0)                                                 \
      shared_probe_kernel<NS, N><<<workgroups, 512, 0, stream>>>(sh, ow, opw, sink); \
    break;
    MLQ_PROBE_NO(0) MLQ_PROBE_NO(1) MLQ_PROBE_NO(2) MLQ_PROBE_NO(3) MLQ_PROBE_NO(4)
    MLQ_PROBE_NO(5) MLQ_PROBE_NO(6) MLQ_PROBE_NO(7) MLQ_PROBE_NO(8)
#undef MLQ_PROBE_NO
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_shared_probe(const void* shared, size_t shared_bytes, const void* own,
                               size_t own_per_wave, int workgroups, uint32_t* sink,
                               hipStream_t stream) {
  if (workgroups <= 0 || own_per_wave > 8 * 1024 || (shared_bytes == 0 && own_per_wave == 0))
    return hipErrorInvalidValue;
  switch (shared_bytes) {
    case 0: return launch_shared_ns<0>(shared, own, own_per_wave, workgroups, sink, stream);
    case 64 * 1024: return launch_shared_ns<8>(shared, own, own_per_wave, workgroups, sink, stream);
    case 128 * 1024:
      return launch_shared_ns<16>(shared, own, own_per_wave, workgroups, sink, stream);
    case 256 * 1024:
      return launch_shared_ns<32>(shared, own, own_per_wave, workgroups, sink, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_read_probe(const void* p, size_t bytes, uint32_t* sink, hipStream_t stream) {
  const uint64_t chunk = (uint64_t)kProbeUnroll * 64 * 16;
  const uint64_t waves = (bytes + chunk - 1) / chunk;
  const uint64_t blocks = (waves + 3) / 4;
  if (blocks == 0 || blocks > 0x7fffffffull) return hipErrorInvalidValue;
  read_probe_kernel<<<(unsigned)blocks, 256, 0, stream>>>((const uint8_t*)p, bytes, sink);
  return hipGetLastError();
}

}  // namespace mlq

extern "C" {

int mlq_probe_read(const void* p, size_t bytes, uint32_t* sink, hipStream_t stream) {
  if (p == nullptr || sink == nullptr) return MLQ_PROBE_ERR_ARG;
  if (bytes == 0 || bytes % 16 != 0 || ((uintptr_t)p & 15) != 0) return MLQ_PROBE_ERR_SHAPE;
  return mlq::launch_read_probe(p, bytes, sink, stream) == hipSuccess ? MLQ_PROBE_OK
                                                                        : MLQ_PROBE_ERR_HIP;
}

int mlq_probe_read_shared(const void* shared, size_t shared_bytes, const void* own,
                          size_t own_bytes, size_t own_per_wave, int workgroups,
                          uint32_t* sink, hipStream_t stream) {
  if (shared == nullptr || own == nullptr || sink == nullptr) return MLQ_PROBE_ERR_ARG;
  const bool shared_ok = shared_bytes == 0 || shared_bytes == (size_t)64 * 1024 ||
                         shared_bytes == (size_t)128 * 1024 ||
                         shared_bytes == (size_t)256 * 1024;
  if (workgroups <= 0 || !shared_ok || own_per_wave % 16 != 0 || own_per_wave > 8 * 1024 ||
      (shared_bytes == 0 && own_per_wave == 0) || ((uintptr_t)shared & 15) != 0 ||
      ((uintptr_t)own & 15) != 0)
    return MLQ_PROBE_ERR_SHAPE;
  // every wave reads own_per_wave bytes at own + (workgroup * 8 + wave) *
  // own_per_wave: the caller's buffer must hold all of them
  if ((size_t)workgroups * 8 * own_per_wave > own_bytes) return MLQ_PROBE_ERR_SHAPE;
  return mlq::launch_shared_probe(shared, shared_bytes, own, own_per_wave, workgroups, sink,
                                  stream) == hipSuccess
             ? MLQ_PROBE_OK
             : MLQ_PROBE_ERR_HIP;
}

}  // extern "C"
