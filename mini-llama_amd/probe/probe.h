/* Bench-only measurement library libmlq_probe.so: read probes that bound
 * what one launch of a given load pattern can do on the device. Not part of
 * the product ABI (include/mlq.h); no counterpart in the reference. */
#ifndef MLQ_PROBE_H_
#define MLQ_PROBE_H_

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

enum { MLQ_PROBE_OK = 0, MLQ_PROBE_ERR_ARG = -1, MLQ_PROBE_ERR_SHAPE = -2, MLQ_PROBE_ERR_HIP = -3 };

#ifdef __cplusplus
namespace mlq {
hipError_t launch_read_probe(const void* p, size_t bytes, uint32_t* sink, hipStream_t stream);
hipError_t launch_shared_probe(const void* shared, size_t shared_bytes, const void* own,
                               size_t own_per_wave, int workgroups, uint32_t* sink,
                               hipStream_t stream);
}  // namespace mlq
extern "C" {
#endif

/* One streaming read of `bytes` (a multiple of 16, 16-byte aligned device
 * pointer) in one launch, dwordx4 loads in 8 KiB chunks per wave,
 * non-temporal like the GEMV's weight lines; sink is one device word
 * written only by chance. Timing it at the byte count of a Linear gives the
 * HBM read ceiling of a single launch of that size (launch ramp and drain
 * included). */
int mlq_probe_read(const void* p, size_t bytes, uint32_t* sink, hipStream_t stream);

/* The skinny GEMM's loads without its arithmetic. `workgroups` workgroups
 * of 8 waves; every workgroup reads all of `shared` (shared_bytes: 0, 64,
 * 128 or 256 KiB; wave w its 1/8 slice in 1 KiB loads) and each wave its
 * own own_per_wave bytes (a multiple of 16, at most 8 KiB; not both sizes 0)
 * at own + (workgroup * 8 + wave) * own_per_wave, which must lie within
 * own_bytes; every load is issued before any is used. 16-byte aligned device
 * pointers; MLQ_PROBE_ERR_SHAPE for any other size. */
int mlq_probe_read_shared(const void* shared, size_t shared_bytes, const void* own,
                          size_t own_bytes, size_t own_per_wave, int workgroups,
                          uint32_t* sink, hipStream_t stream);

#ifdef __cplusplus
}  // extern "C"
#endif

#endif  /* MLQ_PROBE_H_ */
