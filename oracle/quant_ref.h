/*
 * CPU ORACLE — test infrastructure only.
 *
 * A plain-C restatement of the reference's CPU block-quantized Linear path
 * (Haobin-Lee/mini-llama). It exists to CHECK the HIP path, never to be it:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product library (mini-llama_amd/) never links or calls it.
 *
 * Every function cites the reference lines it follows (paths relative to the
 * reference repository root).
 *
 * Parity pinning (what checks each function, see tests/test_oracle_*.py):
 *   ref_fp16_to_f32      exhaustive 65,536-pattern comparison with numpy's
 *                        IEEE binary16 decoder (a library routine).
 *   ref_f32_to_fp16      numpy binary16 on every non-tie input (identical to
 *                        round-to-nearest there) + exact-rational tie cases
 *                        (the reference rounds ties away from zero, not to
 *                        even) + overflow/underflow/NaN special cases.
 *   ref_quantize_*       reference test_quant.cc known answers and bounds +
 *                        per-element invariants (|x - d*q| <= d/2, clamp
 *                        range, zero blocks, padding).
 *   ref_dequantize_*     reference known-value vectors (test_quant.cc:231-248)
 *                        + closed form d*q (+m), exact in fp32.
 *   ref_linear_*         reference known answers (test_quant.cc:250-263,
 *                        265-286) + exact-arithmetic cases whose fp32 sum is
 *                        exact (so any dropped term / wrong nibble / swapped
 *                        index fails) + float64 brute force with a rounding
 *                        bound.
 */
#ifndef MLQ_ORACLE_QUANT_REF_H_
#define MLQ_ORACLE_QUANT_REF_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Block layouts: byte-identical to the reference's GGUF-compatible structs
 * (include/mini_llama/quantized_tensor.h:36-72): 34 / 18 / 20 bytes, 2-byte
 * alignment, no padding. */
typedef struct {
  uint16_t d;
  int8_t qs[32];
} ref_block_q8_0;

typedef struct {
  uint16_t d;
  uint8_t qs[16];
} ref_block_q4_0;

typedef struct {
  uint16_t d;
  uint16_t m;
  uint8_t qs[16];
} ref_block_q4_1;

enum { REF_OK = 0, REF_ERR_SHAPE = -1, REF_ERR_BLOCKS = -2 };

/* Which arithmetic the library was built with: 0 = scalar (-O2),
 * 1 = AVX2+FMA (-O2 -mavx2 -mfma; linearQ80 takes the SIMD path). */
int ref_build_flavor(void);

uint16_t ref_f32_to_fp16(float value);
float ref_fp16_to_f32(uint16_t value);

/* Bulk helpers for the tests (elementwise wrappers of the two above). */
void ref_f32_to_fp16_array(const float* src, uint16_t* dst, size_t n);
void ref_fp16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* Quantizers. `n_rows` x `row_size` is the source tensor viewed as rows
 * (the reference uses the last dim as the row for rank >= 2, the whole
 * tensor for rank 1). Returns the number of blocks written. */
size_t ref_quantize_q8_0(const float* src, int n_rows, int row_size,
                         ref_block_q8_0* out);
size_t ref_quantize_q4_0(const float* src, int n_rows, int row_size,
                         ref_block_q4_0* out);

/* Dequantizers: REF_ERR_BLOCKS when n_blocks != n_rows*ceil(row_size/32). */
int ref_dequantize_q8_0(const ref_block_q8_0* blocks, size_t n_blocks,
                        int n_rows, int row_size, float* dst);
int ref_dequantize_q4_0(const ref_block_q4_0* blocks, size_t n_blocks,
                        int n_rows, int row_size, float* dst);
int ref_dequantize_q4_1(const ref_block_q4_1* blocks, size_t n_blocks,
                        int n_rows, int row_size, float* dst);

/* Quantized Linear y[r, n] = sum_k deq(W[n, k]) * x[r, k].
 * x is [rows, in_features] row-major, W is [out_features, w_in_features]
 * blocks, y is [rows, out_features]. n_threads follows the reference
 * ThreadPool partition (0 = hardware concurrency). */
int ref_linear_q8_0(const float* x, int rows, int in_features,
                    const ref_block_q8_0* w, size_t n_blocks, int out_features,
                    int w_in_features, float* y, int n_threads);
int ref_linear_q4_0(const float* x, int rows, int in_features,
                    const ref_block_q4_0* w, size_t n_blocks, int out_features,
                    int w_in_features, float* y, int n_threads);
int ref_linear_q4_1(const float* x, int rows, int in_features,
                    const ref_block_q4_1* w, size_t n_blocks, int out_features,
                    int w_in_features, float* y, int n_threads);

#ifdef __cplusplus
}
#endif

#endif /* MLQ_ORACLE_QUANT_REF_H_ */
