/*
 * mlq — MI355X (gfx950) block-quantized Linear for mini-llama: the C ABI.
 *
 * Plain C entry points (no C++ or torch types) over hand-written HIP kernels.
 * They replace the launch layer and kernels of the reference's CUDA quantized
 * Linear (src/cuda_quant.cu:78-517, include/mini_llama/cuda_quant.h:13-76)
 * and the raw upload of src/cuda_weight_upload.cc:111-290. The C++ mirror of
 * the reference interface (hipQ80Linear, ... in mini_llama/hip_quant.h) is
 * written on top of these.
 *
 * Conventions
 *  - Every entry point returns an mlq_status (0 = success) and never throws.
 *  - Work is stream-ordered on the given stream (NULL = the null stream);
 *    nothing here synchronizes unless the name says so.
 *  - Device pointers are borrowed: the caller owns every buffer.
 *  - Shapes follow the reference: W is [n = out_features, k = in_features]
 *    stored as rows of ceil(k/32) GGUF blocks (q8_0 34 B, q4_0 18 B,
 *    q4_1 20 B; include/mini_llama/quantized_tensor.h:36-72); x is [m, k]
 *    fp32 row-major, y is [m, n] fp32 row-major. k need not be a multiple of
 *    32 (the last block of a row is partial, as in src/quant.cc:463-464).
 */
#ifndef MLQ_H_
#define MLQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same handle type as HIP's hipStream_t. */
struct ihipStream_t;
typedef struct ihipStream_t* mlq_stream_t;

/* Numeric values follow QuantType's enumerator order
 * (include/mini_llama/quantized_tensor.h:23-28). */
enum mlq_type { MLQ_F32 = 0, MLQ_Q8_0 = 1, MLQ_Q4_0 = 2, MLQ_Q4_1 = 3 };

enum mlq_status {
  MLQ_OK = 0,
  MLQ_ERR_INVALID_ARG = -1,      /* null pointer, unknown type, bad flag   */
  MLQ_ERR_SHAPE = -2,            /* non-positive dims, in_features mismatch */
  MLQ_ERR_BLOCK_COUNT = -3,      /* block_count != n * ceil(k/32)          */
  MLQ_ERR_BUFFER_TOO_SMALL = -4, /* destination/workspace smaller than needed */
  MLQ_ERR_UNSUPPORTED = -5,      /* shape outside what the kernels accept  */
  MLQ_ERR_NO_DEVICE = -6,        /* no usable HIP device                   */
  MLQ_ERR_FORMAT = -7,           /* malformed GGUF file, see mlq_gguf_last_error */
  MLQ_ERR_SCRATCH_LIMIT = -8,    /* needs more than the fixed no-alloc scratch */
  MLQ_ERR_HIP = -100             /* HIP runtime error, see mlq_last_hip_error */
};

/* Layout of a repacked ("tiled") weight held in one device allocation.
 * Rows are grouped in tiles of 16, blocks in groups of 4 (128 k). A (tile,
 * group) unit is one 64-lane wave line: lane L = n + 16*kq holds quarter kq
 * (elements 8kq..8kq+7) of each of the 4 blocks of row n, i.e. the B operand
 * of one v_mfma_f32_16x16x32_f16 per block. With G = ceil(ceil(k/32)/4):
 *   q4_0/q4_1 quants: 16 B per lane at qs_off + ((t*G+g)*64 + L)*16; word j
 *                     = block 4g+j; element 8kq+i at nibble i/2 + 4*(i%2)
 *   q8_0 quants:      32 B per lane as two 16 B lines (h = 0, 1) at
 *                     qs_off + (((t*G+g)*2+h)*64 + L)*16; words 2u, 2u+1 =
 *                     block 4g+2h+u; codes stored as q+128; element 4w+i at
 *                     byte i/2 + 2*(i%2)
 *   scales d (fp16):  d_off + 2*(((t*G+g)*16 + n)*4 + j) for block 4g+j
 *   mins m (q4_1):    same indexing from m_off
 * Padding rows/blocks decode to 0. Sizes come from mlq_weight_layout. */
typedef struct mlq_weight {
  void* base;      /* device (or host) allocation holding every region */
  int32_t type;    /* enum mlq_type (Q8_0, Q4_0, Q4_1)                 */
  int32_t n;       /* out_features                                      */
  int32_t k;       /* in_features                                       */
  int32_t nb;      /* blocks per row = ceil(k/32)                       */
  uint64_t qs_off; /* byte offset of the quant region                   */
  uint64_t d_off;  /* byte offset of the fp16 scale region              */
  uint64_t m_off;  /* byte offset of the fp16 min region (q4_1), else 0 */
  uint64_t bytes;  /* total bytes of the allocation                     */
} mlq_weight;

/* ---------------------------------------------------------------------- */
/* Library / device                                                        */
/* ---------------------------------------------------------------------- */

/* Human-readable text for an mlq_status. */
const char* mlq_status_string(int status);
/* hipError_t of the last MLQ_ERR_HIP returned on this thread (0 if none). */
int mlq_last_hip_error(void);
/* Number of visible HIP devices (0 and MLQ_ERR_NO_DEVICE when none).
 * Replaces cudaDeviceCount (include/mini_llama/cuda_runtime.h:29). */
int mlq_device_count(int* count);
/* GGUF block size in bytes for a quant type (34/18/20), 0 for others.
 * Matches sizeof(BlockQ80/Q40/Q41) (quantized_tensor.h:41-72). */
size_t mlq_block_bytes(int type);

/* ---------------------------------------------------------------------- */
/* Weight upload: GGUF AoS blocks -> tiled layout                          */
/* (replaces the raw AoS copy of src/cuda_weight_upload.cc:111-290)        */
/* ---------------------------------------------------------------------- */

/* Fill *out with the region offsets and total size of the tiled layout for
 * an [n, k] weight of `type` (out->base is set to NULL). */
int mlq_weight_layout(int type, int n, int k, mlq_weight* out);

/* Host-side repack: `aos` holds n*ceil(k/32) GGUF blocks in host memory,
 * `dst` (host, dst_bytes >= layout bytes) receives the tiled layout.
 * Validates block_count like uploadQ*LinearWeight
 * (src/cuda_weight_upload.cc:118-139). */
int mlq_repack_host(int type, const void* aos, size_t block_count, int n, int k,
                    void* dst, size_t dst_bytes);

/* Device-side repack of AoS blocks already in device memory into `dst`
 * (device). Stream-ordered. */
int mlq_repack_device(int type, const void* aos_dev, size_t block_count, int n,
                      int k, void* dst_dev, size_t dst_bytes,
                      mlq_stream_t stream);

/* Dequantize rows [row0, row0+rows) of a tiled weight into fp32 out
 * [rows, k] (device). Element values are exactly d*q (q8_0), d*(q-8)
 * (q4_0), d*q+m (q4_1) as fp32, i.e. dequantizeFromQ* (src/quant.cc:192-392).
 * Used to prove bit-exact dequantization. */
int mlq_dequantize(const mlq_weight* w, int row0, int rows, float* out,
                   mlq_stream_t stream);

/* Quantize fp32 activations x [rows, row_size] (device, row-major) into
 * q8_0 blocks out [rows][ceil(row_size/32)] (device, 34 B each, GGUF AoS):
 * quantizeToQ80 (src/quant.cc:130-190) bit for bit on the GPU. Per block
 * d = fp16(max|x| / 127) with the reference's fp16 rounding (first dropped
 * bit rounds up, src/quant.cc:32-70), q = clamp(round(x / d), +-127) with
 * round half away from zero, the partial last block zero padded, d = 0 and
 * q = 0 when max|x| is 0. Elements with no integer quotient (NaN, or inf
 * under an infinite scale; undefined in the reference) store -127, the x86
 * conversion the reference compiles to. MLQ_ERR_BUFFER_TOO_SMALL when
 * out_bytes < rows * ceil(row_size/32) * 34. Stream-ordered. */
int mlq_quantize_act_q8_0(const float* x, int rows, int row_size, void* out,
                          size_t out_bytes, mlq_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Quantized Linear: y[m, n] = sum_k W[n, k] * x[m, k]                      */
/* ---------------------------------------------------------------------- */

/* Tiled weight (from the upload path). Picks the kernel family by m:
 *  m = 1..8 (decode): HBM-streaming GEMV, fp32-class accuracy. One row:
 *    activations as integers (22 bits below the largest |x| of each K
 *    slice, three fp16 digits), codes fed with their fp16 bias and the
 *    bias removed on the matrix core, every block sum exact; several rows
 *    (and one-row slices of more than 8 groups): codes decoded exactly to
 *    fp16, activations as an fp16 hi+lo pair (two MFMA rows). Each block's
 *    sum is scaled by its fp16 scale in fp32.
 *  m > 8 (prefill / batched): MFMA f16 GEMM on d*q pre-scaled to fp16 and
 *    fp16-rounded activations, fp32 accumulation (~1e-4 relative).
 * Replaces q80/q40/q41LinearKernel + their launchers
 * (src/cuda_quant.cu:78-182, 300-361, 378-439, 456-517). */
int mlq_linear(const mlq_weight* w, const float* x, float* y, int m,
               mlq_stream_t stream);

/* Device workspace bytes mlq_linear_ws needs for m activation rows with
 * weight w (*bytes = 0 when the kernels for that shape need none: the decode
 * GEMV, and 9..16 rows with k <= 6144, k % 4 == 0, whose skinny kernel reads
 * fp32 x itself). The skinny (17..64 rows, or longer rows) and prefill
 * GEMMs use it for a one-pass fp16 copy of x, which halves the activation
 * bytes their stages move; both also for fp32 partial outputs when they
 * split K across workgroups (shapes with few output tiles). The size
 * depends on the shape, the split-K overrides and the device's
 * compute-unit count. */
int mlq_linear_workspace(const mlq_weight* w, int m, size_t* bytes);

/* mlq_linear with a caller workspace of at least mlq_linear_workspace(w, m)
 * bytes (device memory, 256-byte aligned; contents need no initialisation
 * and are scratch for the duration of the call; may be NULL when that size
 * is 0). MLQ_ERR_BUFFER_TOO_SMALL when it is smaller. Calls that share one workspace must be ordered (same
 * stream), like any other buffer. Same result contract as mlq_linear (fp16
 * rounding of x happens in both prefill variants). No counterpart in the
 * reference (its kernels take fp32 x directly, src/cuda_quant.cu:78-182). */
int mlq_linear_ws(const mlq_weight* w, const float* x, float* y, int m,
                  void* workspace, size_t workspace_bytes, mlq_stream_t stream);

/* Int8 variant for q8_0 weights (MLQ_ERR_UNSUPPORTED otherwise): x is first
 * quantized to q8_0 by quantizeToQ80's rules (src/quant.cc:130-190, as
 * mlq_quantize_act_q8_0) into the workspace, then
 * y[m, n] = sum_b dx[m,b] * dw[n,b] * sum_{k in b} qx[m,k] * qw[n,k] runs on
 * int8 MFMA with an fp32 per-block scale fixup. The reference multiplies
 * fp32 x (src/quant.cc:505-628, src/cuda_quant.cu:78-128); this variant adds
 * the activation quantization error (at most d/2 = max|x in block| / 254
 * per element), which grows like sqrt(k) against the tolerance's k: it
 * meets the Linear's tolerance on N(0,1)-like rows from k ~ 1000 on. Range:
 * a 32-element block of x whose largest |x| reaches 127 * 65520 gets an
 * infinite fp16 scale and all-zero codes under quantizeToQ80's rules, and
 * every output of that row is then NaN (inf * 0), as the product with the
 * dequantized q8_0 block is; below that every finite x works (mlq_linear,
 * the fp16 path, has no such limit). Any m >= 1. Workspace: device,
 * 256-byte aligned
 * (else MLQ_ERR_INVALID_ARG), at least mlq_linear_q8act_workspace(w, m)
 * bytes (not NULL). No counterpart in the reference (no int8 kernel exists
 * there). */
int mlq_linear_q8act_workspace(const mlq_weight* w, int m, size_t* bytes);
int mlq_linear_q8act(const mlq_weight* w, const float* x, float* y, int m,
                     void* workspace, size_t workspace_bytes, mlq_stream_t stream);

/* Output epilogues of mlq_linear_epi. */
enum mlq_epilogue { MLQ_EPI_NONE = 0, MLQ_EPI_SWIGLU = 1 };

/* mlq_linear_ws with a fused output epilogue (no counterpart in the
 * reference, which runs the bias add and SwiGLU as separate ops:
 * src/forward.cc:383-416 bias, 361-370 silu(gate) * up). bias[n] (device,
 * may be NULL) is added to every output row. MLQ_EPI_SWIGLU: w is a gate
 * and an up projection of `ffn` = n/2 rows each, interleaved with
 * mlq_interleave_rows (n % 16 == 0, else MLQ_ERR_SHAPE; bias interleaved
 * the same way); y is [m][n/2] with y[r][i] = silu(gate_i + bias) *
 * (up_i + bias), silu(g) = g / (1 + exp(-g)) in fp32. Workspace and
 * result contract as mlq_linear_ws (the decode GEMV, m <= 8, needs none). */
int mlq_linear_epi(const mlq_weight* w, const float* x, float* y, int m,
                   const float* bias, int act, void* workspace,
                   size_t workspace_bytes, mlq_stream_t stream);

/* Host helper for MLQ_EPI_SWIGLU weights: interleave `rows` rows of a gate
 * and an up matrix (any row format of row_bytes bytes: GGUF block rows
 * before repacking, or fp32 bias entries) into out (2 * rows rows): rows
 * 16t..16t+7 of out are gate rows 8t..8t+7, rows 16t+8..16t+15 up rows
 * 8t..8t+7. rows % 8 == 0, else MLQ_ERR_SHAPE. No counterpart in the
 * reference (it keeps ffn_gate and ffn_up as separate tensors). */
int mlq_interleave_rows(const void* gate, const void* up, int rows,
                        size_t row_bytes, void* out);

/* ---- GGUF (v3) weight files ------------------------------------------
 * Replaces the reference's GgufReader::load / readGgufTensorRaw
 * (include/mini_llama/gguf.h:69-96, src/gguf.cc:398-662) for the Linear
 * weights: the file is memory-mapped and validated with the same rules
 * (magic, version 3, entry/string/array limits, unique keys and names,
 * 1..8 non-zero dims, general.alignment a power of two <= 1 MiB, quantized
 * element counts a multiple of 32, data inside the file). */
typedef struct mlq_gguf mlq_gguf;  /* an open, mapped file */
typedef struct {
  const char* name;    /* valid while the file is open */
  uint32_t ggml_type;  /* 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 8 Q8_0, other ids as stored */
  uint32_t n_dims;
  uint64_t dims[8];    /* GGUF order: dims[0] innermost (k of an [n][k] matrix) */
  uint64_t offset;     /* absolute file offset of the tensor data */
  uint64_t bytes;      /* data size; 0 for types without a known size */
} mlq_gguf_tensor;

/* Open and validate; MLQ_ERR_FORMAT with a message in mlq_gguf_last_error
 * (this thread) when the file is not an acceptable GGUF v3 file. */
int mlq_gguf_open(const char* path, mlq_gguf** out);
const char* mlq_gguf_last_error(void);
void mlq_gguf_close(mlq_gguf* g);
int mlq_gguf_tensor_count(const mlq_gguf* g, int64_t* count);
/* Absolute offset of the data section and the alignment in force. */
int mlq_gguf_data_offset(const mlq_gguf* g, uint64_t* offset, uint64_t* alignment);
int mlq_gguf_tensor_info(const mlq_gguf* g, int64_t index, mlq_gguf_tensor* out);
/* Index of a tensor by name (MLQ_ERR_SHAPE and -1 when absent). */
int mlq_gguf_find(const mlq_gguf* g, const char* name, int64_t* index);
/* The tensor's bytes inside the mapping (NULL for unsized types). */
const void* mlq_gguf_data(const mlq_gguf* g, int64_t index);
/* Upload a 2-D Q8_0 / Q4_0 / Q4_1 tensor (dims [k, n]) into the tiled
 * weight w (layout of mlq_weight_layout(type, n, k), w->base on the
 * device): one copy from the mapping into aos_dev (device scratch of at
 * least the tensor's bytes) and the device repack, stream-ordered. No
 * host-side block vector is built (the reference loader holds one per
 * tensor, src/gguf_loader.cc:396-411). MLQ_ERR_UNSUPPORTED for other
 * types, MLQ_ERR_SHAPE when w does not match the tensor. */
int mlq_gguf_upload(const mlq_gguf* g, int64_t index, void* aos_dev, size_t aos_bytes,
                    mlq_weight* w, mlq_stream_t stream);

/* Raw GGUF AoS blocks in device memory: the meaning of the `const void*`
 * weight of cudaQ*LinearDeviceWeight / cudaQ*LinearDeviceInput
 * (src/cuda_quant.cu:300-361). Up to 8 rows of x whose k fits the kernel's
 * LDS staging (mlq_linear_aos_workspace reports 0 bytes) run a GEMV that
 * reads the blocks as they are, every weight byte once; `workspace` may
 * then be NULL. Otherwise the blocks are repacked into `workspace` (device,
 * >= mlq_weight_layout(...).bytes) and run through mlq_linear. Results
 * meet the Linear's tolerance either way (the direct GEMV sums in fp32
 * like the reference's per-element loop, in another order). */
int mlq_linear_aos(int type, const void* aos_dev, size_t block_count, int n,
                   int k, const float* x, float* y, int m, void* workspace,
                   size_t workspace_bytes, mlq_stream_t stream);

/* Workspace bytes mlq_linear_aos needs for m rows: 0 when the direct GEMV
 * takes the shape, the tiled layout's bytes otherwise. No counterpart in
 * the reference. */
int mlq_linear_aos_workspace(int type, int n, int k, int m, size_t* bytes);

/* Kernel-family overrides for tests and measurement: force the GEMV
 * (requires m <= 8 and k within its LDS budget, else MLQ_ERR_UNSUPPORTED)
 * or the GEMM regardless of m. */
enum mlq_path { MLQ_PATH_AUTO = 0, MLQ_PATH_GEMV = 1, MLQ_PATH_MFMA = 2 };
int mlq_linear_path(const mlq_weight* w, const float* x, float* y, int m,
                    int path, mlq_stream_t stream);

/* GEMV work decomposition override for tuning and tests (process-wide):
 * split = waves (K slices) per 16-row tile: 1, 2, 4, 8 or 16; 0 restores
 * the automatic choice. The planner still widens the split when the
 * activation staging would not fit in LDS. How many groups a wave keeps in
 * flight follows from the slice length. Returns MLQ_ERR_INVALID_ARG for
 * other values. */
int mlq_set_gemv_split(int split);

/* Prefill GEMM split-K override for tuning and tests (process-wide): the
 * K range of every output tile is divided over `split` workgroups (capped
 * at one 128-k group each) whose fp32 partials are summed in split order;
 * 0 restores the planner. Applies to mlq_linear_ws calls that take the
 * prefill GEMM (m > 64); query mlq_linear_workspace after changing it.
 * MLQ_ERR_INVALID_ARG outside 0..64. */
int mlq_set_gemm_split(int split);

/* Skinny GEMM (9..64 rows) plan override for tuning and tests
 * (process-wide): `tiles` weight tiles of 16 rows per workgroup (1, 2 or 4)
 * and `splits` K ranges per tile group (1..8; ranges beyond the number of
 * 128-k groups are capped), whose fp32 partial slices a second kernel sums
 * in range order; 0 leaves that choice to the planner. Query
 * mlq_linear_workspace after changing it. MLQ_ERR_INVALID_ARG otherwise. */
int mlq_set_skinny_plan(int tiles, int splits);

/* mlq_linear_epi that allocates nothing and takes no workspace: no
 * counterpart in the reference. For callers that cannot call hipMalloc
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). The scratch that mlq_linear_epi keeps in the caller's
 * workspace (fp16 copy of x, split-K partial slices) comes from a fixed
 * array of MLQ_NOALLOC_SCRATCH_BYTES in the library's device code, one per
 * GPU, held until the process ends. Shapes whose mlq_linear_workspace
 * exceeds that size return MLQ_ERR_SCRATCH_LIMIT (the decode GEMV and F32
 * weights need none). Same kernels and bit-identical results as
 * mlq_linear_epi. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, or host threads) race and must be
 * ordered by the caller. The device is the stream's (the current device for
 * the null stream). */
#define MLQ_NOALLOC_SCRATCH_BYTES (64u << 20)
int mlq_linear_epi_noalloc(const mlq_weight* w, const float* x, float* y, int m,
                           const float* bias, int act, mlq_stream_t stream);

/* Add bias[n] to every row of y[m, n] on the device (the reference adds the
 * bias on the host after download, src/cuda_quant.cu:229-235, 327-329). */
int mlq_add_bias(float* y, const float* bias, int m, int n,
                 mlq_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Decode-step operators (fp32 activations, device pointers)              */
/* ---------------------------------------------------------------------- */
/* F32 Linear weights use mlq_weight with type MLQ_F32: base holds W [n][k]
 * fp32 row-major (mlq_weight_layout(MLQ_F32, n, k) gives bytes = 4nk, every
 * offset 0). mlq_linear, mlq_linear_ws and mlq_linear_epi then run an fp32
 * HBM-streaming GEMV (any m, no workspace, same epilogues), replacing the
 * cuBLAS Sgemm of cudaLinearDeviceInput (src/cuda_matmul.cc:205-241) and the
 * F32 arm of forwardLinearDevice (src/forward.cc:206-209). The GEMM path
 * override (MLQ_PATH_MFMA) is MLQ_ERR_UNSUPPORTED for them. */

/* RopeType enumerator order (include/mini_llama/model.h:17-20). */
enum mlq_rope_type { MLQ_ROPE_NORMAL = 0, MLQ_ROPE_NEOX = 1 };

/* y[r] = x[r] * weight / sqrt(mean(x[r]^2) + eps) for rows r of [rows, dim]
 * (rmsNorm, src/ops.cc:43-72; cudaRmsNormDeviceWeight,
 * include/mini_llama/cuda_ops.h:40). eps must be finite and positive
 * (MLQ_ERR_INVALID_ARG otherwise, as src/cuda_ops.cu:99-101). */
int mlq_rmsnorm(const float* x, const float* weight, float* y, int rows, int dim,
                float eps, mlq_stream_t stream);
/* Elementwise over n floats: a + b (cudaElementwiseAddDeviceInput,
 * cuda_ops.h:57), a * b (cudaElementwiseMulDeviceInput, :52), silu(x) =
 * x / (1 + exp(-x)) (cudaSiluDeviceInput, :49), silu(gate) * up in one pass
 * (forwardSwiGluDevice, src/forward.cc:361-370). */
int mlq_add(const float* a, const float* b, float* y, int64_t n, mlq_stream_t stream);
int mlq_mul(const float* a, const float* b, float* y, int64_t n, mlq_stream_t stream);
int mlq_silu(const float* x, float* y, int64_t n, mlq_stream_t stream);
int mlq_swiglu(const float* gate, const float* up, float* y, int64_t n, mlq_stream_t stream);
/* y[n] = exp(x - max(x)) / sum(exp(x - max(x))) over one vector (softmax,
 * src/ops.cc:74-109; cudaSoftmax, include/mini_llama/cuda_ops.h:68). x and
 * y may alias. */
int mlq_softmax(const float* x, float* y, int64_t n, mlq_stream_t stream);
/* y[dim] = table[token] of an fp32 [vocab, dim] table
 * (cudaEmbeddingLookupDeviceWeight, cuda_ops.h:71); token outside
 * [0, vocab) is MLQ_ERR_INVALID_ARG. */
int mlq_embedding(const float* table, int vocab, int dim, int token, float* y,
                  mlq_stream_t stream);
/* In-place RoPE of q [n_heads, head_dim] and k [n_kv_heads, head_dim] at
 * position pos (rope, src/ops.cc:142-218; cudaRopeDeviceInput,
 * cuda_ops.h:81): pair i rotates by pos * theta^(-2i/head_dim), pairs
 * (2i, 2i+1) for MLQ_ROPE_NORMAL, (i, i + head_dim/2) for MLQ_ROPE_NEOX.
 * head_dim must be positive and even (MLQ_ERR_SHAPE); pos < 0 or theta not
 * finite and positive is MLQ_ERR_INVALID_ARG. */
int mlq_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos,
             float theta, int rope_type, mlq_stream_t stream);

/* A KV cache: keys and values each [n_layers][max_seq_len][n_kv_heads]
 * [head_dim] fp32 on the device, the layout of CudaKvCache
 * (include/mini_llama/cuda_kv_cache.h:28-80, src/cuda_kv_cache.cc). */
typedef struct mlq_kv_cache {
  float* keys;
  float* values;
  int32_t n_layers, max_seq_len, n_kv_heads, head_dim;
} mlq_kv_cache;
/* Bytes of each of the two arrays. */
int mlq_kv_cache_bytes(int n_layers, int max_seq_len, int n_kv_heads, int head_dim,
                       size_t* bytes);
/* Store k and v [n_kv_heads * head_dim] at (layer, pos)
 * (CudaKvCache::writeDevice, cuda_kv_cache.h:53). */
int mlq_kv_write(const mlq_kv_cache* c, int layer, int pos, const float* k, const float* v,
                 mlq_stream_t stream);
/* Workspace of mlq_attention_decode for any pos of this cache. */
int mlq_attention_workspace(const mlq_kv_cache* c, int n_heads, size_t* bytes);
/* out [n_heads, head_dim] = softmax(q . K^T / sqrt(head_dim)) . V over
 * cache positions 0..pos of `layer`, query head h reading kv head
 * h / (n_heads / n_kv_heads) (cudaAttentionDecodeDeviceInput,
 * include/mini_llama/cuda_attention.h:22; src/forward.cc:526-565).
 * Checks of validateAttentionDeviceInputs; n_heads / n_kv_heads > 16 or
 * head_dim > 256 is MLQ_ERR_UNSUPPORTED. ws: mlq_attention_workspace bytes
 * (scratch, no initialisation). */
int mlq_attention_decode(const mlq_kv_cache* c, int layer, int pos, const float* q,
                         int n_heads, float* out, void* ws, size_t ws_bytes,
                         mlq_stream_t stream);
/* *out (device int32) = index of the first maximum of x[n]; NaN never wins
 * and x[0] = NaN gives 0 (argMax, src/ops.cc:230-246). */
int mlq_argmax(const float* x, int64_t n, int32_t* out, mlq_stream_t stream);

/* ---- the decode step: one token through the whole model --------------
 * Weights as uploaded Linear weights (any of F32 / Q8_0 / Q4_0 / Q4_1 per
 * projection) and fp32 norms, biases and embedding table, all on the
 * device. Layer fusions chosen at upload time:
 *  - wk.base == NULL and wv.base == NULL: wq holds the q|k|v rows
 *    concatenated ([(n_heads + 2 n_kv_heads) head_dim, dim]) and bq, if
 *    any, the concatenated bias;
 *  - w_up.base == NULL: w_gate holds gate and up interleaved by
 *    mlq_interleave_rows ([2 hidden_dim, dim]) and runs with the SwiGLU
 *    epilogue. */
typedef struct mlq_layer {
  const float* attn_norm;            /* [dim] */
  mlq_weight wq, wk, wv;             /* see above */
  const float* bq;                   /* optional biases (Qwen2), NULL if none */
  const float* bk;
  const float* bv;
  mlq_weight wo;                     /* [dim, n_heads head_dim] */
  const float* ffn_norm;             /* [dim] */
  mlq_weight w_gate, w_up;           /* [hidden_dim, dim] each, or fused */
  mlq_weight w_down;                 /* [dim, hidden_dim] */
} mlq_layer;

/* ModelConfig (include/mini_llama/model.h:22-34) plus the weights of
 * MiniLlamaModel the forward pass reads. */
typedef struct mlq_model {
  int32_t vocab_size, dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim,
      max_seq_len;
  float rope_theta, rms_norm_eps;
  int32_t rope_type;                 /* enum mlq_rope_type */
  const float* token_embedding;      /* [vocab_size, dim] */
  const float* final_norm;           /* [dim] */
  mlq_weight lm_head;                /* [vocab_size, dim] */
  const mlq_layer* layers;           /* HOST array of n_layers */
} mlq_model;

/* Device workspace bytes of mlq_decode_token (256-byte aligned buffer);
 * also validates every shape of the model. */
int mlq_decode_workspace(const mlq_model* m, size_t* bytes);

/* logits [vocab_size] (device) for `token` at position `pos`, writing the
 * layer's K/V rows at pos into the cache: forwardToken's device branch
 * (src/forward.cc:763-784, forwardLayerDevice :607-640,
 * computeLogitsDevice :736-745) as one stream-ordered sequence of launches.
 * token_dev / pos_dev (device int32, may be NULL) replace token / pos, so a
 * captured HIP graph of one call serves every step; a device token or
 * position out of range yields NaN logits instead of a fault. The cache must
 * match the model (layers, kv heads, head_dim, capacity >= max_seq_len). */
int mlq_decode_token(const mlq_model* m, const mlq_kv_cache* c, int token, int pos,
                     const int32_t* token_dev, const int32_t* pos_dev, float* logits,
                     void* ws, size_t ws_bytes, mlq_stream_t stream);

/* Batched prefill: the n_tokens tokens (host array) at positions start_pos
 * .. start_pos + n_tokens - 1 through the model at once, every Linear on
 * [n_tokens, K] activations (the skinny and prefill GEMMs), their K/V rows
 * written to the cache, and logits [vocab_size] (device) of the last token:
 * the result of forwardBatch (src/batch.cc:32-55), which runs forwardToken
 * once per token. Attention is causal (row r sees positions up to
 * start_pos + r). Tokens out of range or start_pos + n_tokens beyond
 * max_seq_len are MLQ_ERR_INVALID_ARG. ws: mlq_prefill_workspace(m,
 * n_tokens) bytes, 256-byte aligned. */
int mlq_prefill_workspace(const mlq_model* m, int n_tokens, size_t* bytes);
int mlq_prefill(const mlq_model* m, const mlq_kv_cache* c, const int32_t* tokens, int n_tokens,
                int start_pos, float* logits, void* ws, size_t ws_bytes, mlq_stream_t stream);

/* Greedy sampling on the device (argMax, src/ops.cc:230-246, as the
 * sampler's temperature-0 choice, MiniSampler::sampleGreedy,
 * src/sampler.cc:109-114): *token_dev = argmax(logits), then *pos_dev += 1,
 * so decode steps can follow each other with no host round trip. Two
 * passes over slices of the logits; ws (device, 8-byte aligned, no
 * initialisation) holds mlq_argmax_workspace(vocab) bytes. */
int mlq_argmax_workspace(int64_t n, size_t* bytes);
int mlq_greedy_next(const float* logits, int vocab, int32_t* token_dev, int32_t* pos_dev,
                    void* ws, size_t ws_bytes, mlq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MLQ_H_ */
