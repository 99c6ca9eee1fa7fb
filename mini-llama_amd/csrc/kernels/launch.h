// Internal launchers (C++ linkage, library-private). The C ABI in capi.cpp
// validates arguments and then calls these; they only configure and launch.
#pragma once

#include <hip/hip_runtime.h>

#include "../mlq_layout.h"

namespace mlq {

// Output epilogue of the Linear kernels: they store act(acc + bias[row]) for
// output row `row` of W.
//  kEpiNone:   y[r][row] = acc + bias[row] (bias optional).
//  kEpiSwiGLU: W holds a gate and an up projection interleaved per 16-row
//              tile (rows 16t..16t+7 are gate rows 8t..8t+7, rows
//              16t+8..16t+15 the matching up rows); y has n/2 columns and
//              y[r][8t + c] = silu(gate + bias) * (up + bias) with
//              silu(g) = g / (1 + exp(-g)) in fp32 (the reference's SiLU and
//              elementwise product, src/forward.cc:361-370).
enum { kEpiNone = 0, kEpiSwiGLU = 1 };
struct Epilogue {
  const float* bias = nullptr;  // [n] or nullptr
  int act = kEpiNone;
  // Input RMSNorm (decode GEMV with one activation row only): with norm
  // non-null the kernel computes W . (x * norm) / sqrt(mean(x^2) + norm_eps)
  // in place of W . x, i.e. the Linear of rmsNorm(x, norm, eps)
  // (src/ops.cc:43-72) without a separate pass over x.
  const float* norm = nullptr;  // [k] or nullptr
  float norm_eps = 0.0f;
  // Pre-scaled input RMSNorm (decode GEMV, one activation row): x already
  // holds x * norm, and the sum of x^2 over the row is the sum of
  // ssq_parts[0 .. ssq_count) (ssq_count <= kSsqPartsMax), added in a fixed
  // order; the kernel divides its outputs by sqrt(sum / k + norm_eps).
  const float* ssq_parts = nullptr;
  int ssq_count = 0;
  // Producer of that input (decode GEMV, one row, no activation): besides
  // y, write y[r] * next_norm[r] to next_x[r] and, per 16-row tile t, the
  // sum of the tile's y^2 to next_ssq[t].
  const float* next_norm = nullptr;
  float* next_x = nullptr;
  float* next_ssq = nullptr;
};
// Most partial sums a pre-scaled RMSNorm input may carry (one float per
// 16 elements: rows up to 4096).
constexpr int kSsqPartsMax = 256;

// Output option of the prefill GEMM reading the fp16 copy of x and of its
// split-K reduce (launch_gemm_f16, launch_gemm_ws with a workspace that
// holds the copy; else hipErrorInvalidValue): residual [m][ny] added to the
// output after the activation (may alias y: each element is read, then
// written, by one thread). Kept out of Epilogue so that the other kernels'
// arguments do not grow.
struct GemmOut {
  const float* residual = nullptr;
};

// capi.cpp: MLQ status of a HIP result, recorded for mlq_last_hip_error.
int record_hip(hipError_t e);

// gemv.hip: lets `kernel` launch with `lds` bytes of dynamic LDS on the
// current device (above the default 64 KiB the kernel's limit is raised to
// the device maximum, once per device and kernel, under a lock: concurrent
// launches from several host threads never race on the update).
hipError_t allow_dynamic_lds(const void* kernel, size_t lds);

// repack.hip
hipError_t launch_repack(int type, const void* aos, int n, int k,
                         const mlq_weight& w, hipStream_t stream);
hipError_t launch_dequant(const mlq_weight& w, int row0, int rows, float* out,
                          hipStream_t stream);
hipError_t launch_bias(float* y, const float* bias, int m, int n,
                       hipStream_t stream);
// rows x k fp32 (row-major) -> rows * ceil(k/32) q8_0 blocks (34 B each,
// row-major) with quantizeToQ80's rules.
hipError_t launch_quantize_act_q8_0(const float* x, int rows, int k, void* out,
                                    hipStream_t stream);

// gemm_i8.hip: q8_0 weights x q8_0-quantized activations on int8 MFMA
// (activation quantize pass + GEMM). Workspace: gemm_i8_workspace_bytes.
size_t gemm_i8_workspace_bytes(const mlq_weight& w, int m);
hipError_t launch_gemm_i8(const mlq_weight& w, const float* x, float* y, int m,
                          void* workspace, hipStream_t stream);

// gemv.hip: m in 1..8 rows of x.
constexpr int kGemvMaxRows = 8;
// Returns hipErrorInvalidValue when the activation staging does not fit LDS.
hipError_t launch_gemv(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream, const Epilogue& epi = Epilogue());
// Largest k the GEMV accepts for m rows (LDS-bound).
int gemv_max_k(int type, int m);
// epi.norm is honoured by the decode GEMV with m == 1 for the weights this
// accepts (launch_gemv returns hipErrorInvalidValue for the others).
bool gemv_norm_supported(const mlq_weight& w);
// The decode GEMV (one row) runs w with a pre-scaled RMSNorm input
// (epi.ssq_parts), resp. as the producer of one (epi.next_x).
bool gemv_prenorm_supported(const mlq_weight& w);
// Split override (0 = automatic); validated by the caller.
void set_gemv_split(int split);

// gemm_mfma.hip: any m >= 1. The _ws form converts x to fp16 into `ws`
// first when ws_bytes >= f16_copy_bytes(m, k) (else reads fp32 x), and
// splits K over gemm_splits(m, n, k) workgroups per output tile when
// ws_bytes >= gemm_workspace_bytes(m, n, k) (fp32 partial slices after the
// fp16 copy, summed in order by a second kernel).
//
// fp16 copies of activations carry one power-of-two exponent per row: row r
// holds x[r] * 2^rexp[r] with rexp[r] = pow2_scale_exp(max |x[r]|), so any
// finite fp32 row fits fp16 without overflow and far above its subnormal
// floor; the GEMMs scale row r's fp32 results by 2^-rexp[r]. Without a copy
// the GEMM finds the exponents of its rows itself before its K loop.
hipError_t launch_gemm(const mlq_weight& w, const float* x, float* y, int m,
                       hipStream_t stream);
hipError_t launch_gemm_ws(const mlq_weight& w, const float* x, float* y, int m,
                          void* ws, size_t ws_bytes, hipStream_t stream,
                          const Epilogue& epi = Epilogue(), const GemmOut& out = GemmOut());
// Bytes of the fp16 copy of x [m][f16_row_stride(k)] plus its row exponents
// (int32 [m] at f16_copy_exps).
size_t f16_copy_bytes(int m, int k);
int* f16_copy_exps(void* copy, int m, int k);
// The GEMM from an fp16 copy of x already in place (xh [m][f16_row_stride(k)],
// zero past k, with its row exponents rexp [m], e.g. written by
// launch_rmsnorm_f16 or launch_x_to_f16); `ws` (gemm_partial_bytes(m, n, k),
// may be null when that is 0) takes the split-K partial slices.
hipError_t launch_gemm_f16(const mlq_weight& w, const _Float16* xh, const int* rexp, float* y,
                           int m, void* ws, size_t ws_bytes, hipStream_t stream,
                           const Epilogue& epi = Epilogue(), const GemmOut& out = GemmOut());
size_t gemm_partial_bytes(int m, int n, int k);
int gemm_splits(int m, int n, int k);
size_t gemm_workspace_bytes(int m, int n, int k);
// Split-K override (0 = planner); validated by the caller.
void set_gemm_split(int split);
// fp16 copy of x [m][k] into xh [m][f16_row_stride(k)] (zero past k), each
// row scaled by 2^rexp[r] (the exponents written to rexp [m]).
int f16_row_stride(int k);
hipError_t launch_x_to_f16(const float* x, _Float16* xh, int* rexp, int m, int k,
                           hipStream_t stream);

// Compute units of the current device (256 on MI355X), read once.
int device_cus();
// y = epilogue(sum over s of part[s] in order), part [splits][m][n] fp32
// (split-K partial slices of the prefill and skinny GEMMs).
hipError_t launch_split_reduce(const float* part, float* y, int m, int n, int splits,
                               const Epilogue& epi, hipStream_t stream,
                               const GemmOut& out = GemmOut());

// skinny.hip: 9..64 rows of x. launch_skinny_ws makes the fragment-ordered
// fp16 copy of x in ws (not for 9..16 rows with k <= 6144, k % 4 == 0:
// that kernel reads fp32 x itself), then runs the skinny GEMM (K split over
// workgroups when the planner chooses it: partial slices after the copy);
// ws holds skinny_workspace_bytes(type, m, n, k) bytes, 256-byte aligned
// (may be null when that is 0).
constexpr int kSkinnyMaxRows = 64;
size_t skinny_x_bytes(int m, int k);
size_t skinny_workspace_bytes(int type, int m, int n, int k);
hipError_t launch_skinny_ws(const mlq_weight& w, const float* x, float* y, int m,
                            void* ws, size_t ws_bytes, hipStream_t stream,
                            const Epilogue& epi = Epilogue());
// Plan override (0 = planner): weight tiles per workgroup (1, 2, 4) and K
// ranges per tile group (1..8); validated by the caller.
void set_skinny_plan(int tiles, int splits);

// aos_gemv.hip: GEMV straight from GGUF AoS blocks (m <= 8 rows of x, x
// staged in LDS: aos_gemv_supported says whether the shape fits).
bool aos_gemv_supported(int type, int m, int n, int k);
hipError_t launch_aos_gemv(int type, const void* aos, int n, int k, const float* x, float* y,
                           int m, hipStream_t stream);

// linear_f32.hip: fp32 W [n][k], any m (passes of up to 8 rows).
hipError_t launch_linear_f32(const float* w, int n, int k, const float* x, float* y, int m,
                             hipStream_t stream, const Epilogue& epi = Epilogue());

// decode_ops.hip: the decode-step operators.
hipError_t launch_rmsnorm(const float* x, const float* w, float* y, int rows, int dim,
                          float eps, hipStream_t stream);
// RMSNorm rows written as fp16 (round to nearest even) into yh [rows][ld],
// zero for dim <= c < ld: the GEMM's fp16 copy of its input in one pass.
// Row r is stored scaled by 2^rexp[r] (pow2_scale_exp of the row's largest
// |y|), the convention of launch_x_to_f16. Needs dim % 4 == 0, ld % 4 == 0
// and 16-byte aligned x, w, yh rows.
hipError_t launch_rmsnorm_f16(const float* x, const float* w, _Float16* yh, int* rexp, int rows,
                              int dim, int ld, float eps, hipStream_t stream);
// bytes (a multiple of 4) of zeros at p (4-byte aligned): a kernel, so it
// may be captured in a graph.
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream);
enum { kEltAdd = 0, kEltMul = 1, kEltSilu = 2, kEltSwiGLU = 3 };
hipError_t launch_eltwise(int op, const float* a, const float* b, float* y, int64_t n,
                          hipStream_t stream);
// softmax of one vector of n floats (one workgroup).
hipError_t launch_softmax(const float* x, float* y, int64_t n, hipStream_t stream);
// token_dev (device int32, may be null) overrides token. With rt.cs
// non-null the launch also writes the step's RoPE table (cos of pair i at
// cs[i], sin at cs[hd/2 + i]) for position pos (pos_dev overrides).
struct RopeTable {
  float* cs = nullptr;
  const int32_t* pos_dev = nullptr;
  int pos = 0, hd = 0;
  float theta = 10000.0f;
};
// With norm non-null it also writes the first layer's pre-scaled RMSNorm
// input (Epilogue::ssq_parts): xn = y * norm and per 16 elements the sum of
// y^2 to parts.
struct NormInput {
  const float* norm = nullptr;
  float* xn = nullptr;
  float* parts = nullptr;
};
hipError_t launch_embedding(const float* table, int vocab, int dim, const int32_t* token_dev,
                            int token, float* y, hipStream_t stream,
                            const RopeTable& rt = RopeTable(),
                            const NormInput& ni = NormInput());
// RoPE on q [n_heads][hd] and k [n_kv][hd] at position pos (pos_dev
// overrides). With keys/values non-null the rotated k and v go to cache row
// (layer, pos) of a [layers][max_seq][n_kv][hd] cache and k is left as is.
struct RopeLaunch {
  float* q = nullptr;
  float* k = nullptr;
  const float* v = nullptr;
  float* keys = nullptr;
  float* values = nullptr;
  int n_heads = 0, n_kv = 0, hd = 0, neox = 0;
  int layer = 0, max_seq = 0;
  // positions at or past pos_limit write no cache row (0: max_seq)
  int pos_limit = 0;
  const int32_t* pos_dev = nullptr;
  int pos = 0;
  float theta = 10000.0f;
};
hipError_t launch_rope(const RopeLaunch& r, hipStream_t stream);
hipError_t launch_kv_write(float* keys, float* values, const float* k, const float* v,
                           size_t row, int n, hipStream_t stream);
// Decode attention of q [n_heads][hd] over cache positions 0..pos of `layer`.
// max_len bounds pos + 1 (grid and workspace size); ws holds
// attention_workspace_bytes(n_heads, hd, max_len) bytes.
struct AttnLaunch {
  const float* q = nullptr;
  const float* keys = nullptr;
  const float* values = nullptr;
  float* out = nullptr;
  float* ws = nullptr;
  int layer = 0, max_seq = 0, n_heads = 0, n_kv = 0, hd = 0;
  int max_len = 0;
  // A position at or past pos_limit (0: no limit beyond the cache capacity
  // and max_len) writes no cache row and gives NaN outputs.
  int pos_limit = 0;
  const int32_t* pos_dev = nullptr;
  int pos = 0;
  // Fused RoPE + cache write of position pos (attention_fusable shapes):
  // q is then the raw projection, k_new / v_new the raw k and v [n_kv][hd],
  // rope_cs the step's table (launch_embedding), and the cache row (layer,
  // pos) is written here. rope_cs == nullptr: q is rotated and the row is
  // in the cache already.
  const float* k_new = nullptr;
  const float* v_new = nullptr;
  const float* rope_cs = nullptr;
  int neox = 0;
  // Several query rows (prefill, rope_cs == nullptr): row r at position
  // pos + r, q row r at q + r * q_stride, output row at out + r * out_stride;
  // ws holds attention_workspace_bytes(n_heads, hd, max_len, rows).
  int rows = 1, q_stride = 0, out_stride = 0;
};
bool attention_supported(int n_heads, int n_kv, int hd);
bool attention_fusable(int hd, int group);
int attention_chunks(int hd, int max_len);
size_t attention_workspace_bytes(int n_heads, int hd, int max_len, int rows = 1);
// Prefill attention on fp32 MFMA: rows query rows at positions pos + r,
// causal, for head_dim 64 / 128 / 256 and 16-byte aligned caches (else
// hipErrorInvalidValue); no workspace.
bool prefill_attention_supported(int hd, int group);
hipError_t launch_attention_prefill(const AttnLaunch& r, hipStream_t stream);
// Prefill helpers: RoPE + cache write of `rows` consecutive positions pos0
// + r (q rotated in place; rotated k and v to the cache), and embedding rows
// for device tokens.
struct RopeRows {
  float* q = nullptr;
  float* k = nullptr;
  const float* v = nullptr;
  int q_stride = 0, k_stride = 0, v_stride = 0, rows = 0;
  float* keys = nullptr;
  float* values = nullptr;
  int n_heads = 0, n_kv = 0, hd = 0, neox = 0, layer = 0, max_seq = 0, pos0 = 0;
  float theta = 10000.0f;
  // optional [rows][hd] table from launch_rope_table for positions pos0 ..
  // pos0 + rows - 1 (the same values the kernel computes otherwise)
  const float* cs = nullptr;
};
hipError_t launch_rope_rows(const RopeRows& rr, hipStream_t stream);
// cs[r][i] = cos, cs[r][hd/2 + i] = sin of (pos0 + r) * theta^(-2i/hd) for
// i < hd/2: the angles of launch_rope_rows, computed once for all layers.
hipError_t launch_rope_table(float* cs, int rows, int pos0, int hd, float theta,
                             hipStream_t stream);
hipError_t launch_embedding_rows(const float* table, int dim, const int32_t* tokens, int rows,
                                 float* y, hipStream_t stream);
hipError_t launch_attention(const AttnLaunch& r, hipStream_t stream);
// out = argmax(x) (first maximum, NaN never wins); pos_dev += 1 when non-null.
// One workgroup, no workspace:
hipError_t launch_argmax(const float* x, int64_t n, int32_t* out, int32_t* pos_dev,
                         hipStream_t stream);
// Two passes over slices of the vector with argmax_workspace_bytes(n) of
// 8-byte-aligned scratch:
size_t argmax_workspace_bytes(int64_t n);
hipError_t launch_argmax_ws(const float* x, int64_t n, int32_t* out, int32_t* pos_dev,
                            void* ws, hipStream_t stream);

}  // namespace mlq
