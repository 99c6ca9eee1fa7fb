/*
 * CPU ORACLE — test infrastructure only.
 *
 * Plain-C restatement of the reference's CPU decode-step operators around the
 * quantized Linear (Haobin-Lee/mini-llama src/ops.cc, src/forward.cc,
 * src/matmul_dispatch.cc). It checks the HIP decode path and is never part
 * of it: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * Parity pinning (tests/test_oracle_forward.py):
 *   ref_rmsnorm      reference known answers (tests/test_ops.cc:140-185) +
 *                    closed form for constant vectors + exact power-of-two
 *                    scale invariance (eps = 0) + float64 brute force.
 *   ref_softmax      reference known answers (test_ops.cc:190-212) +
 *                    scipy.special.softmax.
 *   ref_silu/swiglu  reference known answers (test_ops.cc:240-277) +
 *                    scipy.special.expit closed form.
 *   ref_rope         position 0 is the identity (exact) + the rotation as a
 *                    complex product in float64, for both pairings (a wrong
 *                    sign, pairing or frequency exponent fails) + pair norms.
 *   ref_attention    the reference's closed-form cases (test_cuda.cc:999-1064:
 *                    pos 0 returns V, uniform scores average V per kv head)
 *                    + float64 matrix-form softmax(QK^T/sqrt(d))V over the
 *                    cache + a one-hot score case.
 *   ref_linear_f32   exact small-integer sums + float64 brute force.
 *   ref_argmax       reference known answer (test_ops.cc:320-345) +
 *                    numpy.argmax on NaN-free data + NaN rules.
 * The forward composition (oracle.forward_token) is pinned separately: the
 * incremental decode with its KV cache must equal a float64 full-sequence
 * causal forward at every position, and the tiny model's greedy tokens.
 */
#ifndef MLQ_ORACLE_FORWARD_REF_H_
#define MLQ_ORACLE_FORWARD_REF_H_

#ifdef __cplusplus
extern "C" {
#endif

/* rmsNorm (src/ops.cc:43-72) on one row of `dim` floats. */
void ref_rmsnorm(const float* x, const float* w, float* y, int dim, float eps);
/* softmax (src/ops.cc:74-109); returns -1 for n <= 0. */
int ref_softmax(const float* x, float* y, int n);
/* silu (src/ops.cc:111-119) and swiGlu = silu(gate) * up (:121-140). */
void ref_silu(const float* x, float* y, int n);
void ref_swiglu(const float* gate, const float* up, float* y, int n);
/* rope (src/ops.cc:142-228) in place on q [n_heads][hd], k [n_kv][hd];
 * type 0 normal, 1 NeoX. Returns -1 on the reference's rejections. */
int ref_rope(float* q, float* k, int n_heads, int n_kv, int hd, int pos, float theta,
             int type);
/* Attention of forwardAttention's CPU branch (src/forward.cc:526-565) for
 * query q [n_heads][hd] over cache positions 0..pos of `layer`, cache
 * [layers][max_seq][n_kv][hd]. */
void ref_attention(const float* q, const float* keys, const float* values, int layer,
                   int pos, int n_heads, int n_kv, int hd, int max_seq, float* out);
/* linearNaive (src/matmul_dispatch.cc:32-50): y[n] = sum_k x[k] W[n][k]. */
void ref_linear_f32(const float* x, const float* w, float* y, int n, int k);
/* argMax (src/ops.cc:230-246); -1 for n <= 0. */
int ref_argmax(const float* x, int n);

#ifdef __cplusplus
}
#endif

#endif /* MLQ_ORACLE_FORWARD_REF_H_ */
