/*
 * oracle.h - CPU restatement of moe.cc's quantized expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * moe.cc_amd/) links, loads or calls this code.  It is the checker that the
 * GPU kernels are compared against: tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py are its only users.
 *
 * Every function restates one piece of the reference's arithmetic, keeping
 * its loop order and its types, so the results are bit-identical to the
 * reference built with its own Makefile flags (gcc -O2, no -march, hence no
 * FMA contraction on x86-64).  Each function names the reference lines it
 * follows.  The restatement is pinned by fixtures written from the compiled
 * reference sources (tests/golden/) and by closed-form / brute-force checks in
 * tests/test_oracle_*.py.
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order and types as the reference's QuantizedWeight
 * (model.h:26-31): {q, s, rows, cols, dtype}.  dtype 2 = Q8, 3 = Q4. */
typedef struct {
  const int8_t* q;
  const float* s;
  int rows, cols;
  int dtype;
} orc_qweight;

/* (int32_t)(v) as compiled by gcc for x86-64 (cvttss2si): truncation toward
 * zero, and INT32_MIN for NaN or a value whose truncation is outside int32. */
int32_t orc_f2i_trunc(float v);

/* kernels.c:51-74  C[m,n] = ((float)sum_k trunc(A[m,k]*127) * B[n,k] / 127) * s[n] */
void orc_gemv_q8(const float* A, const int8_t* Bq, const float* Bs, float* C,
                 int M, int N, int K);
/* kernels.c:96-128 nibble-packed variant (low nibble = even column), 7.0f */
void orc_gemv_q4(const float* A, const uint8_t* Bq, const float* Bs, float* C,
                 int M, int N, int K);
/* kernels.c:149-181 dispatcher: W_q==NULL -> fp32, dtype 2/3, else zeros */
void orc_matmul_adaptive(const float* A, const float* W_fp32, const orc_qweight* W_q,
                         float* C, int M, int N, int K);
/* test_model_trace.c:213-227 (same loop as kernels.c:155-165) */
void orc_matmul_f32(const float* A, const float* B, float* C, int M, int N, int K);
/* test_model_trace.c:229-236 */
void orc_silu(float* x, int n);
/* test_model_trace.c:241-255; w may be NULL (weight 1) */
void orc_rmsnorm(const float* x, const float* w, int T, int D, float eps, float* y);
/* test_model_trace.c:275-288 */
void orc_topk_desc(const float* x, int E, int k, int* idx, float* val);
/* test_model_trace.c:482-487: softmax over the k selected logits, in place */
void orc_softmax_topk(float* val, int k);

/* test_model_trace.c:463-517, the MoE block of layer_forward_f32.
 *   x_norm  [T x D]  router and expert input (x_norm2 in the reference)
 *   x_resid [T x D]  residual added at the end (x_after); NULL -> no residual
 *   out     [T x D]  x_resid + moe_out (or moe_out)
 *   idx_out [T x k], p_out [T x k] optional: selected experts and gates
 *   logits_out [T x E] optional: router logits (after bias)
 * Experts are given as arrays of E quantized weights (gate, up, down). */
void orc_moe_block(const float* x_norm, const float* x_resid, int T, int D,
                   int E, int top_k, int d_ff,
                   const float* router_w, const float* router_b,
                   const orc_qweight* Wg, const orc_qweight* Wu, const orc_qweight* Wd,
                   float* out, int* idx_out, float* p_out, float* logits_out);

/* ---- the dense fp32 half of the model (model_oracle.c) ---- */

/* QwenConfig (model.h:9-23), same field order and types */
typedef struct {
  int d_model, n_layers, head_dim, n_q, n_kv, d_ff, n_experts, top_k, vocab_size, causal;
  float rope_theta, rms_eps;
} orc_config;

/* One layer's tensors (model.h:34-58, quantized experts only); biases and
 * q/k norms may be NULL. */
typedef struct {
  const float *Wq, *bq, *Wk, *bk, *Wv, *bv, *Wo, *bo;
  const float *q_norm, *k_norm, *rms1_w, *rms2_w, *router_w, *router_b;
  const orc_qweight *Wg, *Wu, *Wd;   /* [n_experts] each */
} orc_layer;

/* QwenWeights (model.h:60-69); lm_head NULL = tied to tok_emb */
typedef struct {
  const float* tok_emb;
  const float* final_norm_w;
  const float* lm_head;
  const orc_layer* layers;
} orc_weights;

/* test_model_trace.c:433-521 for T rows at positions pos0.., KV cached */
void orc_layer_rows(const orc_config* cfg, const orc_layer* lw, float* x, int T, int pos0,
                    float* kc, float* vc, int max_seq);
/* test_model_trace.c:526-579 for the new rows; kc/vc [L][n_kv][max_seq][hd] */
void orc_model_forward_kv(const orc_config* cfg, const orc_weights* w, const int* ids, int T,
                          int pos0, float* kc, float* vc, int max_seq, float* out_last,
                          float* x_out);
/* RoPE cos/sin of test_model_trace.c:310-336 for positions 0..n_pos-1:
 * [n_pos][hd/2] each */
void orc_rope_tables(int hd, float theta, int n_pos, float* cos_out, float* sin_out);
/* test_model_trace.c:260-272, rows of cols values in place */
void orc_softmax_rows(float* mat, int rows, int cols);
/* next-token choice: first index of the largest softmax_rows probability
 * (test_model_trace.c:735-746) */
int orc_greedy(const float* v, int n);

/* export.py:23-27 rowwise Q8: s = max(amax,1e-8)/127, q = round-half-even(w/s) */
void orc_quant_q8_rows(const float* W, int N, int K, int8_t* q, float* s);
/* export.py:29-36 rowwise Q4: s = max(amax,1e-8)/7, q = clamp(rne(w/s),-8,7)+8,
 * byte j = q[2j] | q[2j+1] << 4   (K must be even, as the exporter's slicing
 * pairs columns) */
void orc_quant_q4_rows(const float* W, int N, int K, uint8_t* q, float* s);

/* Seeded synthetic data: splitmix64 -> xoshiro256** -> Box-Muller (double). */
void orc_fill_normal(float* out, size_t n, uint64_t seed, float mean, float std);
void orc_fill_uniform_u32(uint32_t* out, size_t n, uint64_t seed);

/* host libm expf, exported so tests compare device expf against it */
void orc_expf_array(const float* x, float* y, size_t n);
/* count of inputs in [lo, hi] (as u32 bit patterns) where f(x) differs from
 * expf(x) bitwise, with f given as a table of device results for that range */
uint64_t orc_expf_mismatch_u32range(uint32_t lo, uint32_t count, const float* dev,
                                    uint32_t* first_bad);

/* Threads of the row-parallel loops: omp_get_max_threads() in the -fopenmp
 * build (liboracle_omp.so), 1 in the single-thread build. */
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
