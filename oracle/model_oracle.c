/*
 * model_oracle.c - CPU restatement of the dense (fp32) half of the
 * reference's Qwen3-MoE forward with a KV cache, around the MoE block of
 * moe_oracle.c.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built with the reference's
 * flags (gcc -O2, no -march): every fp32 multiply and add is rounded on its
 * own, sqrtf / division are IEEE, expf / powf / cosf / sinf are the host
 * glibc's, so the results are bit-identical to the reference.
 *
 * The reference recomputes the whole prefix at every step
 * (test_model_trace.c:526-579).  This restatement keeps K and V of every
 * earlier position in a cache and computes only the new rows.  That gives
 * the same bits for the new rows because
 *   - every per-row operation (embedding, rmsnorm, the projections, q/k
 *     norm, RoPE at absolute position p, the MoE block) reads only its own
 *     row, so cached K/V rows equal the ones the recompute produces;
 *   - a query at position p over positions 0..p sees the same scores, max,
 *     exponentials, sum and weighted V sum, in the same order, as the
 *     reference's row p over 0..T-1 with the causal mask: the masked
 *     positions hold -inf, their expf is +0, and adding +0 to the running
 *     sum or +-0 (0 * v) to an accumulator that started at +0 leaves it
 *     unchanged (an IEEE round-to-nearest sum of nonzero terms is never -0).
 * tests/test_oracle_model.py checks the claim against the compiled reference.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* test_model_trace.c:381-402: per-head RMSNorm of a [n_heads x hd] row:
 * sequential sum of squares, inv = 1/sqrtf(msq/hd + eps), v = (v*inv)*w. */
static void orc_head_norm(float* row, int n_heads, int hd, const float* w, float eps) {
  for (int h = 0; h < n_heads; ++h) {
    float* v = row + (size_t)h * hd;
    float msq = 0.0f;
    for (int d = 0; d < hd; ++d) {
      float z = v[d];
      float zz = z * z;
      msq = msq + zz;
    }
    float m = msq / (float)hd;
    float inv = 1.0f / sqrtf(m + eps);
    for (int d = 0; d < hd; ++d) {
      float a = v[d] * inv;
      v[d] = a * w[d];
    }
  }
}

/* test_model_trace.c:299-338 for one row at absolute position pos:
 * inv_i = powf(theta, (-2*i)/hd), ang = pos * inv_i, and the pair
 * (v[i], v[i + hd/2]) rotated by (cosf(ang), sinf(ang)) (:290-294). */
static void orc_rope_row(float* row, int n_heads, int hd, int pos, float theta) {
  const int d2 = hd / 2;
  const float p = (float)pos;
  for (int h = 0; h < n_heads; ++h) {
    float* v = row + (size_t)h * hd;
    for (int i = 0; i < d2; ++i) {
      float exponent = -2.0f * (float)i / (float)hd;
      float inv = powf(theta, exponent);
      float ang = p * inv;
      float c = cosf(ang), s = sinf(ang);
      float e = v[i], o = v[i + d2];
      float ec = e * c, os = o * s, oc = o * c, es = e * s;
      v[i] = ec - os;
      v[i + d2] = oc + es;
    }
  }
}

void orc_rope_tables(int hd, float theta, int n_pos, float* cos_out, float* sin_out) {
  const int d2 = hd / 2;
  for (int pos = 0; pos < n_pos; ++pos) {
    const float p = (float)pos;
    for (int i = 0; i < d2; ++i) {
      float exponent = -2.0f * (float)i / (float)hd;
      float inv = powf(theta, exponent);
      float ang = p * inv;
      cos_out[(size_t)pos * d2 + i] = cosf(ang);
      sin_out[(size_t)pos * d2 + i] = sinf(ang);
    }
  }
}

/* test_model_trace.c:402-426 for one query row qv of one head at position
 * P: scores over cache positions 0..P (k rows kbase + tk*hd), the softmax
 * (max, expf, sequential sum, 1/(sum + 1e-9)), then the weighted V sum in
 * position order into out[hd].  S: scratch of P + 1 floats. */
static void attention_row(const float* qv, const float* kbase, const float* vbase, int P, int hd,
                          float scale, float* S, float* out) {
  for (int tk = 0; tk <= P; ++tk) {
    const float* kv = kbase + (size_t)tk * hd;
    float dot = 0.0f;
    for (int d = 0; d < hd; ++d) {
      float pr = qv[d] * kv[d];
      dot = dot + pr;
    }
    S[tk] = dot * scale;
  }
  float m = S[0];
  for (int i = 1; i <= P; ++i) if (S[i] > m) m = S[i];
  float ssum = 0.0f;
  for (int i = 0; i <= P; ++i) {
    float e = expf(S[i] - m);
    S[i] = e;
    ssum = ssum + e;
  }
  float inv = 1.0f / (ssum + 1e-9f);
  for (int i = 0; i <= P; ++i) S[i] = S[i] * inv;
  for (int d = 0; d < hd; ++d) out[d] = 0.0f;
  for (int tk = 0; tk <= P; ++tk) {
    const float* vv = vbase + (size_t)tk * hd;
    const float pk = S[tk];
    for (int d = 0; d < hd; ++d) {
      float pv = pk * vv[d];
      out[d] = out[d] + pv;
    }
  }
}

/* test_model_trace.c:341-430 for the T rows at positions pos0..pos0+T-1 of
 * one layer: projections (+ bias), q/k norm, RoPE, K/V appended to the
 * cache (kc/vc: [n_kv][max_seq][hd] of this layer), causal attention of each
 * new row over the cache, output projection (+ bias). */
static void orc_attention_rows(const orc_config* cfg, const orc_layer* lw, const float* xn,
                               int T, int pos0, float* kc, float* vc, int max_seq, float* y) {
  const int D = cfg->d_model, hd = cfg->head_dim, nq = cfg->n_q, nkv = cfg->n_kv;
  const int Dq = nq * hd, Dkv = nkv * hd;
  const float scale = 1.0f / sqrtf((float)hd);
  float* Q = (float*)malloc(sizeof(float) * (size_t)T * Dq);
  float* K = (float*)malloc(sizeof(float) * (size_t)T * Dkv);
  float* V = (float*)malloc(sizeof(float) * (size_t)T * Dkv);
  float* H = (float*)malloc(sizeof(float) * (size_t)T * Dq);
  const size_t ns = (size_t)(pos0 + T);   /* scores of one row, one buffer per head */
  float* Sall = (float*)malloc(sizeof(float) * ns * (size_t)nq);
  orc_matmul_f32(xn, lw->Wq, Q, T, Dq, D);
  orc_matmul_f32(xn, lw->Wk, K, T, Dkv, D);
  orc_matmul_f32(xn, lw->Wv, V, T, Dkv, D);
  if (lw->bq) for (int t = 0; t < T; ++t) for (int i = 0; i < Dq; ++i) Q[(size_t)t * Dq + i] += lw->bq[i];
  if (lw->bk) for (int t = 0; t < T; ++t) for (int i = 0; i < Dkv; ++i) K[(size_t)t * Dkv + i] += lw->bk[i];
  if (lw->bv) for (int t = 0; t < T; ++t) for (int i = 0; i < Dkv; ++i) V[(size_t)t * Dkv + i] += lw->bv[i];
  for (int t = 0; t < T; ++t) {
    if (lw->q_norm) orc_head_norm(Q + (size_t)t * Dq, nq, hd, lw->q_norm, cfg->rms_eps);
    if (lw->k_norm) orc_head_norm(K + (size_t)t * Dkv, nkv, hd, lw->k_norm, cfg->rms_eps);
    orc_rope_row(Q + (size_t)t * Dq, nq, hd, pos0 + t, cfg->rope_theta);
    orc_rope_row(K + (size_t)t * Dkv, nkv, hd, pos0 + t, cfg->rope_theta);
    for (int h = 0; h < nkv; ++h) {
      memcpy(kc + ((size_t)h * max_seq + pos0 + t) * hd, K + (size_t)t * Dkv + (size_t)h * hd,
             sizeof(float) * hd);
      memcpy(vc + ((size_t)h * max_seq + pos0 + t) * hd, V + (size_t)t * Dkv + (size_t)h * hd,
             sizeof(float) * hd);
    }
  }
  const int group = nq / nkv;
  /* heads are independent: with -fopenmp each thread takes whole heads */
#pragma omp parallel for schedule(static) if ((size_t)nq * ns * (size_t)hd >= 65536)
  for (int h = 0; h < nq; ++h)
    for (int t = 0; t < T; ++t)
      attention_row(Q + (size_t)t * Dq + (size_t)h * hd, kc + (size_t)(h / group) * max_seq * hd,
                    vc + (size_t)(h / group) * max_seq * hd, pos0 + t, hd, scale,
                    Sall + (size_t)h * ns, H + (size_t)t * Dq + (size_t)h * hd);
  orc_matmul_f32(H, lw->Wo, y, T, D, Dq);
  if (lw->bo) for (int t = 0; t < T; ++t) for (int i = 0; i < D; ++i) y[(size_t)t * D + i] += lw->bo[i];
  free(Q); free(K); free(V); free(H); free(Sall);
}

/* test_model_trace.c:433-521, one layer for T rows, x updated in place. */
void orc_layer_rows(const orc_config* cfg, const orc_layer* lw, float* x, int T, int pos0,
                    float* kc, float* vc, int max_seq) {
  const int D = cfg->d_model;
  const size_t n = (size_t)T * D;
  float* xn1 = (float*)malloc(sizeof(float) * n);
  float* att = (float*)malloc(sizeof(float) * n);
  float* xa = (float*)malloc(sizeof(float) * n);
  float* xn2 = (float*)malloc(sizeof(float) * n);
  orc_rmsnorm(x, lw->rms1_w, T, D, cfg->rms_eps, xn1);
  orc_attention_rows(cfg, lw, xn1, T, pos0, kc, vc, max_seq, att);
  for (size_t i = 0; i < n; ++i) xa[i] = x[i] + att[i];
  orc_rmsnorm(xa, lw->rms2_w, T, D, cfg->rms_eps, xn2);
  orc_moe_block(xn2, xa, T, D, cfg->n_experts, cfg->top_k, cfg->d_ff, lw->router_w,
                lw->router_b, lw->Wg, lw->Wu, lw->Wd, x, NULL, NULL, NULL);
  free(xn1); free(att); free(xa); free(xn2);
}

/* test_model_trace.c:526-579 restricted to the new rows: embedding
 * (:548-553), the layer stack, final norm and the head on the last row
 * (:567-571; lm_head NULL = tied to the embedding).  kc / vc: caches of all
 * layers, [n_layers][n_kv][max_seq][head_dim]; rows pos0..pos0+T-1 are
 * written.  out_last [vocab]: logits of the last new row.  x_out (optional,
 * [T x D]): the hidden state after the last layer. */
void orc_model_forward_kv(const orc_config* cfg, const orc_weights* w, const int* ids, int T,
                          int pos0, float* kc, float* vc, int max_seq, float* out_last,
                          float* x_out) {
  const int D = cfg->d_model;
  const size_t per_layer = (size_t)cfg->n_kv * max_seq * cfg->head_dim;
  float* x = (float*)malloc(sizeof(float) * (size_t)T * D);
  for (int t = 0; t < T; ++t)
    memcpy(x + (size_t)t * D, w->tok_emb + (size_t)ids[t] * D, sizeof(float) * D);
  for (int l = 0; l < cfg->n_layers; ++l)
    orc_layer_rows(cfg, &w->layers[l], x, T, pos0, kc + l * per_layer, vc + l * per_layer,
                   max_seq);
  if (x_out) memcpy(x_out, x, sizeof(float) * (size_t)T * D);
  float* xf = (float*)malloc(sizeof(float) * D);
  orc_rmsnorm(x + (size_t)(T - 1) * D, w->final_norm_w, 1, D, cfg->rms_eps, xf);
  const float* head = w->lm_head ? w->lm_head : w->tok_emb;
  orc_matmul_f32(xf, head, out_last, 1, cfg->vocab_size, D);
  free(xf);
  free(x);
}

/* The reference's choice of the next token (test_model_trace.c:735-746):
 * softmax_rows over the logits (:736), then the first index whose
 * probability beats every earlier one (start at index 0, replace on a
 * strict '>').  Equal probabilities keep the lower index, also where the
 * logits differ but round to the same probability; a NaN or +inf logit
 * (or all -inf) turns every probability into NaN, so the answer is 0. */
int orc_greedy(const float* v, int n) {
  float* p = (float*)malloc(sizeof(float) * (size_t)n);
  memcpy(p, v, sizeof(float) * (size_t)n);
  orc_softmax_rows(p, 1, n);
  int best = 0;
  float mx = p[0];
  for (int i = 1; i < n; ++i)
    if (p[i] > mx) { mx = p[i]; best = i; }
  free(p);
  return best;
}

/* test_model_trace.c:260-272: per row, max (first element, then every
 * larger one), e = expf(v - max) stored in place and summed in order,
 * then every entry multiplied by 1/(sum + 1e-9). */
void orc_softmax_rows(float* mat, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    float* row = mat + (size_t)r * cols;
    float maxv = row[0];
    for (int c = 1; c < cols; ++c) if (row[c] > maxv) maxv = row[c];
    float sum = 0.0f;
    for (int c = 0; c < cols; ++c) {
      float e = expf(row[c] - maxv);
      row[c] = e;
      sum = sum + e;
    }
    float inv = 1.0f / (sum + 1e-9f);
    for (int c = 0; c < cols; ++c) row[c] = row[c] * inv;
  }
}
