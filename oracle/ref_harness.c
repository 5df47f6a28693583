/*
 * ref_harness.c - exposes the reference's own static MoE/model functions so
 * that the C restatement (moe_oracle.c) can be checked against them.
 *
 * TEST INFRASTRUCTURE ONLY.  This file contains none of the reference's code:
 * it compiles /root/reference/test_model_trace.c in place (the include path
 * points at the read-only reference tree; nothing is copied) and adds
 * extern "C" wrappers around its static functions.  oracle/Makefile builds it
 * into oracle/_ref/libref_trace.so together with the reference's io.c,
 * utils.c and kernels.c, with the reference Makefile:3 flags.  The library is
 * used only in this container, to write tests/golden/ fixtures and to
 * cross-check the restatement; it never travels to the GPU box as a checker
 * the tests depend on (tests skip the comparison when it is absent).
 */
#define main moe_ref_trace_main
#include "test_model_trace.c"
#undef main

/* The reference's profiler registers an atexit dump on first use; clearing
 * its table after each wrapped call keeps that dump empty. */
static void quiet_profiler(void) { memset(__prof_tab, 0, sizeof(__prof_tab)); }

void ref_matmul_f32(const float* A, const float* B, float* C, int M, int N, int K) {
  matmul_f32(A, B, C, M, N, K);
  quiet_profiler();
}

void ref_silu(float* x, int n) {
  silu_f32(x, n);
  quiet_profiler();
}

void ref_rmsnorm(const float* x, const float* w, int T, int D, float eps, float* y) {
  rmsnorm_forward_f32(x, w, T, D, eps, y);
  quiet_profiler();
}

void ref_topk_desc(const float* x, int E, int k, int* idx, float* val) {
  topk_desc(x, E, k, idx, val);
  quiet_profiler();
}

void ref_softmax_rows(float* m, int rows, int cols) {
  softmax_rows(m, rows, cols);
  quiet_profiler();
}

/* One call of layer_forward_f32 (test_model_trace.c:433-521) with every
 * attention weight zero and a 1-head, head_dim-2 attention, so that its
 * output is exactly zero and the layer reduces to
 *     x <- x + MoE(rmsnorm(x, rms2_w))
 * i.e. the MoE block (:460-517) including norm2 and the residual.
 * x [T x D] is updated in place.  Expert arrays hold E entries each. */
void ref_moe_layer(float* x, int T, int D, int E, int top_k, int d_ff,
                   const float* rms2_w, const float* router_w, const float* router_b,
                   QuantizedWeight* Wg, QuantizedWeight* Wu, QuantizedWeight* Wd) {
  const int n_q = 1, n_kv = 1, hd = 2;
  const int Dq = n_q * hd, Dkv = n_kv * hd;
  float* zq = (float*)calloc((size_t)Dq * D, sizeof(float));
  float* zkv = (float*)calloc((size_t)Dkv * D, sizeof(float));
  float* zo = (float*)calloc((size_t)D * Dq, sizeof(float));
  QwenLayerWeights lw;
  memset(&lw, 0, sizeof(lw));
  lw.Wq = zq; lw.Wk = zkv; lw.Wv = zkv; lw.Wo = zo;
  lw.rms1_w = NULL;
  lw.rms2_w = rms2_w;
  lw.router_w = router_w;
  lw.router_b = router_b;
  lw.Wg_q = Wg; lw.Wu_q = Wu; lw.Wd_q = Wd;
  lw.experts_quantized = 1;
  size_t attn_f = (size_t)T * (Dq + 2 * Dkv) + (size_t)T * T + (size_t)T * Dq;
  size_t temps_f = 4ull * (size_t)T * D;
  float* scratch_attn = (float*)calloc(attn_f + temps_f, sizeof(float));
  float* scratch_moe = (float*)calloc((size_t)T * E + (size_t)T * D, sizeof(float));
  int* tidx = (int*)calloc((size_t)top_k, sizeof(int));
  float* tval = (float*)calloc((size_t)top_k, sizeof(float));
  layer_forward_f32(x, T, D, &lw, n_q, n_kv, hd, 1, 10000000.f, 1e-6f,
                    E, top_k, d_ff, scratch_attn, scratch_moe, tidx, tval);
  free(zq); free(zkv); free(zo);
  free(scratch_attn); free(scratch_moe); free(tidx); free(tval);
  quiet_profiler();
}

/* model_forward_f32 (test_model_trace.c:526-579) on a QW3W file: loads it
 * with the reference's bin_load + load_all_weights and returns the last-row
 * logits [vocab].  Returns the vocab size, or -1 if the file cannot be read. */
int ref_model_forward_file(const char* path, const int* ids, int T, float* out_last,
                           int vocab_cap) {
  BinFile* bf = bin_load(path);
  if (!bf) return -1;
  QwenConfig cfg;
  QwenWeights w;
  load_all_weights(bf, &cfg, &w);
  if (cfg.vocab_size > vocab_cap) { bin_free(bf); return -1; }
  model_forward_f32(ids, T, &cfg, &w, 0, out_last);
  for (int l = 0; l < cfg.n_layers; ++l) {
    free((void*)w.layers[l].Wg); free((void*)w.layers[l].Wu); free((void*)w.layers[l].Wd);
    free(w.layers[l].Wg_q); free(w.layers[l].Wu_q); free(w.layers[l].Wd_q);
  }
  free(w.layers);
  int V = cfg.vocab_size;
  bin_free(bf);
  quiet_profiler();
  return V;
}

/* bin_load + load_all_weights (io.c:193-285, model.h:107-323) on a QW3W
 * file; reports the inferred config and, for layer `layer` and expert
 * `expert`, the gate/up/down QuantizedWeight fields and the first bytes of
 * their data, so that a writer's output can be checked against the reader. */
typedef struct {
  int count;
  int d_model, n_layers, head_dim, n_q, n_kv, d_ff, n_experts, top_k, vocab;
  int experts_quantized;
  int rows[3], cols[3], dtype[3];
  unsigned char q_head[3][16];
  float s_head[3][4];
  float router_w0, rms2_w0;
} ref_bin_summary;

int ref_bin_describe(const char* path, int layer, int expert, ref_bin_summary* out) {
  BinFile* bf = bin_load(path);
  if (!bf) return -1;
  QwenConfig cfg;
  QwenWeights w;
  memset(out, 0, sizeof(*out));
  load_all_weights(bf, &cfg, &w);
  out->count = bf->count;
  out->d_model = cfg.d_model; out->n_layers = cfg.n_layers; out->head_dim = cfg.head_dim;
  out->n_q = cfg.n_q; out->n_kv = cfg.n_kv; out->d_ff = cfg.d_ff;
  out->n_experts = cfg.n_experts; out->top_k = cfg.top_k; out->vocab = cfg.vocab_size;
  QwenLayerWeights* lw = &w.layers[layer];
  out->experts_quantized = lw->experts_quantized;
  out->router_w0 = lw->router_w[0];
  out->rms2_w0 = lw->rms2_w[0];
  if (lw->experts_quantized) {
    QuantizedWeight* qs[3] = { &lw->Wg_q[expert], &lw->Wu_q[expert], &lw->Wd_q[expert] };
    for (int i = 0; i < 3; ++i) {
      out->rows[i] = qs[i]->rows; out->cols[i] = qs[i]->cols; out->dtype[i] = qs[i]->dtype;
      memcpy(out->q_head[i], qs[i]->q, 16);
      memcpy(out->s_head[i], qs[i]->s, 4 * sizeof(float));
    }
  }
  for (int l = 0; l < cfg.n_layers; ++l) {
    free((void*)w.layers[l].Wg); free((void*)w.layers[l].Wu); free((void*)w.layers[l].Wd);
    free(w.layers[l].Wg_q); free(w.layers[l].Wu_q); free(w.layers[l].Wd_q);
  }
  free(w.layers);
  bin_free(bf);
  return 0;
}
