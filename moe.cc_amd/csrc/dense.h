// dense.h - host-side launchers of the fp32 (non-expert) kernels of
// dense.hip.  Internal; the public ABI is include/moehip.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_lib.h"

namespace moe {

// C[m][n] = epilogue(sum_k A[m][k] * W[n][k]), k ascending, every product
// and every sum rounded on its own (test_model_trace.c:213-227); epilogue:
// c = acc, then c + bias[n] if bias (the reference's separate bias loops),
// then resid[m][n] + c if resid (a residual add of the same row).
struct DenseArgs {
  const float* A; long long lda;
  const float* W; long long ldw;
  const float* bias;
  const float* resid; long long ldr;
  float* C; long long ldc;
  int M, N, K;
};
moe_status dense_matmul(const DenseArgs& a, hipStream_t s);

// x[t] = emb[ids[t]] (ids clamped to [0, V)), T rows of D floats.
moe_status embed_rows(const int32_t* ids, int T, const float* emb, int V, int D, float* x,
                      hipStream_t s);

// Per row t (absolute position pos0 + t) of qkv [T][ld] = [Q | K | V] heads:
// q/k per-head RMSNorm (when the weights are given) and RoPE from the
// cos/sin tables [max_seq][hd/2]; Q is rewritten in place, K and V rows go
// to the caches kc/vc [n_kv][max_seq][hd].
struct HeadArgs {
  float* qkv; int ld;
  int T, pos0, nq, nkv, hd, max_seq;
  const float* q_norm; const float* k_norm; float eps;
  const float* rope_cos; const float* rope_sin;
  float* kc; float* vc;
};
moe_status heads_norm_rope(const HeadArgs& a, hipStream_t s);

// Causal attention of the T new rows (test_model_trace.c:404-426): scores
// S[t][h][tk] = (q . k_tk) * scale for tk <= pos0 + t, then the softmax and
// the weighted V sum into H [T][nq*hd].  S is scratch [T][nq][max_seq].
struct AttnArgs {
  const float* qkv; int ld;
  const float* kc; const float* vc;
  float* S; float* H;
  int T, pos0, nq, nkv, hd, max_seq;
  float scale;
};
moe_status attention_rows(const AttnArgs& a, hipStream_t s);

// Greedy choice over n logits: the first index of the largest value
// (test_model_trace.c:742-746); written to *out and, if out_hist, to
// out_hist[*hist_pos] with *hist_pos incremented (device counters).
moe_status argmax_vec(const float* v, int n, int32_t* out, int32_t* out_hist, int32_t* hist_pos,
                      hipStream_t s);

// softmax_rows (test_model_trace.c:260-272) of one row of n values in place.
moe_status softmax_vec(float* v, int n, hipStream_t s);

}  // namespace moe
