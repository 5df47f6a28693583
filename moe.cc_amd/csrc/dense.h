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
  // Optional rmsnorm of the A rows inside the product (few tokens only, see
  // dense_norm_ok): A is replaced by rmsnorm(A, norm_w, eps)
  // (test_model_trace.c:241-255, norm_w NULL = weight 1).  Each block then
  // writes a column slice of the normalized rows to xn_out [M][K] (if given)
  // and, with the fused selection below, packs that slice into activation
  // tables for the expert GEMVs (pack_dtype 2 / 3, tables of
  // act_table_bytes(K) bytes at pack_tabs; pack_part: scratch of
  // M * gridDim.x * 2 words for the slices' headers, reduced by the last
  // block).  The 5-16 token rows kernel (dense_rows4_path) packs given rows
  // without a norm or a fused selection: pack_part then holds N * 16 uint2
  // {limbs, sum}, slice-major, combined by select_kernel.
  int norm = 0;
  const float* norm_w = nullptr;
  float eps = 0.0f;
  float* xn_out = nullptr;
  int pack_dtype = 0;
  uint8_t* pack_tabs = nullptr;
  uint32_t* pack_part = nullptr;
  // Optional expert selection after the product (few tokens, C = router
  // logits [M][N]): the last block to finish picks each token's top
  // sel_topk of the N logits by the insertion rule and their softmax gates
  // (test_model_trace.c:275-288, :482-487) into sel_idx / sel_p ([M][topk])
  // and the caller's copies (may be null).  sel_counter: a device counter
  // that is zero between launches (the last block resets it).
  unsigned* sel_counter = nullptr;
  int sel_topk = 0;
  int* sel_idx = nullptr;
  float* sel_p = nullptr;
  int32_t* sel_idx_user = nullptr;
  float* sel_p_user = nullptr;
  // With the fused selection, only where dense_row_path(a) holds: the row
  // kernel runs alone, and the caller's next kernel reads C and pack_part
  // and does the selection and the tables' headers itself.
  int sel_defer = 0;
  // Optional, one token (dense_amax_ok): each block of dense_amax_rows(N)
  // consecutive outputs also writes its largest value (NaN if it has one)
  // to amax_part[block], for greedy_vec.
  float* amax_part = nullptr;
  // Optional (row kernel): one thread advances this device word by one
  // (skipping 0) -- the tag of the launch that follows.
  uint32_t* epoch_bump = nullptr;
};
moe_status dense_matmul(const DenseArgs& a, hipStream_t s);
bool dense_amax_ok(const DenseArgs& a);
int dense_amax_rows(int N);
// Whether dense_matmul can fuse the rmsnorm for M rows of K columns.
bool dense_norm_ok(int M, int K);
// Whether dense_matmul can fuse the expert selection (M tokens, N experts).
bool dense_select_ok(int M, int N);
// Whether dense_matmul runs `a` with the one-token row kernel (one block
// per output row; with packing, pack_part then holds N partial headers).
bool dense_row_path(const DenseArgs& a);
// True where dense_matmul runs a (5-16 token, no norm, no fused selection)
// product on the rows kernel, which can also pack the rows.
bool dense_rows4_path(const DenseArgs& a);

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
  float* kc; float* vc;
  float* S; float* H;
  int T, pos0, nq, nkv, hd, max_seq;
  float scale;
  // T == 1 only: the score launch also does heads_norm_rope's work for its
  // row (q/k norm, RoPE, K and V into the caches); qkv holds the raw
  // projections then and heads_norm_rope is not called.
  int fuse_heads = 0;
  const float* q_norm = nullptr; const float* k_norm = nullptr; float eps = 0.0f;
  const float* rope_cos = nullptr; const float* rope_sin = nullptr;
  // set by attention_rows: the one-row kernels' blocks of one KV head group
  // share an XCD (attn_xcd_map)
  int xcd_map = 0;
  // Optional, T == 1: the matrix of the product that follows (the O
  // projection, pf_n rows of leading dimension pf_ld).  Block b of the
  // softmax launch requests the first kAttnPfCols columns of rows
  // kAttnPfRows b .. kAttnPfRows b + kAttnPfRows - 1 while it waits for
  // its scores, so that the product's first chunks come from the
  // memory-side cache; the values are not used.
  const float* pf_w = nullptr;
  int pf_ld = 0, pf_n = 0;
};
constexpr int kAttnPfRows = 8, kAttnPfCols = 512;
moe_status attention_rows(const AttnArgs& a, hipStream_t s);

// The reference's next token over n logits (test_model_trace.c:735-746):
// the first index of the largest softmax_rows probability.  part / rows:
// the head product's block maxima (DenseArgs::amax_part) or null.  Written
// to *out and, if out_hist, to out_hist[*hist_pos] with *hist_pos
// incremented (device counters).
moe_status greedy_vec(const float* v, int n, const float* part, int rows, int32_t* out,
                      int32_t* out_hist, int32_t* hist_pos, hipStream_t s);

// softmax_rows (test_model_trace.c:260-272) of one row of n values in place.
moe_status softmax_vec(float* v, int n, hipStream_t s);

}  // namespace moe
