// moe_layer.h - device state of one MoE layer and the routing helpers shared
// by the decode kernels (moe_layer.hip) and the grouped multi-token kernels
// (moe_grouped.hip).  Internal; the public ABI is include/moehip.h.
#pragma once
#include <stdint.h>

#include "moe_device.h"
#include "moe_lib.h"

namespace moe {

constexpr int kMaxTopK = 32;

// Pairs of one task (one expert) of the grouped GEMM kernels
// (expert_gemm.hip) at most: 32, 64 or 256 by block shape.
constexpr int kEgPairs = 256;
// The smallest task split (sizes the task list).
constexpr int kMinSplitPairs = 32;
// Blocks of the many-pair grouping at most (sizes L->ghist).
constexpr int kGroupBlocks = 64;

struct LayerDev {
  int dtype = 2, D = 0, dff = 0, E = 0, topk = 0;
  long long rbg = 0, rbd = 0;          // row bytes of gate/up and of down
  float* router_w = nullptr;           // [E][D]
  float* router_b = nullptr;           // [E] or null
  float* rms2_w = nullptr;             // [D] or null
  uint8_t* gq = nullptr; float* gs = nullptr;   // [E][dff][rbg], [E][dff]
  uint8_t* uq = nullptr; float* us = nullptr;
  uint8_t* dq = nullptr; float* ds = nullptr;   // [E][D][rbd], [E][D]
  int grouped_min_T = 0;               // 0: library default
  // per-forward scratch: views of the process-wide shared scratch, set by
  // ensure_scratch before every forward
  int capT = 0;
  float* logits = nullptr;   // [T][E]
  int* idx = nullptr;        // [T][topk]
  float* p = nullptr;        // [T][topk]
  uint8_t* xtab = nullptr;   // [T] packed x_norm rows
  uint8_t* htab = nullptr;   // [T*topk] packed h rows
  float* h = nullptr;        // [T*topk][dff] (decode kernels)
  float* xn = nullptr;       // [T][D] normed input (block forward)
  uint32_t* hpart = nullptr; // [T*topk][h segments][2] partial headers of the h tables
  uint32_t* xpart = nullptr; // partial headers of the x tables packed by the router: up to 4
                             // tokens [T][router blocks][2], 5-16 [router blocks][16][2]
  // grouped kernels: pairs per expert, first pair of each expert in `perm`,
  // pair ids (t * topk + j) grouped by expert, expert outputs per pair
  int* ecount = nullptr;     // [E]
  int* eoff = nullptr;       // [E]
  int* perm = nullptr;       // [T*topk]
  int2* tasks = nullptr;     // [T*topk/kMinSplitPairs + E + 1] tasks of the expert kernels:
                             // {expert | pairs << 16, first pair in perm}, x = -1 past the last
  float* y = nullptr;        // [T*topk][D] fp32 expert outputs (Q8; Q4: the rows whose dot
                             // leaves int16, the others read 0x8000 in y16)
  int16_t* y16 = nullptr;    // Q4: [T*topk][D] down dots (after the -8 sum correction) that fit
                             // int16; -32768 marks an output held in y instead
  int* ghist = nullptr;      // [kGroupBlocks][E] pairs per expert of each grouping block
  uint2* rpart = nullptr;    // [T/16 + 1][ceil(E/4)][16] the router blocks' partial x-table headers
  unsigned* sel_counter = nullptr;   // block counter of the fused selection
  uint64_t* ftag = nullptr;   // one token: tagged words of the gate/up + down launch (or null)
  uint32_t* epoch = nullptr;  // its tag, advanced by the router launch before it
};

// Top-k and softmax gates of T tokens from L->logits into L->idx / L->p
// (and the caller's copies, when given): one wave per token.
// With xpart set, each token's wave also combines the router blocks'
// partial x-table headers (neg per token group of 16) into its table.
// hist (optional): per-grouping-block pair counts, block b taking pairs
// b * per .. (b + 1) * per - 1, added with atomics (zeroed beforehand).
moe_status launch_select(const LayerDev* L, int T, int32_t* idx_out, float* p_out, hipStream_t s,
                         const uint2* xpart = nullptr, int neg = 0, int* hist = nullptr,
                         int per = 0);

// Grouped (expert-major) forward for many tokens; requires grouped_ok(L).
bool grouped_ok(const LayerDev* L);
moe_status layer_forward_grouped(LayerDev* L, const float* xn, const float* resid, int T,
                                 float* out, int32_t* idx_out, float* p_out);

// The grouped GEMM expert kernels (expert_gemm.hip): x unit tables into
// L->xtab; gate/up + SwiGLU into L->htab / L->hpart (one segment per row
// tile of d_ff), then down into L->y, for the tasks group_kernel listed with
// a split of expert_gemm_split(nt) pairs (nt = expert_gemm_tiles, the block
// shape).
bool expert_gemm_ok(const LayerDev* L);
int expert_gemm_tiles(const LayerDev* L, int T);
int expert_gemm_split(int nt);
moe_status launch_expert_gemm(const LayerDev* L, int nt, int ntask, hipStream_t s);

// ---- routing: top-k by the insertion rule, softmax over the selection ----

// 64-bit ordering key of logit v at index i: a larger key comes first in
// the top-k order of test_model_trace.c:275-288 (larger value first, the
// lower index first among equal values).  High word: the value's bits
// mapped to an order-preserving unsigned integer (-0 folded to +0), or 0
// when v is NaN or -inf, which the insertion rule never selects; low word:
// 0xFFFFFFFF - i.
__device__ __forceinline__ uint64_t topk_key(float v, int i) {
  uint32_t k = 0;
  if (v > -__builtin_inff()) {
    const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
    k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}

// The gates of one token's K slots (sidx / sval in LDS, empty slots -1 /
// -inf): p_i = expf(v_i - max) / (sum + 1e-9f), max over the slots in order
// (a larger value replaces it), sum in slot order (test_model_trace.c:
// 482-487); slot i to idx[i] / p[i] and the caller's copies (may be null).
// One wave; sexp is its LDS scratch of K floats.
__device__ __forceinline__ void select_gates(int K, const int* sidx, const float* sval, float* sexp,
                                             int* idx, float* p, int* idx_user, float* p_user) {
  const int lane = threadIdx.x % kWave;
  if (lane < K) {
    float mx = sval[0];
    for (int i = 1; i < K; ++i) if (sval[i] > mx) mx = sval[i];
    sexp[lane] = expf_glibc(sval[lane] - mx);
  }
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
  float sum = 0.0f;
  for (int i = 0; i < K; ++i) sum = sum + sexp[i];
  const float inv = 1.0f / (sum + 1e-9f);
  if (lane < K) {
    const float pv = sexp[lane] * inv;
    idx[lane] = sidx[lane];
    p[lane] = pv;
    if (idx_user) idx_user[lane] = sidx[lane];
    if (p_user) p_user[lane] = pv;
  }
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
}

// One wave selects the experts of one token: every lane ranks its
// candidates e = lane + 64c (c < C, E <= 64*C) among the token's E logits,
// rank = number of keys above the candidate's (topk_key), and a live
// candidate (not NaN, not -inf) with rank < K takes slot `rank` -- the
// result of the insertion rule of test_model_trace.c:275-288 computed
// without a serial pass; slots left over keep index -1.  Then
// p_i = expf(v_i - max) / (sum + 1e-9f), sum in slot order (:482-487).
// keys: this wave's LDS scratch of E uint64 (16-byte aligned);
// sidx/sval/sexp: its LDS slots (kMaxTopK each).  Outputs are rows of K
// entries; the user copies may be null.
template <int C>
__device__ void select_token(const float* __restrict__ logit_row, int E, int K, uint64_t* keys,
                             int* sidx, float* sval, float* sexp, int* idx, float* p,
                             int* idx_user, float* p_user) {
  const int lane = threadIdx.x % kWave;
  float v[C];
  uint64_t kc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int e = lane + kWave * c;
    v[c] = e < E ? logit_row[e] : -__builtin_inff();
    kc[c] = topk_key(v[c], e);
    if (e < E) keys[e] = kc[c];
  }
  if (lane < K) { sidx[lane] = -1; sval[lane] = -__builtin_inff(); }
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
  int rank[C];
#pragma unroll
  for (int c = 0; c < C; ++c) rank[c] = 0;
  const ulonglong2* k2 = reinterpret_cast<const ulonglong2*>(keys);
  int j = 0;
  for (; j + 8 <= E; j += 8) {
    ulonglong2 w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] = k2[j / 2 + u];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < C; ++c) rank[c] += (int)(w[u].x > kc[c]) + (int)(w[u].y > kc[c]);
  }
  for (; j < E; ++j) {
    const uint64_t w = keys[j];
#pragma unroll
    for (int c = 0; c < C; ++c) rank[c] += (int)(w > kc[c]);
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int e = lane + kWave * c;
    if (e < E && v[c] > -__builtin_inff() && rank[c] < K) {
      sidx[rank[c]] = e;
      sval[rank[c]] = v[c];
    }
  }
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
  select_gates(K, sidx, sval, sexp, idx, p, idx_user, p_user);
}

// The slots of one token's selection, by a whole block of NT threads
// (E <= NT, whole waves; contains barriers): the same rank rule as
// select_token (rank = keys above the candidate's; a live candidate with
// rank < K takes slot `rank`, slots left over keep -1 / -inf), the key range
// split into NT / E' parts (E' = E rounded up to a power of two, at most 4
// parts) whose partial ranks add.  v: this thread's logit (candidate
// threadIdx.x, when < E; read by the caller, so that its load can be issued
// early).  keys: LDS scratch of E uint64 (16-byte aligned); part: NT ints.
template <int NT>
__device__ void block_select_slots(float v, int E, int K, uint64_t* keys, int* part, int* sidx,
                                   float* sval) {
  const int tid = threadIdx.x;
  if (tid < E) keys[tid] = topk_key(v, tid);
  if (tid < K) { sidx[tid] = -1; sval[tid] = -__builtin_inff(); }
  __syncthreads();
  int ep = 1;
  while (ep < E) ep *= 2;
  const int np = NT / ep < 4 ? NT / ep : 4;
  const int c = tid % ep, pi = tid / ep;
  if (pi < np && c < E) {
    const uint64_t kc = keys[c];
    const int span = (E + np - 1) / np;
    const int j0 = pi * span, j1 = j0 + span < E ? j0 + span : E;
    int rank = 0;
    int j = j0;
    for (; j + 2 <= j1 && (j & 1) == 0; j += 2) {
      const ulonglong2 w = reinterpret_cast<const ulonglong2*>(keys)[j / 2];
      rank += (int)(w.x > kc) + (int)(w.y > kc);
    }
    for (; j < j1; ++j) rank += (int)(keys[j] > kc);
    part[tid] = rank;
  }
  __syncthreads();
  if (tid < E) {
    int rank = 0;
    for (int q = 0; q < np; ++q) rank += part[tid + q * ep];
    if (v > -__builtin_inff() && rank < K) {
      sidx[rank] = tid;
      sval[rank] = v;
    }
  }
  __syncthreads();
}

// select_token with the candidates-per-lane count chosen for E (<= 1024).
__device__ __forceinline__ void select_token_any(const float* logit_row, int E, int K,
                                                 uint64_t* keys, int* sidx, float* sval,
                                                 float* sexp, int* idx, float* p, int* idx_user,
                                                 float* p_user) {
  if (E <= 64) select_token<1>(logit_row, E, K, keys, sidx, sval, sexp, idx, p, idx_user, p_user);
  else if (E <= 128) select_token<2>(logit_row, E, K, keys, sidx, sval, sexp, idx, p, idx_user, p_user);
  else if (E <= 256) select_token<4>(logit_row, E, K, keys, sidx, sval, sexp, idx, p, idx_user, p_user);
  else select_token<16>(logit_row, E, K, keys, sidx, sval, sexp, idx, p, idx_user, p_user);
}

}  // namespace moe
