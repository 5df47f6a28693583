// moe_layer.h - device state of one MoE layer and the routing helpers shared
// by the decode kernels (moe_layer.hip) and the grouped multi-token kernels
// (moe_grouped.hip).  Internal; the public ABI is include/moehip.h.
#pragma once
#include <stdint.h>

#include "moe_device.h"
#include "moe_lib.h"

namespace moe {

constexpr int kMaxTopK = 32;

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
  // grouped kernels: pairs per expert, first pair of each expert in `perm`,
  // pair ids (t * topk + j) grouped by expert, expert outputs per pair
  int* ecount = nullptr;     // [E]
  int* eoff = nullptr;       // [E]
  int* perm = nullptr;       // [T*topk]
  float* y = nullptr;        // [T*topk][D]
  unsigned* sel_counter = nullptr;   // block counter of the fused selection
};

// Top-k and softmax gates of T tokens from L->logits into L->idx / L->p
// (and the caller's copies, when given): one wave per token.
moe_status launch_select(const LayerDev* L, int T, int32_t* idx_out, float* p_out, hipStream_t s);

// Grouped (expert-major) forward for many tokens; requires grouped_ok(L).
bool grouped_ok(const LayerDev* L);
moe_status layer_forward_grouped(LayerDev* L, const float* xn, const float* resid, int T,
                                 float* out, int32_t* idx_out, float* p_out);

// ---- routing: top-k by the insertion rule, softmax over the selection ----

// (v, i) beats (w, j): valid and larger, or equal with the lower index.
__device__ __forceinline__ bool beats(float v, int i, float w, int j) {
  if (i < 0) return false;
  if (j < 0) return true;
  return v > w || (v == w && i < j);
}

template <int CTRL>
__device__ __forceinline__ void argmax_step_dpp(float& bv, int& bi) {
  const float ov = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bv), CTRL, 0xF, 0xF, true));
  const int oi = __builtin_amdgcn_update_dpp(-1, bi, CTRL, 0xF, 0xF, false);
  if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
}

// Wave-wide arg-max of (value, index) pairs under `beats`; every lane ends
// with the winner.  DPP within rows of 16, then two cross-row exchanges.
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
  argmax_step_dpp<0xB1>(bv, bi);    // quad_perm [1,0,3,2]
  argmax_step_dpp<0x4E>(bv, bi);    // quad_perm [2,3,0,1]
  argmax_step_dpp<0x141>(bv, bi);   // row_half_mirror
  argmax_step_dpp<0x140>(bv, bi);   // row_mirror
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
}

// One wave selects the experts of one token and their gates:
//   top-k by repeated arg-max (the largest remaining logit, lowest index
//   among equals) = the insertion rule of test_model_trace.c:275-288; NaN
//   and -inf never selected, slots left over keep index -1;
//   p_i = expf(v_i - max) / (sum + 1e-9f), sum in slot order (:482-487).
// C = candidates per lane (E <= 64*C).  sidx/sval/sexp: this wave's LDS
// slots (kMaxTopK each).  Outputs are per-token rows of K entries; the user
// copies may be null.
template <int C>
__device__ void select_token(const float* __restrict__ logit_row, int E, int K, int* sidx,
                             float* sval, float* sexp, int* idx, float* p, int* idx_user,
                             float* p_user) {
  const int lane = threadIdx.x % kWave;
  float v[C];
  bool live[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int e = lane + kWave * c;
    v[c] = e < E ? logit_row[e] : -__builtin_inff();
    live[c] = e < E && v[c] > -__builtin_inff();   // false for NaN and -inf
  }
  for (int r = 0; r < K; ++r) {
    float bv = -__builtin_inff();
    int bi = -1;
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (live[c] && beats(v[c], lane + kWave * c, bv, bi)) { bv = v[c]; bi = lane + kWave * c; }
    wave_argmax(bv, bi);
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (bi == lane + kWave * c) live[c] = false;
    if (lane == 0) { sidx[r] = bi; sval[r] = bi >= 0 ? bv : -__builtin_inff(); }
  }
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
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

// Block-wide selection for one token (any block size, E <= 1024): every
// thread ranks its candidates among all E logits, rank = number of live
// logits that beat it (larger, or equal with a lower index; NaN and -inf
// are never live), and a live candidate with rank < K takes slot `rank`.
// This is the result of the insertion rule of test_model_trace.c:275-288
// (ties keep the lower index first, NaN / -inf never enter, leftover slots
// keep index -1), computed without a serial pass.  Then wave 0 forms the
// softmax over the slots (:482-487) as select_token does.  sv: LDS scratch
// of E floats, 16-byte aligned; all threads of the block must call this.
__device__ __forceinline__ void select_token_block(const float* __restrict__ logit_row, int E,
                                                  int K, float* sv, int* sidx, float* sval,
                                                  float* sexp, int* idx, float* p,
                                                  int* idx_user, float* p_user) {
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int e = tid; e < E; e += nt) sv[e] = logit_row[e];
  if (tid < K) { sidx[tid] = -1; sval[tid] = -__builtin_inff(); }
  __syncthreads();
  for (int i = tid; i < E; i += nt) {
    const float vi = sv[i];
    if (!(vi > -__builtin_inff())) continue;
    // w beats vi iff w > vi, or w == vi at a lower index; NaN and -inf
    // never beat a live vi, so no liveness test is needed for w
    int rank = 0;
    int j = 0;
    const float4* sv4 = reinterpret_cast<const float4*>(sv);
    for (; j + 32 <= E; j += 32) {
      float4 w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = sv4[j / 4 + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int jj = j + 4 * u;
        rank += (int)((w[u].x > vi) | ((w[u].x == vi) & (jj < i)));
        rank += (int)((w[u].y > vi) | ((w[u].y == vi) & (jj + 1 < i)));
        rank += (int)((w[u].z > vi) | ((w[u].z == vi) & (jj + 2 < i)));
        rank += (int)((w[u].w > vi) | ((w[u].w == vi) & (jj + 3 < i)));
      }
    }
    for (; j < E; ++j) {
      const float w = sv[j];
      rank += (int)((w > vi) | ((w == vi) & (j < i)));
    }
    if (rank < K) { sidx[rank] = i; sval[rank] = vi; }
  }
  __syncthreads();
  if (tid < kWave) {
    const int lane = tid;
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
  }
  __syncthreads();
}

}  // namespace moe
