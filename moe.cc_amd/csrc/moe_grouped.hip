// moe_grouped.hip - the MoE block for many tokens (prefill), expert-major,
// bit-identical to the per-token loop of test_model_trace.c:463-517.
//
// The reference runs three GEMVs per (token, rank) pair and re-reads the
// expert for every pair.  Here every expert's rows are read once per launch
// for all the pairs routed to it:
//   act_pack    x_norm rows -> packed limb tables (gemv.hip)
//   router      logits[t,e] = sum_k x[t,k] * Wr[e,k], k ascending, one
//               sequential fp32 chain per (token, expert) over LDS-staged
//               chunks (:465-468 -> :213-227)
//   select      one wave per token: top-k by the insertion rule and the
//               softmax gates (:480-487)
//   group       one block: pairs per expert, offsets, pair ids grouped by
//               expert (a histogram and a permutation of the top-k table)
//   gate_up     per (expert, 128 rows of d_ff): gate and up rows streamed
//               once, int8 MFMA over 16-pair tiles of that expert's pairs,
//               then h = silu(g) * u (:496-501) packed into the pair's table
//   down        per (expert, 128 rows of D): y = Q(h Wd) (:502-503) per pair
//   combine     out[t] = x_resid[t] + (((0 + p0 y0) + p1 y1) + ...) in rank
//               order (:513, :517)
//
// The integer dots are exact in any order, so MFMA tiles (16 rows x 16
// pairs x 64 columns of v_mfma_i32_16x16x64_i8) change nothing: a quantized
// activation a is split into int8 limbs a = sum_l b_l 256^l (one MFMA pass
// per limb), Q4 weights enter as unsigned nibbles u = w + 8 with the offset
// removed once per output (sum a*w = sum a*u - 8 * sum a), and the fp32
// epilogues are the reference's operations in the reference's order.
//
// MFMA operand layout (checked on gfx950): lane l supplies row (A) or column
// (B) l % 16 and 16 bytes of the k-group l / 16; byte b of A lane i + 16g
// meets byte b of B lane j + 16g.  Result register r of lane l is row
// 4 * (l / 16) + r, column l % 16.  Which columns a (group, byte) slot
// stands for is this file's choice, made identically for both operands:
//   Q8: a 128-column step, lane group g covers columns 32g .. 32g + 31,
//       slice s (0, 1) of them columns 32g + 16s .. + 15 in order;
//   Q4: a 256-column step, lane group g covers columns 64g .. 64g + 63,
//       slice s (0..3) columns c0 = 64g + 16s .. c0 + 15 as bytes
//       [c0, c0+2, .., c0+14, c0+1, c0+3, .., c0+15] (low nibbles, then high
//       nibbles, of the 8 packed weight bytes; the even and odd planes of the
//       activation table hold the same columns in the same order).
#include <algorithm>
#include <cstdlib>

#include "moe_device.h"
#include "moe_internal.h"
#include "moe_layer.h"
#include "moe_lib.h"
#include "moe_qtile.h"

namespace moe {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGroupThreads = 1024;
constexpr int kMmaWaves = 8;                  // waves per expert block
constexpr int kMmaThreads = kMmaWaves * kWave;
constexpr int kMmaRows = kMmaWaves * 16;      // output rows per expert block
constexpr int kPairsPerPass = 64;             // 4 tiles of 16 pairs
constexpr int kSelectWaves = 4;

// ---------------------------------------------------------------- router

struct RouterTileArgs {
  const float* x;      // [T][D]
  const float* W;      // [E][D]
  const float* b;      // [E] or null
  float* logits;       // [T][E]
  int T, D, E;
};

// Logits of a tile of 16*CT tokens x 16*CE experts.  Thread (ti, ei) owns
// tokens t0 + ti + 16c and experts e0 + ei + 16c: CT*CE sequential chains,
// k ascending, every product and sum rounded on its own.  x and W rows
// stream through two LDS chunk buffers of KC columns, the next-but-one
// chunk held in registers while the current one is consumed.  D % KC == 0.
template <int CT, int CE, int KC>
__global__ __launch_bounds__(256) void router_tile_kernel(RouterTileArgs a) {
  constexpr int RX = 16 * CT, RW = 16 * CE, R = RX + RW;
  constexpr int LD = KC + 4;                      // padded row (floats)
  constexpr int V4 = KC / 4;                      // float4 per row chunk
  constexpr int NV = R * V4 / 256;                // float4 per thread per chunk
  static_assert(R * V4 % 256 == 0, "chunk must split evenly over the block");
  extern __shared__ float4 lds4[];
  float* buf = reinterpret_cast<float*>(lds4);    // [2][R][LD]
  const int tid = threadIdx.x;
  const int ti = tid / 16, ei = tid % 16;
  const int t0 = blockIdx.y * RX, e0 = blockIdx.x * RW;
  const int D = a.D;
  const int nc = D / KC;
  // this thread's 4 staging slots: source (float4 units) and LDS offsets
  static_assert(NV == 4, "staging is written for 4 float4 per thread");
  const float4* srcp[4];
  int dst[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int i = tid + 256 * v;
    const int row = i / V4, c4 = i % V4;
    const float* base = row < RX ? a.x + (size_t)min(t0 + row, a.T - 1) * D
                                 : a.W + (size_t)min(e0 + row - RX, a.E - 1) * D;
    srcp[v] = reinterpret_cast<const float4*>(base) + c4;
    dst[v] = row * LD + 4 * c4;
  }
  float4 r0, r1, r2, r3;
#define ROUTER_LOAD(c)                                                         \
  {                                                                            \
    const size_t o_ = (size_t)(c) * V4;                                        \
    r0 = srcp[0][o_]; r1 = srcp[1][o_]; r2 = srcp[2][o_]; r3 = srcp[3][o_];    \
  }
#define ROUTER_STORE(bsel)                                                     \
  {                                                                            \
    float* b_ = buf + (bsel) * R * LD;                                         \
    *reinterpret_cast<float4*>(b_ + dst[0]) = r0;                              \
    *reinterpret_cast<float4*>(b_ + dst[1]) = r1;                              \
    *reinterpret_cast<float4*>(b_ + dst[2]) = r2;                              \
    *reinterpret_cast<float4*>(b_ + dst[3]) = r3;                              \
  }
  float acc[CT][CE];
#pragma unroll
  for (int i = 0; i < CT; ++i)
#pragma unroll
    for (int j = 0; j < CE; ++j) acc[i][j] = 0.0f;
  // loads and stores are unconditional (chunk index clamped; a store past
  // the last chunk fills the idle buffer) so `reg` stays in registers
  ROUTER_LOAD(0)
  ROUTER_STORE(0)
  ROUTER_LOAD(min(1, nc - 1))
  __syncthreads();
  for (int c = 0; c < nc; ++c) {
    const float* B = buf + (c & 1) * R * LD;
    const float* xr[CT];
    const float* wr[CE];
#pragma unroll
    for (int i = 0; i < CT; ++i) xr[i] = B + (ti + 16 * i) * LD;
#pragma unroll
    for (int j = 0; j < CE; ++j) wr[j] = B + (RX + ei + 16 * j) * LD;
#pragma unroll 4
    for (int k = 0; k < KC; k += 4) {
      float4 xv[CT], wv[CE];
#pragma unroll
      for (int i = 0; i < CT; ++i) xv[i] = *reinterpret_cast<const float4*>(xr[i] + k);
#pragma unroll
      for (int j = 0; j < CE; ++j) wv[j] = *reinterpret_cast<const float4*>(wr[j] + k);
#pragma unroll
      for (int i = 0; i < CT; ++i)
#pragma unroll
        for (int j = 0; j < CE; ++j) {
          const float p0 = xv[i].x * wv[j].x, p1 = xv[i].y * wv[j].y;
          const float p2 = xv[i].z * wv[j].z, p3 = xv[i].w * wv[j].w;
          float s = acc[i][j];
          s = s + p0;
          s = s + p1;
          s = s + p2;
          s = s + p3;
          acc[i][j] = s;
        }
    }
    ROUTER_STORE((c + 1) & 1)
    ROUTER_LOAD(min(c + 2, nc - 1))
    __syncthreads();
  }
#undef ROUTER_LOAD
#undef ROUTER_STORE
#pragma unroll
  for (int i = 0; i < CT; ++i)
#pragma unroll
    for (int j = 0; j < CE; ++j) {
      const int t = t0 + ti + 16 * i, e = e0 + ei + 16 * j;
      if (t < a.T && e < a.E) a.logits[(size_t)t * a.E + e] = a.b ? acc[i][j] + a.b[e] : acc[i][j];
    }
}

// ---------------------------------------------------------------- select

struct SelectArgs {
  const float* logits;
  int T, E, topk;
  int* idx;
  float* p;
  int* idx_user;
  float* p_user;
};

template <int C>
__global__ __launch_bounds__(kSelectWaves * kWave) void select_kernel(SelectArgs a) {
  __shared__ int sidx[kSelectWaves][kMaxTopK];
  __shared__ float sval[kSelectWaves][kMaxTopK];
  __shared__ float sexp[kSelectWaves][kMaxTopK];
  const int wave = threadIdx.x / kWave;
  const int t = blockIdx.x * kSelectWaves + wave;
  if (t >= a.T) return;
  const size_t q = (size_t)t * a.topk;
  select_token<C>(a.logits + (size_t)t * a.E, a.E, a.topk, sidx[wave], sval[wave], sexp[wave],
                  a.idx + q, a.p + q, a.idx_user ? a.idx_user + q : nullptr,
                  a.p_user ? a.p_user + q : nullptr);
}

// ---------------------------------------------------------------- group

// One block: count the pairs of each expert, exclusive prefix sum, then
// scatter the pair ids.  The order of pairs within an expert does not
// affect any result (every pair's outputs are computed independently).
__global__ __launch_bounds__(kGroupThreads) void group_kernel(const int* __restrict__ idx,
                                                              int npairs, int E,
                                                              int* __restrict__ ecount,
                                                              int* __restrict__ eoff,
                                                              int* __restrict__ perm) {
  __shared__ int cnt[kGroupThreads];
  __shared__ int scan[kGroupThreads];
  const int tid = threadIdx.x;
  cnt[tid] = 0;
  __syncthreads();
  for (int q = tid; q < npairs; q += kGroupThreads) {
    const int e = idx[q];
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // inclusive scan (Hillis-Steele) over the E <= 1024 counts
  scan[tid] = cnt[tid];
  __syncthreads();
  for (int off = 1; off < kGroupThreads; off <<= 1) {
    const int v = tid >= off ? scan[tid - off] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  const int start = scan[tid] - cnt[tid];
  if (tid < E) {
    ecount[tid] = cnt[tid];
    eoff[tid] = start;
  }
  __syncthreads();
  cnt[tid] = start;   // cursor
  __syncthreads();
  for (int q = tid; q < npairs; q += kGroupThreads) {
    const int e = idx[q];
    if (e >= 0) perm[atomicAdd(&cnt[e], 1)] = q;
  }
}

// ---------------------------------------------------------------- MFMA core

__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Columns per step and slices per step of one lane group (see file header).
template <bool Q4> struct Step {
  static constexpr int COLS = Q4 ? 256 : 128;   // columns per step
  static constexpr int SL = Q4 ? 4 : 2;         // 16-column slices per lane group
};

// Weight fragment of one step for one matrix: 32 bytes of the lane's row.
struct WFrag {
  u32x4 w[2];
};

template <bool Q4>
__device__ __forceinline__ WFrag load_wfrag(const uint8_t* row, int step, int g) {
  // Q8: columns step*128 + 32g .. +31 = bytes at the same offset;
  // Q4: columns step*256 + 64g .. +63 = bytes step*128 + 32g .. +31
  const u32x4* p = reinterpret_cast<const u32x4*>(row + (size_t)step * 128 + 32 * g);
  WFrag f;
  f.w[0] = __builtin_nontemporal_load(p);
  f.w[1] = __builtin_nontemporal_load(p + 1);
  return f;
}

// A operand of slice s.
template <bool Q4>
__device__ __forceinline__ v4i a_slice(const WFrag& f, int s) {
  v4i r;
  if constexpr (!Q4) {
    const u32x4 w = f.w[s];
    r[0] = (int)w[0]; r[1] = (int)w[1]; r[2] = (int)w[2]; r[3] = (int)w[3];
  } else {
    const u32x4 w = f.w[s >> 1];
    const uint32_t w0 = (s & 1) ? w[2] : w[0];
    const uint32_t w1 = (s & 1) ? w[3] : w[1];
    constexpr uint32_t M = 0x0F0F0F0Fu;
    r[0] = (int)(w0 & M);
    r[1] = (int)(w1 & M);
    r[2] = (int)((w0 >> 4) & M);
    r[3] = (int)((w1 >> 4) & M);
  }
  return r;
}

// B operand of slice s, limb l, from one activation table (K columns).
template <bool Q4>
__device__ __forceinline__ v4i b_slice(const uint8_t* tab, int K, int l, int step, int g, int s) {
  const uint8_t* plane = reinterpret_cast<const uint8_t*>(act_plane(tab, K, l));
  v4i r;
  if constexpr (!Q4) {
    const uint4 v = *reinterpret_cast<const uint4*>(plane + (size_t)step * 128 + 32 * g + 16 * s);
    r[0] = (int)v.x; r[1] = (int)v.y; r[2] = (int)v.z; r[3] = (int)v.w;
  } else {
    const int c0 = step * 256 + 64 * g + 16 * s;
    const uint2 e = *reinterpret_cast<const uint2*>(plane + c0 / 2);
    const uint2 o = *reinterpret_cast<const uint2*>(plane + K / 2 + c0 / 2);
    r[0] = (int)e.x; r[1] = (int)e.y; r[2] = (int)o.x; r[3] = (int)o.y;
  }
  return r;
}

// acc[m][tt][l] += W_m[rows] x tables[tt] over all K columns, for NM weight
// matrices (gate, up) sharing the activations, nt live 16-pair tiles (of NT)
// and NL limbs.  W[m] points at this lane's row.  Weights are prefetched
// one step ahead.
template <bool Q4, int NM, int NL, int NT>
__device__ __forceinline__ void mma_rows(const uint8_t* const W[NM], int K,
                                         const uint8_t* const tab[NT], int nt,
                                         v4i acc[NM][NT][NL]) {
  const int g = (threadIdx.x % kWave) / 16;
  const int nsteps = K / Step<Q4>::COLS;
  WFrag cur[NM], nxt[NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) cur[m] = load_wfrag<Q4>(W[m], 0, g);
  for (int st = 0; st < nsteps; ++st) {
    if (st + 1 < nsteps) {
#pragma unroll
      for (int m = 0; m < NM; ++m) nxt[m] = load_wfrag<Q4>(W[m], st + 1, g);
    }
#pragma unroll
    for (int s = 0; s < Step<Q4>::SL; ++s) {
      v4i av[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) av[m] = a_slice<Q4>(cur[m], s);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        if (tt >= nt) break;
#pragma unroll
        for (int l = 0; l < NL; ++l) {
          const v4i bv = b_slice<Q4>(tab[tt], K, l, st, g, s);
#pragma unroll
          for (int m = 0; m < NM; ++m) acc[m][tt][l] = mfma16(av[m], bv, acc[m][tt][l]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < NM; ++m) cur[m] = nxt[m];
  }
}

template <int NL>
__device__ __forceinline__ uint32_t limb_dot(const v4i* acc_l, int r) {
  int32_t v[4] = {0, 0, 0, 0};
#pragma unroll
  for (int l = 0; l < NL; ++l) v[l] = acc_l[l][r];
  return combine_limbs<NL == 3 ? 4 : NL>(v);
}

// Pair of column j of tile tt in a pass over an expert's pairs, or -1.
__device__ __forceinline__ int pass_pair(const int* perm, int first, int n, int idx) {
  return idx < n ? perm[first + idx] : -1;
}

// ---------------------------------------------------------------- gate/up

struct GateUpGArgs {
  const uint8_t* gq; const float* gs; const uint8_t* uq; const float* us;
  long long rb; int D, dff, topk;
  const int* ecount; const int* eoff; const int* perm;
  const uint8_t* xtab; size_t xtab_bytes;
  uint8_t* htab; size_t htab_bytes;
  uint32_t* hpart;   // [pair][nseg][2]
  int nseg;
};

// Tiles tile0 .. tile0 + NT - 1 of a pass over up to 64 of expert e's pairs.
template <bool Q4, int NL, int NT>
__device__ void gate_up_pass(const GateUpGArgs& a, int e, int first, int n, int tile0,
                             uint32_t xsum_lane, int* red_nl, unsigned* red_sum) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 16, j = lane % 16;
  const int rowA = blockIdx.x * kMmaRows + wave * 16 + j;   // this lane's A row
  const int rowA_c = rowA < a.dff ? rowA : a.dff - 1;
  const uint8_t* W[2] = {a.gq + ((size_t)e * a.dff + rowA_c) * a.rb,
                         a.uq + ((size_t)e * a.dff + rowA_c) * a.rb};
  const int nt = min(NT, (n - tile0 * 16 + 15) / 16);
  const uint8_t* tab[NT];
  int pair[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    pair[tt] = pass_pair(a.perm, first, n, (tile0 + tt) * 16 + j);
    const int q = pair[tt] >= 0 ? pair[tt] : a.perm[first];
    tab[tt] = a.xtab + (size_t)(q / a.topk) * a.xtab_bytes;
  }
  v4i acc[2][NT][NL];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int l = 0; l < NL; ++l) acc[m][tt][l] = v4i{0, 0, 0, 0};
  mma_rows<Q4, 2, NL, NT>(W, a.D, tab, nt, acc);
  const float div = Q4 ? 7.0f : 127.0f;
  const int rbase = blockIdx.x * kMmaRows + wave * 16 + 4 * g;   // rows of this lane's results
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    if (tt >= nt) break;
    const int q = pair[tt];
    const int col = (tile0 + tt) * 16 + j;   // pair index within the pass
    // activation sum of this column's token (Q4 offset correction)
    const uint32_t xs = (uint32_t)__shfl((int)xsum_lane, col, kWave);
    int nl = 1;
    uint32_t hs = 0;
    uint32_t bytes[4][4];   // [limb][r]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = rbase + r;
      uint32_t dg = limb_dot<NL>(acc[0][tt], r);
      uint32_t du = limb_dot<NL>(acc[1][tt], r);
      if (Q4) { dg -= 8u * xs; du -= 8u * xs; }
      int32_t hv = 0;
      if (q >= 0 && row < a.dff) {
        const float gv = qdot_epilogue(dg, div, a.gs[(size_t)e * a.dff + row]);
        const float uv = qdot_epilogue(du, div, a.us[(size_t)e * a.dff + row]);
        const float h = silu_mul(gv, uv);
        hv = f2i_trunc_x86(h * div);
      }
      const int nn = limbs_needed(hv);
      nl = nn > nl ? nn : nl;
      hs += (uint32_t)hv;
      uint32_t b[4];
      split_limbs(hv, b);
#pragma unroll
      for (int l = 0; l < 4; ++l) bytes[l][r] = b[l];
    }
    if (q >= 0 && rbase < a.dff) {
      uint8_t* tabq = a.htab + (size_t)q * a.htab_bytes;
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        uint8_t* plane = reinterpret_cast<uint8_t*>(const_cast<uint32_t*>(act_plane(tabq, a.dff, l)));
        if constexpr (!Q4) {
          *reinterpret_cast<uint32_t*>(plane + rbase) =
              pack4(bytes[l][0], bytes[l][1], bytes[l][2], bytes[l][3]);
        } else {
          *reinterpret_cast<uint16_t*>(plane + rbase / 2) =
              (uint16_t)(bytes[l][0] | (bytes[l][2] << 8));
          *reinterpret_cast<uint16_t*>(plane + a.dff / 2 + rbase / 2) =
              (uint16_t)(bytes[l][1] | (bytes[l][3] << 8));
        }
      }
    }
    // partial header of this block's rows for the column's pair: reduce the
    // 4 lane groups, then the waves through LDS
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const int on = __shfl_xor(nl, off, kWave);
      nl = on > nl ? on : nl;
      hs += (uint32_t)__shfl_xor((int)hs, off, kWave);
    }
    if (g == 0 && q >= 0) {
      atomicMax(&red_nl[col], nl);
      atomicAdd(&red_sum[col], hs);
    }
  }
}

template <bool Q4>
__global__ __launch_bounds__(kMmaThreads) void gate_up_grouped_kernel(GateUpGArgs a) {
  __shared__ int red_nl[kPairsPerPass];
  __shared__ unsigned red_sum[kPairsPerPass];
  const int e = blockIdx.y;
  const int n_all = a.ecount[e];
  if (n_all == 0) return;
  const int first_all = a.eoff[e];
  const int lane = threadIdx.x % kWave;
  for (int p0 = 0; p0 < n_all; p0 += kPairsPerPass) {
    const int n = min(kPairsPerPass, n_all - p0);
    const int first = first_all + p0;
    // limb count (max) and activation sums of the pass's tokens: lane i <-> pair i
    int nl = 1;
    uint32_t xsum = 0;
    if (lane < n) {
      const int q = a.perm[first + lane];
      const uint8_t* tb = a.xtab + (size_t)(q / a.topk) * a.xtab_bytes;
      nl = act_nl(tb);
      xsum = act_asum(tb);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int on = __shfl_xor(nl, off, kWave);
      nl = on > nl ? on : nl;
    }
    if (threadIdx.x < kPairsPerPass) { red_nl[threadIdx.x] = 1; red_sum[threadIdx.x] = 0; }
    __syncthreads();
    if (nl == 1) {
      gate_up_pass<Q4, 1, 4>(a, e, first, n, 0, xsum, red_nl, red_sum);
    } else if (nl == 2) {
      gate_up_pass<Q4, 2, 4>(a, e, first, n, 0, xsum, red_nl, red_sum);
    } else {   // four limbs: two tiles at a time keeps the accumulators in registers
      gate_up_pass<Q4, 4, 2>(a, e, first, n, 0, xsum, red_nl, red_sum);
      if (n > 32) gate_up_pass<Q4, 4, 2>(a, e, first, n, 2, xsum, red_nl, red_sum);
    }
    __syncthreads();
    if (threadIdx.x < n) {
      const int q = a.perm[first + threadIdx.x];
      uint32_t* pp = a.hpart + ((size_t)q * a.nseg + blockIdx.x) * 2;
      pp[0] = (uint32_t)red_nl[threadIdx.x];
      pp[1] = red_sum[threadIdx.x];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- down

struct DownGArgs {
  const uint8_t* dq; const float* ds;
  long long rb; int D, dff;
  const int* ecount; const int* eoff; const int* perm;
  const uint8_t* htab; size_t htab_bytes;
  const uint32_t* hpart; int nseg;
  float* y;            // [pair][D]
};

template <bool Q4, int NL, int NT>
__device__ void down_pass(const DownGArgs& a, int e, int first, int n, int tile0,
                          uint32_t hsum_lane) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 16, j = lane % 16;
  const int rowA = blockIdx.x * kMmaRows + wave * 16 + j;
  const int rowA_c = rowA < a.D ? rowA : a.D - 1;
  const uint8_t* W[1] = {a.dq + ((size_t)e * a.D + rowA_c) * a.rb};
  const int nt = min(NT, (n - tile0 * 16 + 15) / 16);
  const uint8_t* tab[NT];
  int pair[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    pair[tt] = pass_pair(a.perm, first, n, (tile0 + tt) * 16 + j);
    const int q = pair[tt] >= 0 ? pair[tt] : a.perm[first];
    tab[tt] = a.htab + (size_t)q * a.htab_bytes;
  }
  v4i acc[1][NT][NL];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int l = 0; l < NL; ++l) acc[0][tt][l] = v4i{0, 0, 0, 0};
  mma_rows<Q4, 1, NL, NT>(W, a.dff, tab, nt, acc);
  const float div = Q4 ? 7.0f : 127.0f;
  const int rbase = blockIdx.x * kMmaRows + wave * 16 + 4 * g;
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    if (tt >= nt) break;
    const int q = pair[tt];
    const uint32_t hs = (uint32_t)__shfl((int)hsum_lane, (tile0 + tt) * 16 + j, kWave);
    if (q < 0 || rbase >= a.D) continue;
    float yv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t d = limb_dot<NL>(acc[0][tt], r);
      if (Q4) d -= 8u * hs;
      yv[r] = qdot_epilogue(d, div, a.ds[(size_t)e * a.D + rbase + r]);
    }
    *reinterpret_cast<float4*>(a.y + (size_t)q * a.D + rbase) = make_float4(yv[0], yv[1], yv[2], yv[3]);
  }
}

template <bool Q4>
__global__ __launch_bounds__(kMmaThreads) void down_grouped_kernel(DownGArgs a) {
  const int e = blockIdx.y;
  const int n_all = a.ecount[e];
  if (n_all == 0) return;
  const int first_all = a.eoff[e];
  const int lane = threadIdx.x % kWave;
  for (int p0 = 0; p0 < n_all; p0 += kPairsPerPass) {
    const int n = min(kPairsPerPass, n_all - p0);
    const int first = first_all + p0;
    // limb count and activation sum of each pair's h: reduce its segments
    int nl = 1;
    uint32_t hsum = 0;
    if (lane < n) {
      const int q = a.perm[first + lane];
      for (int s = 0; s < a.nseg; ++s) {
        const uint32_t* pp = a.hpart + ((size_t)q * a.nseg + s) * 2;
        nl = (int)pp[0] > nl ? (int)pp[0] : nl;
        hsum += pp[1];
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int on = __shfl_xor(nl, off, kWave);
      nl = on > nl ? on : nl;
    }
    if (nl == 1) {
      down_pass<Q4, 1, 4>(a, e, first, n, 0, hsum);
    } else if (nl == 2) {
      down_pass<Q4, 2, 4>(a, e, first, n, 0, hsum);
    } else {
      down_pass<Q4, 4, 2>(a, e, first, n, 0, hsum);
      if (n > 32) down_pass<Q4, 4, 2>(a, e, first, n, 2, hsum);
    }
  }
}

// ---------------------------------------------------------------- combine

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y,
                                                      const int* __restrict__ idx,
                                                      const float* __restrict__ p,
                                                      const float* __restrict__ resid,
                                                      float* __restrict__ out, int D, int topk) {
  const int t = blockIdx.y;
  const int o = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (o >= D) return;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int jj = 0; jj < topk; ++jj) {
    const int q = t * topk + jj;
    if (idx[q] < 0) continue;
    const float pj = p[q];
    const float4 yv = *reinterpret_cast<const float4*>(y + (size_t)q * D + o);
    const float a0 = pj * yv.x, a1 = pj * yv.y, a2 = pj * yv.z, a3 = pj * yv.w;
    acc.x = acc.x + a0;
    acc.y = acc.y + a1;
    acc.z = acc.z + a2;
    acc.w = acc.w + a3;
  }
  const size_t oi = (size_t)t * D + o;
  if (resid) {
    const float4 rv = *reinterpret_cast<const float4*>(resid + oi);
    acc = make_float4(rv.x + acc.x, rv.y + acc.y, rv.z + acc.z, rv.w + acc.w);
  }
  *reinterpret_cast<float4*>(out + oi) = acc;
}

template <class T>
moe_status galloc(T** p, size_t count) {
  *p = nullptr;
  if (count == 0) return MOE_OK;
  return check_hip(hipMalloc((void**)p, count * sizeof(T)), "hipMalloc(grouped)");
}

bool is16(const void* p) { return ((uintptr_t)p % 16) == 0; }

template <int CT, int CE, int KC>
moe_status launch_router_tile(const RouterTileArgs& a, hipStream_t s) {
  constexpr size_t lds = 2 * (size_t)(16 * CT + 16 * CE) * (KC + 4) * 4;
  static bool attr_set = false;
  if (lds > 65536 && !attr_set) {
    moe_status st = check_hip(hipFuncSetAttribute((const void*)router_tile_kernel<CT, CE, KC>,
                                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  (int)lds),
                              "router tile LDS attribute");
    if (st) return st;
    attr_set = true;
  }
  dim3 grid((unsigned)((a.E + 16 * CE - 1) / (16 * CE)), (unsigned)((a.T + 16 * CT - 1) / (16 * CT)));
  hipLaunchKernelGGL((router_tile_kernel<CT, CE, KC>), grid, dim3(256), lds, s, a);
  return check_hip(hipGetLastError(), "router tile launch");
}

}  // namespace

bool grouped_ok(const LayerDev* L) {
  const int step = L->dtype == 3 ? 256 : 128;
  return L->D % step == 0 && L->dff % step == 0 && L->D % 128 == 0 && L->E <= kGroupThreads &&
         is16(L->router_w);
}

moe_status ensure_grouped_scratch(LayerDev* L, int T) {
  // grown together with the decode scratch (capT), see ensure_scratch
  moe_status st;
  const size_t np = (size_t)T * L->topk;
  if (!L->ecount && (st = galloc(&L->ecount, (size_t)L->E))) return st;
  if (!L->eoff && (st = galloc(&L->eoff, (size_t)L->E))) return st;
  if (L->perm) (void)hipFree(L->perm);
  if (L->y) (void)hipFree(L->y);
  L->perm = nullptr;
  L->y = nullptr;
  if ((st = galloc(&L->perm, np))) return st;
  if ((st = galloc(&L->y, np * L->D))) return st;
  return MOE_OK;
}

moe_status layer_forward_grouped(LayerDev* L, const float* xn, const float* resid, int T,
                                 float* out, int32_t* idx_out, float* p_out) {
  hipStream_t s = stream();
  const bool q4 = L->dtype == 3;
  moe_status st;
  if (!is16(xn) || !is16(out) || (resid && !is16(resid)))
    return set_error(MOE_ERR_ARG, "grouped forward: arrays must be 16-byte aligned");
  // 1. x tables
  QShape sh;
  sh.dtype = L->dtype; sh.M = T; sh.N = 1; sh.K = L->D; sh.lda = L->D; sh.ldc = 1;
  sh.rs = L->rbg;
  QJob one{nullptr, nullptr, xn, nullptr};
  if ((st = check_hip(launch_act_pack(sh, nullptr, one, 1, L->xtab, s), "act pack"))) return st;
  // 2. router logits
  RouterTileArgs ra{xn, L->router_w, L->router_b, L->logits, T, L->D, L->E};
  if (T >= 512) st = launch_router_tile<2, 2, 64>(ra, s);
  else st = launch_router_tile<1, 1, 128>(ra, s);
  if (st) return st;
  // 3. top-k and gates
  SelectArgs sa{L->logits, T, L->E, L->topk, L->idx, L->p, idx_out, p_out};
  dim3 sg((unsigned)((T + kSelectWaves - 1) / kSelectWaves));
  if (L->E <= 64) hipLaunchKernelGGL(select_kernel<1>, sg, dim3(kSelectWaves * kWave), 0, s, sa);
  else if (L->E <= 128) hipLaunchKernelGGL(select_kernel<2>, sg, dim3(kSelectWaves * kWave), 0, s, sa);
  else if (L->E <= 256) hipLaunchKernelGGL(select_kernel<4>, sg, dim3(kSelectWaves * kWave), 0, s, sa);
  else hipLaunchKernelGGL(select_kernel<16>, sg, dim3(kSelectWaves * kWave), 0, s, sa);
  if ((st = check_hip(hipGetLastError(), "select launch"))) return st;
  // 4. group pairs by expert
  const int npairs = T * L->topk;
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(kGroupThreads), 0, s, L->idx, npairs, L->E,
                     L->ecount, L->eoff, L->perm);
  if ((st = check_hip(hipGetLastError(), "group launch"))) return st;
  // 5. gate/up + SwiGLU
  const int nseg = (L->dff + kMmaRows - 1) / kMmaRows;
  GateUpGArgs ga{L->gq, L->gs, L->uq, L->us, L->rbg, L->D, L->dff, L->topk,
                 L->ecount, L->eoff, L->perm, L->xtab, act_table_bytes(L->D),
                 L->htab, act_table_bytes(L->dff), L->hpart, nseg};
  dim3 gg((unsigned)nseg, (unsigned)L->E);
  if (q4) hipLaunchKernelGGL(gate_up_grouped_kernel<true>, gg, dim3(kMmaThreads), 0, s, ga);
  else hipLaunchKernelGGL(gate_up_grouped_kernel<false>, gg, dim3(kMmaThreads), 0, s, ga);
  if ((st = check_hip(hipGetLastError(), "grouped gate/up launch"))) return st;
  // 6. down
  DownGArgs da{L->dq, L->ds, L->rbd, L->D, L->dff, L->ecount, L->eoff, L->perm,
               L->htab, act_table_bytes(L->dff), L->hpart, nseg, L->y};
  dim3 dg((unsigned)((L->D + kMmaRows - 1) / kMmaRows), (unsigned)L->E);
  if (q4) hipLaunchKernelGGL(down_grouped_kernel<true>, dg, dim3(kMmaThreads), 0, s, da);
  else hipLaunchKernelGGL(down_grouped_kernel<false>, dg, dim3(kMmaThreads), 0, s, da);
  if ((st = check_hip(hipGetLastError(), "grouped down launch"))) return st;
  // 7. ordered combine + residual
  dim3 cg((unsigned)((L->D / 4 + 255) / 256), (unsigned)T);
  hipLaunchKernelGGL(combine_kernel, cg, dim3(256), 0, s, L->y, L->idx, L->p, resid, out, L->D,
                     L->topk);
  return check_hip(hipGetLastError(), "combine launch");
}

}  // namespace moe
