// moe_grouped.hip - the MoE block for many tokens (prefill), expert-major,
// bit-identical to the per-token loop of test_model_trace.c:463-517.
//
// The reference runs three GEMVs per (token, rank) pair and re-reads the
// expert for every pair.  Here every expert's rows are read once per task
// (up to 32, 64 or 256 of its pairs, by block shape) for all the pairs
// routed to it:
//   router      logits[t,e] = sum_k x[t,k] * Wr[e,k], k ascending, one
//               sequential fp32 chain per (token, expert); x staged in LDS,
//               the weights broadcast from registers by DPP (:465-468 ->
//               :213-227); the same blocks then pack the x_norm rows into
//               the int8 limb unit tables of the expert kernels
//   select      one wave per token: top-k by the insertion rule and the
//               softmax gates (:480-487); the x tables' headers
//   group       pairs per expert, offsets, pair ids grouped by expert (a
//               histogram and a permutation of the top-k table) and the
//               task list of the expert kernels: one block, or above 4096
//               pairs a count and a scatter launch over up to 64 blocks
//   gate_up     grouped int8 MFMA GEMM, SwiGLU epilogue (:496-501), h packed
//               into the pairs' unit tables (expert_gemm.hip)
//   down        grouped int8 MFMA GEMM, y per pair (:502-503)
//   combine     out[t] = x_resid[t] + (((0 + p0 y0) + p1 y1) + ...) in rank
//               order (:513, :517)
#include <utility>

#include "moe_device.h"
#include "moe_internal.h"
#include "moe_layer.h"
#include "moe_lib.h"
#include "moe_qtile.h"

namespace moe {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGroupThreads = 1024;
// Pairs up to which one block groups them (group_kernel); above, the
// selection kernel counts the pairs of at most kGroupBlocks grouping blocks
// and group_scatter_kernel scatters them.
constexpr int kGroupOneBlockPairs = 4096;
constexpr int kGroupBatch = 8;   // pair ids per thread in flight in group_kernel
constexpr int kSelectWaves = 4;

// ---------------------------------------------------------------- router

struct RouterTileArgs {
  const float* x;      // [T][D]
  const float* W;      // [E][D]
  const float* b;      // [E] or null
  float* logits;       // [T][E]
  int T, D, E;
  uint8_t* tabs;       // [T] x unit tables (tab_bytes each), packed by the same blocks
  size_t tab_bytes;
  int q4;              // tables for Q4 experts (else Q8)
  uint2* part;         // [token groups][expert groups][16] partial table headers {nl, sum}
  int* hist_zero = nullptr;   // block 0 zeroes hist_n ints here (the selection's pair counts)
  int hist_n = 0;
};

// Router weights reach every lane by DPP row broadcast: within each 16-lane
// row of a wave all lanes work for one expert, lane l holding W[e][k0 + l %
// 16] of a 16-column group, and v_mul_f32_dpp with row_newbcast:i
// multiplies each lane's own x by W[e][k0 + i].
template <int I>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + I, 0xF, 0xF, false));
}

// x is staged as native 4-float vectors: copies of HIP's float4 struct
// are memcpys that keep a register array in scratch memory.
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Block of WPB waves = 16 tokens x 4 * CE * WPB experts: lane l of a wave
// runs the chains of token t0 + l % 16 with the CE experts of its row l /
// 16, so the four rows of a wave read the same x addresses from LDS (the
// LDS serves a repeated address once; with one token per lane the x reads
// bound the kernel).  The 16 x rows stream through two LDS buffers of KC
// columns, each wave's weight groups are loaded one chunk ahead.
template <int CE, int KC, int WPB>
struct RouterShape {
  static constexpr int NT = 64 * WPB;        // threads
  static constexpr int TOK = 16;             // tokens per block
  static constexpr int LD = KC + 4;          // padded x row (floats)
  static constexpr int V4 = KC / 4;          // float4 per row chunk
  static constexpr int NV = TOK * V4 / NT;   // float4 per thread per chunk
  static constexpr int NG = KC / 16;         // weight groups per chunk
  static constexpr int EPB = 4 * CE * WPB;   // experts per block
  static_assert(TOK * V4 % NT == 0, "chunk must split evenly over the block");
};

// The register state of one lane across a chunk: the x values of the
// current and the next 16-column group (X[g % 2]), the products of the
// column in flight (P[j % 2]) and the CE sums.
template <int CE>
struct RouterRegs {
  float X[2][16];
  float P[2][CE];
  float acc[CE];
};

__device__ __forceinline__ void router_read_group(const float* src, float (&xv)[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * q);
    xv[4 * q] = v[0]; xv[4 * q + 1] = v[1]; xv[4 * q + 2] = v[2]; xv[4 * q + 3] = v[3];
  }
}

template <int CE, int I>
__device__ __forceinline__ void router_mul(const float (&w)[CE], float xv, float (&p)[CE]) {
#pragma unroll
  for (int c = 0; c < CE; ++c) p[c] = row_bcast<I>(w[c]) * xv;
}

// The KC columns of a chunk in a fixed software-pipelined order: the
// products of column j + 1 are issued before the sums of column j, so that
// each add waits only on the previous add of its chain, never on its own
// product; the next group's x is read from LDS at the start of a group and
// the staged next chunk is written to LDS halfway through (the compiler's
// scheduler would put every product right before its add: one dependent
// stall and one DPP hazard wait per column).  k ascending in every chain.
template <int CE, int KC, int WPB, int H, int... J>
__device__ __forceinline__ void router_cols(RouterRegs<CE>& r,
                                            const float (&wg)[2][RouterShape<CE, KC, WPB>::NG][CE],
                                            const float* B,
                                            const f32x4 (&rg)[RouterShape<CE, KC, WPB>::NV],
                                            const int (&dst)[RouterShape<CE, KC, WPB>::NV], float* nbuf,
                                            std::integer_sequence<int, J...>) {
  using RS = RouterShape<CE, KC, WPB>;
  (
      [&] {
        constexpr int g = J / 16, i = J % 16;
        if constexpr (i == 0 && g + 1 < RS::NG) router_read_group(B + 16 * (g + 1), r.X[(g + 1) & 1]);
        if constexpr (J == KC / 2) {
#pragma unroll
          for (int v = 0; v < RS::NV; ++v) *reinterpret_cast<f32x4*>(nbuf + dst[v]) = rg[v];
        }
        if constexpr (J + 1 < KC) {
          constexpr int g1 = (J + 1) / 16, i1 = (J + 1) % 16;
          router_mul<CE, i1>(wg[H][g1], r.X[g1 & 1][i1], r.P[(J + 1) & 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < CE; ++c) r.acc[c] = r.acc[c] + r.P[J & 1][c];
        __builtin_amdgcn_sched_barrier(0);
      }(),
      ...);
}

// Chunk cc of the router loop, weight slot H (= cc % 2): the next chunk's
// weights into slot H ^ 1, the KC columns of this chunk from LDS buffer
// cc % 2 (the staged chunk cc + 1 written into the other buffer on the
// way), then the loads of chunk cc + 2 and the block barrier.
template <int CE, int KC, int WPB, int H>
__device__ __forceinline__ void router_chunk(
    const f32x4* const (&srcp)[RouterShape<CE, KC, WPB>::NV],
    const int (&dst)[RouterShape<CE, KC, WPB>::NV], const float* const (&wrow)[CE],
    f32x4 (&rg)[RouterShape<CE, KC, WPB>::NV], float (&wg)[2][RouterShape<CE, KC, WPB>::NG][CE],
    RouterRegs<CE>& r, const float* xr, float* buf, int cc, int nc) {
  using RS = RouterShape<CE, KC, WPB>;
  constexpr int BS = RS::TOK * RS::LD;
  const int nx = min(cc + 1, nc - 1);
#pragma unroll
  for (int g = 0; g < RS::NG; ++g)
#pragma unroll
    for (int c = 0; c < CE; ++c) wg[H ^ 1][g][c] = wrow[c][(size_t)nx * KC + 16 * g];
  const float* B = xr + (cc & 1) * BS;
  router_read_group(B, r.X[0]);
  router_mul<CE, 0>(wg[H][0], r.X[0][0], r.P[0]);
  __builtin_amdgcn_sched_barrier(0);
  router_cols<CE, KC, WPB, H>(r, wg, B, rg, dst, buf + ((cc + 1) & 1) * BS,
                              std::make_integer_sequence<int, KC>{});
  const size_t o = (size_t)min(cc + 2, nc - 1) * RS::V4;
#pragma unroll
  for (int v = 0; v < RS::NV; ++v) rg[v] = srcp[v][o];
  __syncthreads();
}

// The x unit tables of a token group, packed by its router blocks (the x
// rows are in L2 from the router loop; a separate pack launch cost more):
// block eg packs units [eg U / neg, (eg + 1) U / neg) of each of the 16
// tokens (U = D / 16), thread i the units of token i % 16.  The limb counts
// (max) and activation sums (wrapping add) reduce per block into
// part[tg][eg]; select_kernel combines a token's partials into its table
// header (both reductions are order-free; no fence between blocks needed).
template <int NT>
__device__ __forceinline__ void router_pack(const RouterTileArgs& a, int t0, int tg, int eg, int neg) {
  __shared__ int pk_nl[16];
  __shared__ unsigned pk_sum[16];
  const int tid = threadIdx.x, lane = tid % kWave;
  if (tid < 16) { pk_nl[tid] = 1; pk_sum[tid] = 0; }
  __syncthreads();
  const int U = a.D / 16, u0 = eg * U / neg, nu = (eg + 1) * U / neg - u0;
  const int tok = tid % 16, t = t0 + tok;
  int nl = 1;
  uint32_t sum = 0;
  if (t < a.T) {
    const float* xr = a.x + (size_t)t * a.D;
    uint8_t* tab = a.tabs + (size_t)t * a.tab_bytes;
    for (int k = tid / 16; k < nu; k += NT / 16) {
      const int u = u0 + k;
      float v[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 w = reinterpret_cast<const f32x4*>(xr + 16 * u)[q];
        v[4 * q] = w[0]; v[4 * q + 1] = w[1]; v[4 * q + 2] = w[2]; v[4 * q + 3] = w[3];
      }
      if (a.q4) pack_unit16<true>(v, tab, a.D, u, nl, sum);
      else pack_unit16<false>(v, tab, a.D, u, nl, sum);
    }
  }
  // lanes l, l + 16, l + 32, l + 48 hold the same token
#pragma unroll
  for (int off = 16; off < kWave; off *= 2) {
    const int o = __shfl_xor(nl, off, kWave);
    nl = o > nl ? o : nl;
    sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
  }
  if (lane < 16) {
    atomicMax(&pk_nl[tok], nl);
    atomicAdd(&pk_sum[tok], sum);
  }
  __syncthreads();
  if (tid < 16) a.part[((size_t)tg * neg + eg) * 16 + tid] = make_uint2((unsigned)pk_nl[tid], pk_sum[tid]);
}

// Logits of 16 tokens x EPB experts per block (k ascending, :213-227).
// Blocks of one token group share an XCD (block id mod 8), so that its x
// rows come from that XCD's L2 after the first read: blocks 0 .. 8 * NEG *
// (NTG / 8) - 1 map to (token group xcd + 8 * (slot / NEG), expert group
// slot % NEG) with xcd = id % 8, slot = id / 8; the rest (NTG % 8 token
// groups) in row order.  D % KC == 0.
template <int CE, int KC, int WPB>
__global__ __launch_bounds__(64 * WPB) void router_bcast_kernel(RouterTileArgs a) {
  using RS = RouterShape<CE, KC, WPB>;
  extern __shared__ float4 lds4[];
  float* buf = reinterpret_cast<float*>(lds4);   // [2][16][LD]
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int neg = (a.E + RS::EPB - 1) / RS::EPB;
  const int ntg8 = ((a.T + RS::TOK - 1) / RS::TOK) & ~7;
  const int id = blockIdx.x;
  int tg, eg;
  if (id < ntg8 * neg) {
    const int slot = id / 8;
    tg = id % 8 + 8 * (slot / neg);
    eg = slot % neg;
  } else {
    tg = ntg8 + (id - ntg8 * neg) / neg;
    eg = (id - ntg8 * neg) % neg;
  }
  const int t0 = tg * RS::TOK;
  const int eb = eg * RS::EPB + wave * 4 * CE + (lane / 16) * CE;
  const int D = a.D, nc = D / KC;
  const f32x4* srcp[RS::NV];
  int dst[RS::NV];
  const float* wrow[CE];
  f32x4 rg[RS::NV];
  float wg[2][RS::NG][CE];
  RouterRegs<CE> r;
#pragma unroll
  for (int v = 0; v < RS::NV; ++v) {
    const int i = tid + RS::NT * v;
    const int row = i / RS::V4, c4 = i % RS::V4;
    srcp[v] = reinterpret_cast<const f32x4*>(a.x + (size_t)min(t0 + row, a.T - 1) * D) + c4;
    dst[v] = row * RS::LD + 4 * c4;
  }
#pragma unroll
  for (int c = 0; c < CE; ++c) {
    wrow[c] = a.W + (size_t)min(eb + c, a.E - 1) * D + lane % 16;
    r.acc[c] = 0.0f;
  }
  // loads and stores are unconditional (chunk index clamped; a store past
  // the last chunk fills the idle buffer) so the staging stays in registers
#pragma unroll
  for (int v = 0; v < RS::NV; ++v) rg[v] = srcp[v][0];
#pragma unroll
  for (int g = 0; g < RS::NG; ++g)
#pragma unroll
    for (int c = 0; c < CE; ++c) wg[0][g][c] = wrow[c][16 * g];
#pragma unroll
  for (int v = 0; v < RS::NV; ++v) *reinterpret_cast<f32x4*>(buf + dst[v]) = rg[v];
  const size_t o1 = (size_t)min(1, nc - 1) * RS::V4;
#pragma unroll
  for (int v = 0; v < RS::NV; ++v) rg[v] = srcp[v][o1];
  __syncthreads();
  const float* xr = buf + (lane % 16) * RS::LD;
  // two chunks per iteration, so that each weight slot is a fixed register set
  for (int cc = 0;;) {
    router_chunk<CE, KC, WPB, 0>(srcp, dst, wrow, rg, wg, r, xr, buf, cc, nc);
    if (++cc >= nc) break;
    router_chunk<CE, KC, WPB, 1>(srcp, dst, wrow, rg, wg, r, xr, buf, cc, nc);
    if (++cc >= nc) break;
  }
  const int t = t0 + lane % 16;
#pragma unroll
  for (int c = 0; c < CE; ++c) {
    const int e = eb + c;
    if (t < a.T && e < a.E) a.logits[(size_t)t * a.E + e] = a.b ? r.acc[c] + a.b[e] : r.acc[c];
  }
  router_pack<RS::NT>(a, t0, tg, eg, neg);
  if (a.hist_zero && blockIdx.x == 0)
    for (int i = threadIdx.x; i < a.hist_n; i += RS::NT) a.hist_zero[i] = 0;
}

// ---------------------------------------------------------------- select

struct SelectArgs {
  const float* logits;
  int T, E, topk;
  int* idx;
  float* p;
  int* idx_user;
  float* p_user;
  const uint2* part;   // the router blocks' partial x-table headers, or null
  int neg;             // router blocks per token group
  uint8_t* tabs;       // x unit tables
  size_t tab_bytes;
  // optional: pairs per expert of each grouping block (block b takes pairs
  // b * per .. (b + 1) * per - 1), hist[b][E], added here (the router zeroes
  // it) for group_scatter_kernel
  int* hist = nullptr;
  int per = 0;
};

__global__ __launch_bounds__(kSelectWaves * kWave) void select_kernel(SelectArgs a) {
  __shared__ int sidx[kSelectWaves][kMaxTopK];
  __shared__ float sval[kSelectWaves][kMaxTopK];
  __shared__ float sexp[kSelectWaves][kMaxTopK];
  __shared__ ulonglong2 keys2[kSelectWaves][512];   // E <= 1024 keys per wave
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int t = blockIdx.x * kSelectWaves + wave;
  if (t >= a.T) return;
  if (a.part) {
    // the token's x-table header from the router blocks' partials
    const uint2* pp = a.part + (size_t)(t / 16) * a.neg * 16 + t % 16;
    int nl = 1;
    uint32_t sum = 0;
    for (int q = lane; q < a.neg; q += kWave) {
      const uint2 v = pp[(size_t)q * 16];
      nl = (int)v.x > nl ? (int)v.x : nl;
      sum += v.y;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const int o = __shfl_xor(nl, off, kWave);
      nl = o > nl ? o : nl;
      sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
    }
    if (lane == 0) {
      uint8_t* tab = a.tabs + (size_t)t * a.tab_bytes;
      reinterpret_cast<int*>(tab)[0] = nl;
      reinterpret_cast<uint32_t*>(tab)[1] = sum;
    }
  }
  const size_t q = (size_t)t * a.topk;
  select_token_any(a.logits + (size_t)t * a.E, a.E, a.topk, reinterpret_cast<uint64_t*>(keys2[wave]),
                   sidx[wave], sval[wave], sexp[wave], a.idx + q, a.p + q,
                   a.idx_user ? a.idx_user + q : nullptr, a.p_user ? a.p_user + q : nullptr);
  if (a.hist && lane < a.topk) {
    const int e = sidx[wave][lane];
    if (e >= 0) atomicAdd(&a.hist[((int)q + lane) / a.per * a.E + e], 1);
  }
}

// ---------------------------------------------------------------- group

// Exclusive prefix sum of v over the kGroupThreads threads of the block (a
// shuffle scan per wave, then the wave totals); *total gets the sum.
__device__ __forceinline__ int group_excl_scan(int v, int* wsum, int* total) {
  constexpr int NW = kGroupThreads / kWave;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) wsum[w] = x;
  __syncthreads();
  if (w == 0) {
    int t = lane < NW ? wsum[lane] : 0;
#pragma unroll
    for (int off = 1; off < NW; off <<= 1) {
      const int y = __shfl_up(t, off, kWave);
      if (lane >= off) t += y;
    }
    if (lane < NW) wsum[lane] = t;
  }
  __syncthreads();
  *total = wsum[NW - 1];
  const int base = w > 0 ? wsum[w - 1] : 0;
  __syncthreads();   // wsum may be reused
  return base + x - v;
}

// Thread e's expert (c pairs from pair start on, c == 0 past E) in runs of
// at most split pairs: {e | pairs << 16, first pair}, then {-1, 0} up to
// ntask_max.  Every thread of the block calls this.
__device__ __forceinline__ void write_tasks(int c, int start, int* wsum, int2* __restrict__ tasks,
                                            int ntask_max, int split) {
  const int tid = threadIdx.x;
  const int nsplit = (c + split - 1) / split;
  int ntasks;
  const int t0 = group_excl_scan(nsplit, wsum, &ntasks);
  for (int k = 0; k < nsplit; ++k) {
    const int p0 = k * split, n = min(split, c - p0);
    tasks[t0 + k] = make_int2(tid | (n << 16), start + p0);
  }
  for (int i = ntasks + tid; i < ntask_max; i += kGroupThreads) tasks[i] = make_int2(-1, 0);
}

// One block: count the pairs of each expert, exclusive prefix sum, then
// scatter the pair ids.  The order of pairs within an expert does not
// affect any result (every pair's outputs are computed independently).
// Also the tasks of the expert kernels, in expert order: expert e's pairs
// in runs of at most `split`, {e | pairs << 16, first pair}, then {-1, 0}
// up to ntask_max.
__global__ __launch_bounds__(kGroupThreads) void group_kernel(const int* __restrict__ idx,
                                                              int npairs, int E,
                                                              int* __restrict__ ecount,
                                                              int* __restrict__ eoff,
                                                              int* __restrict__ perm,
                                                              int2* __restrict__ tasks,
                                                              int ntask_max, int split) {
  __shared__ int cnt[kGroupThreads];
  __shared__ int wsum[kGroupThreads / kWave];
  // each thread's pair ids are read kGroupBatch at a time, all loads in
  // flight together (one load then its atomic per pair serialised the
  // loop on memory latency)
  constexpr int G = kGroupBatch;
  const int tid = threadIdx.x;
  cnt[tid] = 0;
  __syncthreads();
  for (int base = 0; base < npairs; base += G * kGroupThreads) {
    int e[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int q = base + g * kGroupThreads + tid;
      e[g] = q < npairs ? idx[q] : -1;
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (e[g] >= 0) atomicAdd(&cnt[e[g]], 1);
  }
  __syncthreads();
  const int c = cnt[tid];   // zero past E
  int total;
  const int start = group_excl_scan(c, wsum, &total);
  if (tid < E) {
    ecount[tid] = c;
    eoff[tid] = start;
  }
  if (tasks) write_tasks(c, start, wsum, tasks, ntask_max, split);
  cnt[tid] = start;   // cursor
  __syncthreads();
  for (int base = 0; base < npairs; base += G * kGroupThreads) {
    int e[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int q = base + g * kGroupThreads + tid;
      e[g] = q < npairs ? idx[q] : -1;
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (e[g] >= 0) perm[atomicAdd(&cnt[e[g]], 1)] = base + g * kGroupThreads + tid;
  }
}

// The same grouping over many pairs on nb blocks, block b taking pairs
// b*per .. (b+1)*per - 1 (one atomic per pair on a single block's LDS was
// the cost of group_kernel): select_kernel has added each block's pair
// counts per expert into hist[b][E]; block b starts expert e's cursor at
// start(e) + sum over b' < b of hist[b'][e] and scatters its pairs; block 0
// also writes ecount, eoff and the tasks.
__global__ __launch_bounds__(kGroupThreads) void group_scatter_kernel(
    const int* __restrict__ idx, int npairs, int E, int per, const int* __restrict__ hist, int nb,
    int* __restrict__ ecount, int* __restrict__ eoff, int* __restrict__ perm, int2* __restrict__ tasks,
    int ntask_max, int split) {
  __shared__ int cur[kGroupThreads];
  __shared__ int red[2][kGroupThreads];
  __shared__ int wsum[kGroupThreads / kWave];
  const int tid = threadIdx.x, b = blockIdx.x;
  // expert totals and this block's prefix: G threads per expert read the nb
  // block counts together, then one thread per expert adds their parts
  const int G = kGroupThreads / E, e = tid % E, g = tid / E;
  int c = 0, pre = 0;
  if (g < G) {
#pragma unroll 8
    for (int k = g; k < nb; k += G) {
      const int v = hist[(size_t)k * E + e];
      pre += k < b ? v : 0;
      c += v;
    }
  }
  red[0][tid] = c;
  red[1][tid] = pre;
  __syncthreads();
  c = pre = 0;
  if (tid < E)
    for (int k = 0; k < G; ++k) {
      c += red[0][k * E + tid];
      pre += red[1][k * E + tid];
    }
  int total;
  const int start = group_excl_scan(c, wsum, &total);
  if (b == 0) {
    if (tid < E) {
      ecount[tid] = c;
      eoff[tid] = start;
    }
    write_tasks(c, start, wsum, tasks, ntask_max, split);
  }
  cur[tid] = start + pre;
  __syncthreads();
  const int q0 = b * per, q1 = min(q0 + per, npairs);
  for (int q = q0 + tid; q < q1; q += kGroupThreads) {
    const int e = idx[q];
    if (e >= 0) perm[atomicAdd(&cur[e], 1)] = q;
  }
}

// ---------------------------------------------------------------- combine

// combine_kernel for a fixed top-k: the token's ranks, gates and all K y
// rows requested before the first add (the adds keep the rank order).
template <int K>
__global__ __launch_bounds__(256) void combine_k_kernel(const float* __restrict__ y,
                                                        const int* __restrict__ idx,
                                                        const float* __restrict__ p,
                                                        const float* __restrict__ resid,
                                                        float* __restrict__ out, int D) {
  const int t = blockIdx.y;
  const int o = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (o >= D) return;
  int e[K];
  float pj[K];
  float4 yv[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    e[j] = idx[t * K + j];
    pj[j] = p[t * K + j];
  }
#pragma unroll
  for (int j = 0; j < K; ++j)
    yv[j] = *reinterpret_cast<const float4*>(y + (size_t)(t * K + j) * D + o);
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (e[j] < 0) continue;
    const float a0 = pj[j] * yv[j].x, a1 = pj[j] * yv[j].y, a2 = pj[j] * yv[j].z, a3 = pj[j] * yv[j].w;
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

// One Q4 expert output from the down kernel's int16 dot (y16, -32768: the
// fp32 value is in y instead): ((float)dot / 7) * scale, the operations of
// the down epilogue (kernels.c:125).
__device__ __forceinline__ float y16_value(int16_t v, float s, const float* yrow, int c) {
  return v != -32768 ? qdot_epilogue((uint32_t)(int32_t)v, 7.0f, s) : yrow[c];
}

// combine for Q4 layers: y from the int16 dots and the experts' down row
// scales ds [E][D] (1 MB at E = 128, D = 2048, read from the caches), so
// half the bytes of fp32 y come from memory; same adds in the same order.
// Eight columns a thread: one 16-byte load of a rank's dots, two of its
// scales.  The down kernel marks whole groups of four outputs, so one test
// per group picks the fp32 values.
template <int K>
__global__ __launch_bounds__(256) void combine_y16_k_kernel(const int16_t* __restrict__ y16,
                                                            const float* __restrict__ y,
                                                            const float* __restrict__ ds,
                                                            const int* __restrict__ idx,
                                                            const float* __restrict__ p,
                                                            const float* __restrict__ resid,
                                                            float* __restrict__ out, int D) {
  const int t = blockIdx.y;
  const int o = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (o >= D) return;
  int e[K];
  float pj[K];
  uint4 yv[K];
  float4 s0[K], s1[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    e[j] = idx[t * K + j];
    pj[j] = p[t * K + j];
  }
#pragma unroll
  for (int j = 0; j < K; ++j)
    yv[j] = *reinterpret_cast<const uint4*>(y16 + (size_t)(t * K + j) * D + o);
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const float4* sr = reinterpret_cast<const float4*>(ds + (size_t)(e[j] >= 0 ? e[j] : 0) * D + o);
    s0[j] = sr[0];
    s1[j] = sr[1];
  }
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < K; ++j) {
    if (e[j] < 0) continue;
    const uint32_t w[4] = {yv[j].x, yv[j].y, yv[j].z, yv[j].w};
    const float sc[8] = {s0[j].x, s0[j].y, s0[j].z, s0[j].w, s1[j].x, s1[j].y, s1[j].z, s1[j].w};
    float v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int16_t d = (int16_t)((w[c / 2] >> (16 * (c % 2))) & 0xFFFFu);
      v[c] = qdot_epilogue((uint32_t)(int32_t)d, 7.0f, sc[c]);
    }
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      if (w[2 * g] == 0x80008000u) {
        const float4 f = *reinterpret_cast<const float4*>(y + (size_t)(t * K + j) * D + o + 4 * g);
        v[4 * g] = f.x; v[4 * g + 1] = f.y; v[4 * g + 2] = f.z; v[4 * g + 3] = f.w;
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float a = pj[j] * v[c];
      acc[c] = acc[c] + a;
    }
  }
  const size_t oi = (size_t)t * D + o;
  if (resid) {
    const float4 r0 = *reinterpret_cast<const float4*>(resid + oi);
    const float4 r1 = *reinterpret_cast<const float4*>(resid + oi + 4);
    acc[0] = r0.x + acc[0]; acc[1] = r0.y + acc[1]; acc[2] = r0.z + acc[2]; acc[3] = r0.w + acc[3];
    acc[4] = r1.x + acc[4]; acc[5] = r1.y + acc[5]; acc[6] = r1.z + acc[6]; acc[7] = r1.w + acc[7];
  }
  *reinterpret_cast<float4*>(out + oi) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  *reinterpret_cast<float4*>(out + oi + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

__global__ __launch_bounds__(256) void combine_y16_kernel(const int16_t* __restrict__ y16,
                                                          const float* __restrict__ y,
                                                          const float* __restrict__ ds,
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
    const int e = idx[q];
    if (e < 0) continue;
    const float pj = p[q];
    const uint2 yv = *reinterpret_cast<const uint2*>(y16 + (size_t)q * D + o);
    const float4 sv = *reinterpret_cast<const float4*>(ds + (size_t)e * D + o);
    const float* yrow = y + (size_t)q * D + o;
    const float y0 = y16_value((int16_t)(yv.x & 0xFFFFu), sv.x, yrow, 0);
    const float y1 = y16_value((int16_t)(yv.x >> 16), sv.y, yrow, 1);
    const float y2 = y16_value((int16_t)(yv.y & 0xFFFFu), sv.z, yrow, 2);
    const float y3 = y16_value((int16_t)(yv.y >> 16), sv.w, yrow, 3);
    const float a0 = pj * y0, a1 = pj * y1, a2 = pj * y2, a3 = pj * y3;
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

bool is16(const void* p) { return ((uintptr_t)p % 16) == 0; }

template <int CE, int KC, int WPB>
moe_status launch_router_bcast(const RouterTileArgs& a, hipStream_t s) {
  using RS = RouterShape<CE, KC, WPB>;
  constexpr size_t lds = 2 * (size_t)RS::TOK * RS::LD * 4;
  static_assert(lds <= 65536, "router LDS");
  const unsigned blocks = (unsigned)(((a.T + RS::TOK - 1) / RS::TOK) * ((a.E + RS::EPB - 1) / RS::EPB));
  hipLaunchKernelGGL((router_bcast_kernel<CE, KC, WPB>), dim3(blocks), dim3(RS::NT), lds, s, a);
  return check_hip(hipGetLastError(), "router launch");
}

// Waves per router block: eight from 1024 tokens, four from 256, two below
// (measured at E = 128, D = 2048), fewer where the block would hold more
// experts than the layer.
moe_status launch_router(const RouterTileArgs& a, hipStream_t s, int* neg) {
  int wpb = a.T >= 1024 ? 8 : a.T >= 256 ? 4 : 2;
  while (wpb > 1 && 4 * wpb > a.E) wpb /= 2;
  *neg = (a.E + 4 * wpb - 1) / (4 * wpb);
  switch (wpb) {
    case 8: return launch_router_bcast<1, 128, 8>(a, s);
    case 4: return launch_router_bcast<1, 128, 4>(a, s);
    case 2: return launch_router_bcast<1, 128, 2>(a, s);
    default: return launch_router_bcast<1, 128, 1>(a, s);
  }
}

}  // namespace

moe_status launch_select(const LayerDev* L, int T, int32_t* idx_out, float* p_out, hipStream_t s,
                         const uint2* xpart, int neg, int* hist, int per) {
  SelectArgs sa{L->logits, T, L->E, L->topk, L->idx, L->p, idx_out, p_out,
                xpart, neg, L->xtab, act_table_bytes(L->D)};
  sa.hist = hist;
  sa.per = per;
  dim3 sg((unsigned)((T + kSelectWaves - 1) / kSelectWaves));
  hipLaunchKernelGGL(select_kernel, sg, dim3(kSelectWaves * kWave), 0, s, sa);
  return check_hip(hipGetLastError(), "select launch");
}

bool grouped_ok(const LayerDev* L) {
  // router chunks of 128 columns; expert kernel stages of 64 weight bytes
  return L->D % 128 == 0 && expert_gemm_ok(L) && L->E <= kGroupThreads && is16(L->router_w);
}

moe_status layer_forward_grouped(LayerDev* L, const float* xn, const float* resid, int T,
                                 float* out, int32_t* idx_out, float* p_out) {
  hipStream_t s = stream();
  moe_status st;
  if (!is16(xn) || !is16(out) || (resid && !is16(resid)))
    return set_error(MOE_ERR_ARG, "grouped forward: arrays must be 16-byte aligned");
  // 1-2. router logits (one sequential chain per lane) and, in the same
  // blocks, the x unit tables of the expert kernels
  const int npairs = T * L->topk;
  // many pairs: the grouping runs on nb blocks of `per` pairs; the selection
  // counts each block's pairs per expert into ghist (zeroed by the router)
  const bool two = npairs > kGroupOneBlockPairs;
  const int nb = std::min(kGroupBlocks, (npairs + 255) / 256);
  const int per = (npairs + nb - 1) / nb;
  RouterTileArgs ra{xn, L->router_w, L->router_b, L->logits, T, L->D, L->E,
                    L->xtab, act_table_bytes(L->D), L->dtype == 3, L->rpart};
  if (two) {
    ra.hist_zero = L->ghist;
    ra.hist_n = nb * L->E;
  }
  int neg = 0;
  if ((st = launch_router(ra, s, &neg))) return st;
  // 3. top-k and gates; the x tables' headers; the grouping blocks' counts
  if ((st = launch_select(L, T, idx_out, p_out, s, L->rpart, neg, two ? L->ghist : nullptr, per)))
    return st;
  // 4. group pairs by expert, tasks of at most one block's pairs
  const int nt = expert_gemm_tiles(L, T);
  const int split = expert_gemm_split(nt);
  const int ntask_max = npairs / split + L->E + 1;
  if (!two) {
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(kGroupThreads), 0, s, L->idx, npairs, L->E,
                       L->ecount, L->eoff, L->perm, L->tasks, ntask_max, split);
  } else {
    hipLaunchKernelGGL(group_scatter_kernel, dim3((unsigned)nb), dim3(kGroupThreads), 0, s, L->idx, npairs,
                       L->E, per, L->ghist, nb, L->ecount, L->eoff, L->perm, L->tasks, ntask_max, split);
  }
  if ((st = check_hip(hipGetLastError(), "group launch"))) return st;
  // 5-6. gate/up + SwiGLU, down: grouped GEMMs on the 32x32x32 int8 MFMA
  if ((st = launch_expert_gemm(L, nt, ntask_max, s))) return st;
  // 7. ordered combine + residual
  dim3 cg((unsigned)((L->D / 4 + 255) / 256), (unsigned)T);
  if (L->y16 && L->topk == 8 && L->D % 8 == 0)
    hipLaunchKernelGGL(combine_y16_k_kernel<8>, dim3((unsigned)((L->D / 8 + 255) / 256), (unsigned)T), dim3(256), 0,
                       s, L->y16, L->y, L->ds, L->idx, L->p, resid, out, L->D);
  else if (L->y16)
    hipLaunchKernelGGL(combine_y16_kernel, cg, dim3(256), 0, s, L->y16, L->y, L->ds, L->idx, L->p, resid, out,
                       L->D, L->topk);
  else if (L->topk == 8)
    hipLaunchKernelGGL(combine_k_kernel<8>, cg, dim3(256), 0, s, L->y, L->idx, L->p, resid, out, L->D);
  else
    hipLaunchKernelGGL(combine_kernel, cg, dim3(256), 0, s, L->y, L->idx, L->p, resid, out, L->D,
                       L->topk);
  return check_hip(hipGetLastError(), "combine launch");
}

}  // namespace moe
