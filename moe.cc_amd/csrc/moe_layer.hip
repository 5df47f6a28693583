// moe_layer.hip - the MoE block of one Qwen3-MoE layer on gfx950
// (test_model_trace.c:460-517), bit-identical to the reference.
//
// Launch sequence of one forward (T tokens):
//   [rmsnorm]   x_norm = rmsnorm(x, rms2_w)          (block forward only; :461)
//   act_pack    x_norm rows -> packed limb tables for the expert GEMVs
//   router      logits[t,e] = sum_k x_norm[t,k] * Wr[e,k], k ascending,
//               separate roundings (:465 -> :213-227), + bias (:466-468):
//               the exact fp32 products of dense.hip
//   select      top-k by the insertion rule (:480 -> :275-288) and the
//               softmax over the selected logits (:482-487), a wave per token
//               (in the router launch's last block for few tokens)
//   gate_up     per (token, rank) pair and row chunk: g = Q(x Wg), u = Q(x Wu),
//               exact integer dots; h = (g / (1 + expf(-g))) * u (:496-501),
//               written straight into the pair's packed table for down.
//   down        per token and row chunk, one wave per rank: y_j = Q(h_j Wd_j)
//               (:502-503) into LDS, then out = x_resid + (((0 + p0 y0) +
//               p1 y1) + ...) in rank order, each product and sum rounded on
//               its own (:513, :517).
// Cross-block hand-offs go through kernel boundaries, never through
// per-block device fences.  These kernels serve few tokens (decode); many
// tokens go through the expert-major kernels of moe_grouped.hip.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <type_traits>
#include <vector>

#include "dense.h"
#include "moe_device.h"
#include "moe_internal.h"
#include "moe_layer.h"
#include "moe_lib.h"
#include "moe_qtile.h"

namespace moe {

namespace {

constexpr int kCombineThreads = 512;           // 8 waves
constexpr int kCombineWaves = kCombineThreads / kWave;
constexpr size_t kMaxLds = 160 * 1024 - 2048;  // dynamic LDS budget (static LDS fits in the rest)

// Marks the untiled expert path: one wave per row, int32 arithmetic on the
// fp32 activations (any row size; used for small or irregular layers).
struct GenericGeom {
  static constexpr int WR = 1;
};

// Epilogue of gate/up: hb[row - r0] = silu(g) * u  (LDS)
struct GateUpEpi {
  const float* gs;
  const float* us;
  float* hb;
  int r0;
  float div;
  using Pre = float2;
  __device__ Pre pre(int row) const { return make_float2(gs[row], us[row]); }
  template <class Tot>
  __device__ void operator()(int row, const Tot& tot, float2 sc) const {
    const float g = qdot_epilogue(tot[0][0], div, sc.x);
    const float u = qdot_epilogue(tot[1][0], div, sc.y);
    hb[row - r0] = silu_mul(g, u);
  }
  template <class Tot>
  __device__ void operator()(int row, const Tot& tot) const { (*this)(row, tot, pre(row)); }
};
struct GateUpEpiMaker {
  GateUpEpi e;
  template <int MTI>
  __device__ GateUpEpi at(int) const { return e; }
};

// Block -> (row chunk r, item q) of an nr x nq launch (1-D grid) so that
// all items of one row chunk run on one XCD (blocks are dealt to the 8 XCDs
// in turn) one after another: pairs or tokens that share an expert then
// read its rows of that chunk from HBM once and from that XCD's L2 after.
// Row chunks past the last multiple of 8 go in row order.
__device__ __forceinline__ void xcd_chunk_item(int nr, int nq, int* r, int* q) {
  const int L = blockIdx.x, nr8 = nr & ~7;
  if (L < nr8 * nq) {
    const int slot = L / 8;
    *r = (slot / nq) * 8 + L % 8;
    *q = slot % nq;
  } else {
    const int k = L - nr8 * nq;
    *r = nr8 + k / nq;
    *q = k % nq;
  }
}

struct GateUpArgs {
  const uint8_t* gq; const float* gs; const uint8_t* uq; const float* us;
  long long rb; int D, dff, topk;
  const int* idx; const uint8_t* xtab; size_t tab_bytes; const float* xn;
  float* h; uint8_t* htab; size_t htab_bytes;
  uint32_t* hpart;      // [pair][chunk][2] partial (limbs, sum) of each row chunk of h
  int nchunks, rows_per_block;
  int npairs;           // the launch is nchunks x npairs blocks (xcd_chunk_item)
  // SEL (E <= kTileBlock): the selection is made here, from the router
  // logits and the x tables' nxpart partial headers (token t's partial of
  // slice b at uint2 index t * xp_tok + b * xp_slice); p and the caller's
  // copies (may be null) get the gates
  const float* logits = nullptr;
  const uint32_t* xpart = nullptr;
  int nxpart = 0, E = 0;
  int xp_tok = 0, xp_slice = 1;
  int* idx_w = nullptr;
  float* p = nullptr;
  int32_t* idx_user = nullptr;
  float* p_user = nullptr;
};

// gate/up + SwiGLU for one (token, rank) pair and one row chunk:
// h = (g / (1 + expf(-g))) * u with g, u exact (:496-501).  h is written as
// fp32 and, packed, into its rows of the pair's table for the down GEMV; the
// chunk's limb count and activation sum go to hpart (no atomics).  Row chunks
// start at multiples of 8, so a chunk owns whole packed dwords.
// SEL (decode): every block ranks its token's E logits itself
// (block_select_slots) and takes the expert of its slot; it also reduces the
// router blocks' partial headers of the token's x table (the largest limb
// count, the wrapping sum), so no kernel runs between the router and this
// one.  The block of the token's rank 0 and row chunk 0 writes the token's
// selection and gates (select_gates) and its x table's header.
// Tagged copies of gate/up's outputs for the one-token gate/up + down
// launch, and that launch's tag: an epoch that the router launch before it
// advances (so every launch, graph replays included, has its own tag and a
// word left from an earlier launch never passes for a current one -- the
// 32-bit epoch would come round again only after 2^32 launches, ~4 days of
// continuous decode, and every launch rewrites the words it reads).
struct FuseTags {
  uint64_t* tab = nullptr;     // [pair][4 planes][pw] the h tables' plane dwords
  uint64_t* h = nullptr;       // [pair][dff] fp32 h (for the exact fallback)
  uint64_t* part = nullptr;    // [pair][pchunks][2] each row chunk's {limbs}, {sum}
  const uint32_t* epoch = nullptr;
  int pw = 0;                  // dwords per plane (act table layout)
  int pchunks = 0;             // chunk stride of part
  long long wait_ticks = 0;    // longest wait, wall-clock ticks
};

template <bool Q4, class G, bool SEL, bool NT>
__device__ __forceinline__ void gate_up_block(const GateUpArgs& a, int rc, int q, float* hb,
                                              const FuseTags* ft, uint32_t tag) {
  __shared__ int red[2];   // limb count, activation sum
  const int t = q / a.topk;
  int e;
  int x_nl = 0;
  // the token's activation sum, handed to the row streaming by address: in
  // LDS (a local array whose address is taken would live in scratch memory)
  __shared__ uint32_t x_sum[1];
  if constexpr (SEL) {
    __shared__ __align__(16) uint64_t keys[kTileBlock];
    __shared__ int part[kTileBlock];
    __shared__ int sidx[kMaxTopK];
    __shared__ float sval[kMaxTopK], sexp[kMaxTopK];
    __shared__ int xred[2];
    const int tid = threadIdx.x;
    // both loads first: the logits and the partial headers
    const float v = tid < a.E ? a.logits[(size_t)t * a.E + tid] : -__builtin_inff();
    uint2 pp = make_uint2(1u, 0u);
    if (tid < a.nxpart)
      pp = reinterpret_cast<const uint2*>(a.xpart)[(size_t)t * a.xp_tok + (size_t)tid * a.xp_slice];
    if (tid == 0) { xred[0] = 1; xred[1] = 0; }
    block_select_slots<kTileBlock>(v, a.E, a.topk, keys, part, sidx, sval);
    block_max_sum((int)pp.x, pp.y, xred);
    __syncthreads();
    // (no partials: the table's header was written by its own pack kernel)
    x_nl = a.nxpart > 0 ? xred[0] : 0;
    x_sum[0] = (uint32_t)xred[1];   // every thread stores the same value before reading it
    const int j = q - t * a.topk;
    e = sidx[j];
    if (rc == 0 && j == 0) {
      const size_t o = (size_t)t * a.topk;
      if (tid < kWave)
        select_gates(a.topk, sidx, sval, sexp, a.idx_w + o, a.p + o, a.idx_user ? a.idx_user + o : nullptr,
                     a.p_user ? a.p_user + o : nullptr);
      if (tid == 0 && a.nxpart > 0) {
        uint32_t* hh = reinterpret_cast<uint32_t*>(const_cast<uint8_t*>(a.xtab) + (size_t)t * a.tab_bytes);
        hh[0] = (uint32_t)x_nl;
        hh[1] = (uint32_t)xred[1];
      }
    }
  } else {
    e = a.idx[q];
  }
  if (e < 0) return;
  const int r0 = rc * a.rows_per_block;
  const int r1 = r0 + a.rows_per_block < a.dff ? r0 + a.rows_per_block : a.dff;
  const uint8_t* W[2] = {a.gq + (size_t)e * a.dff * a.rb, a.uq + (size_t)e * a.dff * a.rb};
  const uint8_t* tabs[1] = {a.xtab + (size_t)t * a.tab_bytes};
  const float* xs[1] = {a.xn + (size_t)t * a.D};
  GateUpEpiMaker mk{GateUpEpi{a.gs + (size_t)e * a.dff, a.us + (size_t)e * a.dff, hb, r0,
                              Q4 ? 7.0f : 127.0f}};
  if (threadIdx.x == 0) { red[0] = 1; red[1] = 0; }
  if constexpr (std::is_same<G, GenericGeom>::value) {
    auto epi = mk.e;
    generic_rows_fp32<Q4, 2>(W, a.rb, a.D, xs[0], r0, r1, epi);
  } else {
    stream_tokens<Q4, G, 2, 1, NT>(W, a.rb, a.D, tabs, xs, 1, r0, r1, mk, x_nl,
                                   x_nl > 0 ? x_sum : nullptr);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < r1 - r0; i += blockDim.x) {
    a.h[(size_t)q * a.dff + r0 + i] = hb[i];
    if (ft) tag_put(ft->h + (size_t)q * a.dff + r0 + i, tag, __float_as_uint(hb[i]));
  }
  int nl;
  uint32_t sum;
  pack_act_cols<Q4>(hb - r0, a.dff, r0, r1, a.htab + (size_t)q * a.htab_bytes, threadIdx.x,
                    blockDim.x, nl, sum, ft ? ft->tab + (size_t)q * 4 * ft->pw : nullptr, tag);
  block_max_sum(nl, sum, red);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* pp = a.hpart + ((size_t)q * a.nchunks + rc) * 2;
    pp[0] = (uint32_t)red[0];
    pp[1] = (uint32_t)red[1];
    if (ft) {
      uint64_t* tp = ft->part + ((size_t)q * ft->pchunks + rc) * 2;
      tag_put(tp, tag, (uint32_t)red[0]);
      tag_put(tp + 1, tag, (uint32_t)red[1]);
    }
  }
}

template <bool Q4, class G, bool SEL, bool NT>
__global__ __launch_bounds__(kTileBlock) void gate_up_kernel(GateUpArgs a) {
  extern __shared__ float hb[];   // [rows_per_block]
  int rc, q;
  xcd_chunk_item(a.nchunks, a.npairs, &rc, &q);
  gate_up_block<Q4, G, SEL, NT>(a, rc, q, hb, nullptr, 0u);
}

struct DownArgs {
  const uint8_t* dq; const float* ds; long long rb; int T, D, dff, topk;
  const int* idx; const float* p; const uint8_t* htab; size_t tab_bytes; const float* h;
  const uint32_t* hpart; int nchunks;
  const float* resid; float* out; int rows_per_block;
  int nrc;   // row chunks: the launch is nrc x T blocks (xcd_chunk_item)
};

// Epilogue of down: yb[j][row - r0] = Q(h_j Wd_j)  (LDS)
struct DownEpi {
  const float* ds;
  float* yb;
  int r0;
  float div;
  using Pre = float;
  __device__ Pre pre(int row) const { return ds[row]; }
  template <class Tot>
  __device__ void operator()(int row, const Tot& tot, float sc) const {
    yb[row - r0] = qdot_epilogue(tot[0][0], div, sc);
  }
  template <class Tot>
  __device__ void operator()(int row, const Tot& tot) const { (*this)(row, tot, ds[row]); }
};
struct DownEpiMaker {
  DownEpi e;
  template <int MTI>
  __device__ DownEpi at(int) const { return e; }
};

// down + weighted sum for one token and one row chunk: wave w computes
// y_j for ranks j = w, w+8, ... into LDS; then out[t, o] = x_resid +
// (((0 + p0 y0) + p1 y1) + ...) in rank order (test_model_trace.c:502-517).
// NT: nontemporal weight loads; false from down_cached_min_tokens() tokens
// up, where tokens routed to one expert read its rows again.
template <bool Q4, class G, bool NT>
__global__ __launch_bounds__(kCombineThreads) void down_combine_kernel(DownArgs a) {
  extern __shared__ float yb[];   // [topk][rows_per_block]
  int rc, t;
  xcd_chunk_item(a.nrc, a.T, &rc, &t);
  const int r0 = rc * a.rows_per_block;
  const int r1 = r0 + a.rows_per_block < a.D ? r0 + a.rows_per_block : a.D;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (int j = wave; j < a.topk; j += kCombineWaves) {
    const int q = t * a.topk + j;
    const int e = a.idx[q];
    if (e < 0) continue;
    const uint8_t* W[1] = {a.dq + (size_t)e * a.D * a.rb};
    const uint8_t* tab = a.htab + (size_t)q * a.tab_bytes;
    const float* x = a.h + (size_t)q * a.dff;
    DownEpiMaker mk{DownEpi{a.ds + (size_t)e * a.D, yb + (size_t)j * a.rows_per_block, r0,
                            Q4 ? 7.0f : 127.0f}};
    if constexpr (std::is_same<G, GenericGeom>::value) {
      auto epi = mk.e;
      generic_rows_fp32_wave<Q4, 1>(W, a.rb, a.dff, x, r0, r1, epi);
    } else {
      // limb count and activation sum of h: reduce the gate/up chunk partials
      int nl = 1;
      uint32_t sum = 0;
      for (int c = lane; c < a.nchunks; c += kWave) {
        const uint32_t* pp = a.hpart + ((size_t)q * a.nchunks + c) * 2;
        nl = (int)pp[0] > nl ? (int)pp[0] : nl;
        sum += pp[1];
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const int on = __shfl_xor(nl, off, kWave);
        nl = on > nl ? on : nl;
        sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
      }
      stream_row_wave<Q4, G, 1, NT>(W, a.rb, a.dff, tab, x, r0, r1, mk, nl, sum);
    }
  }
  __syncthreads();
  for (int o = r0 + threadIdx.x; o < r1; o += blockDim.x) {
    float acc = 0.0f;
    for (int j = 0; j < a.topk; ++j) {
      const int q = t * a.topk + j;
      if (a.idx[q] < 0) continue;
      const float py = a.p[q] * yb[(size_t)j * a.rows_per_block + (o - r0)];
      acc = acc + py;
    }
    const size_t oi = (size_t)t * a.D + o;
    a.out[oi] = a.resid ? a.resid[oi] + acc : acc;
  }
}

// ---- one token: gate/up and down in one launch ----
//
// Blocks [0, ngu) are the gate/up blocks of gate_up_kernel<SEL> (the same
// selection, rows, tables and partial headers, each also stored as tagged
// words); blocks [ngu, ngu + nrc) are down blocks of G::WR output rows,
// 256 threads, wave w taking ranks w and w + 4.  A down block makes the
// token's selection itself (the gate/up blocks' rule on the same logits),
// requests its experts' weight rows and scales, and only then waits for
// the tagged words: each pair's chunk partials (limb count, activation sum),
// then the table dwords its lanes multiply -- straight into registers -- or,
// for activations past the register budget, the fp32 h (exact fallback).
// The combine is down_combine_kernel's (rank order, one rounding per
// product and sum).  Every down block comes after every gate/up block in
// the grid, and blocks are dispatched in order, so the blocks it waits on
// are running or done; a wait still ends at a deadline, and a block that
// hit one writes NaN rows instead of a result.
struct FuseArgs {
  GateUpArgs gu;
  DownArgs dn;
  FuseTags ft;
  int ngu;
};
constexpr int kFuseTopK = 8;   // ranks of the fused launch (two a wave)
constexpr int kFusePlaneWords = 3;   // table dwords a lane per plane: d_ff <= 768

template <bool Q4, class G>
__device__ void down_fused_block(const FuseArgs& f, int rc, uint32_t tag, float* lds) {
  const DownArgs& a = f.dn;
  constexpr int NWV = kTileWaves;
  constexpr int JP = kFuseTopK / NWV;   // ranks per wave
  __shared__ __align__(16) uint64_t keys[kTileBlock];
  __shared__ int part[kTileBlock];
  __shared__ int sidx[kFuseTopK], gidx[kFuseTopK];
  __shared__ float sval[kFuseTopK], sexp[kFuseTopK], gp[kFuseTopK];
  __shared__ int late_any;
  float* yb = lds;                         // [kFuseTopK][G::WR]
  uint32_t* tabl = reinterpret_cast<uint32_t*>(lds + kFuseTopK * G::WR);   // [kFuseTopK][2][pw]
  float* hx = lds + kFuseTopK * G::WR + kFuseTopK * 2 * f.ft.pw;   // [topk][dff] fallback h
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const long long deadline = wall_clock64() + f.ft.wait_ticks;
  const int r0 = rc * G::WR, r1 = min(r0 + G::WR, a.D);
  const int g = lane / G::LPR, r = lane % G::LPR;
  const int row = r0 + g;
  const float v = tid < f.gu.E ? f.gu.logits[tid] : -__builtin_inff();
  // the residual rows now, not after the waits
  const float rv = a.resid && r0 + tid < r1 ? a.resid[r0 + tid] : 0.0f;
  if (tid == 0) late_any = 0;
  block_select_slots<kTileBlock>(v, f.gu.E, a.topk, keys, part, sidx, sval);
  __syncthreads();
  if (wave == 0) select_gates(a.topk, sidx, sval, sexp, gidx, gp, nullptr, nullptr);
  // the weight rows and scales of this wave's ranks first
  uint32_t w[JP][G::DW];
  float sc[JP];
  int ej[JP];
#pragma unroll
  for (int i = 0; i < JP; ++i) {
    const int j = wave + NWV * i;
    ej[i] = j < a.topk ? sidx[j] : -1;
    if (ej[i] >= 0 && row < r1) {
      load_row_regs<G, true>(a.dq + ((size_t)ej[i] * a.D + row) * (size_t)a.rb, w[i]);
      sc[i] = a.ds[(size_t)ej[i] * a.D + row];
    } else {
#pragma unroll
      for (int d = 0; d < G::DW; ++d) w[i][d] = 0;
      sc[i] = 0.0f;
    }
  }
  // Waiting: first one thread polls a single probe word (the last chunk
  // partial of one rank) with long sleeps -- the gate/up blocks all run at
  // once, so when it is there the rest nearly are -- then each wave fetches
  // both of its ranks' chunk partials and the table dwords its lanes
  // multiply (Q4 one limb plane, Q8 two) in one batch, polling again only
  // what is stale.  (Every lane polling everything from the start floods
  // the memory system under the gate/up weight streams.)
  bool late = false;
  const bool any = sidx[0] >= 0;   // rank 0 is live unless every logit is NaN or -inf
  if (any && tid == 0) {
    int pj = rc % a.topk;
    if (sidx[pj] < 0) pj = 0;
    const uint64_t* pr = f.ft.part + ((size_t)pj * f.ft.pchunks + f.gu.nchunks - 1) * 2;
    uint32_t pv[1];
    tag_wait_all<1, 10>([&](int) { return pr; }, pv, tag, deadline, late);
    if (late) late_any = 1;
  }
  __syncthreads();
  if (late_any) late = true;
  const int K = a.dff, KW = (K + 7) / 8, pw = f.ft.pw;
  const int nw = Q4 ? 2 * KW : (K + 3) / 4;   // plane dwords the gate/up blocks write
  const float div = Q4 ? 7.0f : 127.0f;
  constexpr int NLF = Q4 ? 1 : 2;                 // limb planes fetched up front
  constexpr int NWD = 4 + NLF * kFusePlaneWords;  // words a lane per rank
  uint32_t tv[JP * NWD];
  if (any) {
    tag_wait_all<JP * NWD>(
        [&](int i2) {
          const int ip = i2 / NWD, u = i2 % NWD;
          const int jj = ej[ip] >= 0 ? wave + NWV * ip : 0;   // dead rank: rank 0's words, unused
          if (u < 4) {   // chunks lane and lane + 64 (clamped to the last)
            const int c = lane + kWave * (u / 2);
            return f.ft.part + ((size_t)jj * f.ft.pchunks + (c < f.gu.nchunks ? c : f.gu.nchunks - 1)) * 2 +
                   u % 2;
          }
          const int l = (u - 4) / kFusePlaneWords, t = (u - 4) % kFusePlaneWords;
          const int dw = lane + kWave * t;
          return f.ft.tab + ((size_t)jj * 4 + l) * pw + (dw < nw ? dw : nw - 1);
        },
        tv, tag, deadline, late);
  }
  // each rank's limb count and sum; its first NLF table planes into this
  // wave's LDS (then read back in load_act_regs' layout)
  int nlr[JP];
  uint32_t smr[JP];
  bool one = true;   // every live rank at one limb (the common case)
#pragma unroll
  for (int i = 0; i < JP; ++i) {
    const int j = wave + NWV * i;
    int n = lane < f.gu.nchunks ? (int)tv[i * NWD] : 1;
    uint32_t sm = lane < f.gu.nchunks ? tv[i * NWD + 1] : 0u;
    if (lane + kWave < f.gu.nchunks) {
      n = (int)tv[i * NWD + 2] > n ? (int)tv[i * NWD + 2] : n;
      sm += tv[i * NWD + 3];
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const int o = __shfl_xor(n, off, kWave);
      n = o > n ? o : n;
      sm += (uint32_t)__shfl_xor((int)sm, off, kWave);
    }
    nlr[i] = n <= 1 ? 1 : (n <= 2 ? 2 : 4);
    smr[i] = sm;
    if (ej[i] < 0) continue;
    one = one && nlr[i] == 1;
    uint32_t* tl = tabl + (size_t)j * NLF * pw;
#pragma unroll
    for (int l = 0; l < NLF; ++l)
#pragma unroll
      for (int t = 0; t < kFusePlaneWords; ++t) {
        const int dw = lane + kWave * t;
        if (dw < nw) tl[l * pw + dw] = tv[i * NWD + 4 + l * kFusePlaneWords + t];
      }
  }
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
  auto dot_rank = [&](int i, auto nl_tag) {
    constexpr int NL = decltype(nl_tag)::value;
    const uint32_t* tl = tabl + (size_t)(wave + NWV * i) * NLF * pw;
    ActRegs<Q4, G, NL> ar;
#pragma unroll
    for (int l = 0; l < NL; ++l)
#pragma unroll
      for (int p = 0; p < G::P; ++p) {
        const int d = (p * G::LPR + r) * 4;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          ar.a[l][4 * p + u] = tl[l * pw + d + u];
          if constexpr (Q4) ar.a[l][G::DW + 4 * p + u] = tl[l * pw + KW + d + u];
        }
      }
    const uint32_t v2 = group_sum_dpp<G::LPR>(lane_dot<Q4, G, NL>(w[i], ar));
    return Q4 ? v2 - 8u * smr[i] : v2;
  };
  if (one) {
    // both ranks' dots side by side (a dead rank's weights are zero; its
    // result is not stored)
    uint32_t tot[JP];
#pragma unroll
    for (int i = 0; i < JP; ++i) tot[i] = dot_rank(i, std::integral_constant<int, 1>());
#pragma unroll
    for (int i = 0; i < JP; ++i)
      if (ej[i] >= 0 && r == 0 && row < r1)
        yb[(size_t)(wave + NWV * i) * G::WR + g] = qdot_epilogue(tot[i], div, sc[i]);
  } else {
#pragma unroll
    for (int i = 0; i < JP; ++i) {
      const int j = wave + NWV * i;
      if (ej[i] < 0) continue;
      if (nlr[i] <= NLF) {
        const uint32_t tot = nlr[i] == 1 ? dot_rank(i, std::integral_constant<int, 1>())
                                         : dot_rank(i, std::integral_constant<int, NLF>());
        if (r == 0 && row < r1) yb[(size_t)j * G::WR + g] = qdot_epilogue(tot, div, sc[i]);
      } else {
        // activations past the register budget: the exact fallback on the
        // fp32 h (its weights reloaded by the wave)
        float* hj = hx + (size_t)j * K;
        const uint64_t* th = f.ft.h + (size_t)j * K;
        for (int k = lane; k < K; k += kWave) hj[k] = __uint_as_float(tag_wait(th + k, tag, deadline, late));
        __threadfence_block();
        __builtin_amdgcn_wave_barrier();
        const uint8_t* W[1] = {a.dq + (size_t)ej[i] * a.D * a.rb};
        DownEpi epi{a.ds + (size_t)ej[i] * a.D, yb + (size_t)j * G::WR, r0, div};
        generic_rows_fp32<Q4, 1>(W, a.rb, K, hj, r0, r1, epi, 0, 1);
      }
    }
  }
  if (late) late_any = 1;
  __syncthreads();
  static_assert(G::WR <= kTileBlock, "a thread an output row");
  if (r0 + tid < r1) {
    const int o = r0 + tid;
    float acc = 0.0f;
    for (int j = 0; j < a.topk; ++j) {
      if (gidx[j] < 0) continue;
      const float py = gp[j] * yb[(size_t)j * G::WR + (o - r0)];
      acc = acc + py;
    }
    float res = a.resid ? rv + acc : acc;
    if (late_any) res = __builtin_nanf("");
    a.out[o] = res;
  }
}

template <bool Q4, class GG, class GD>
__global__ __launch_bounds__(kTileBlock) void gate_up_down_kernel(FuseArgs f) {
  extern __shared__ float fl[];
  const uint32_t tag = *f.ft.epoch;
  if ((int)blockIdx.x < f.ngu) {
    int rc, q;
    xcd_chunk_item(f.gu.nchunks, f.gu.npairs, &rc, &q);
    gate_up_block<Q4, GG, true, true>(f.gu, rc, q, fl, &f.ft, tag);
  } else {
    down_fused_block<Q4, GD>(f, (int)blockIdx.x - f.ngu, tag, fl);
  }
}

// rmsnorm (test_model_trace.c:241-255): one block per token; the squares
// x_i * x_i are formed by all threads into LDS and summed in order by
// block_seq_sum (msq / D, 1 / sqrtf(msq + eps)).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      float* __restrict__ y, int D, float eps,
                                                      int fast) {
  extern __shared__ float4 sq4[];
  __shared__ float inv_s;
  __shared__ SeqSumScratch seq;
  const int t = blockIdx.x;
  const float* xt = x + (size_t)t * D;
  if (fast) {
    for (int i = threadIdx.x; i < D / 4; i += blockDim.x) {
      const float4 v = reinterpret_cast<const float4*>(xt)[i];
      sq4[i] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
    }
    __syncthreads();
    const float acc = block_seq_sum<256>(reinterpret_cast<const float*>(sq4), D, seq);
    if (threadIdx.x == 0) {
      const float msq = acc / (float)D;
      inv_s = 1.0f / sqrtf(msq + eps);
    }
  } else if (threadIdx.x == 0) {
    float msq = 0.0f;
    for (int i = 0; i < D; ++i) {
      const float sq = xt[i] * xt[i];
      msq = msq + sq;
    }
    msq = msq / (float)D;
    inv_s = 1.0f / sqrtf(msq + eps);
  }
  __syncthreads();
  const float inv = inv_s;
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    const float v = xt[i] * inv;
    y[(size_t)t * D + i] = v * (w ? w[i] : 1.0f);
  }
}

// ---- host helpers ----
template <class T>
void dfree(T* p) {
  if (p) (void)hipFree((void*)p);
}

template <class T>
moe_status dev_alloc(T** p, size_t count) {
  *p = nullptr;
  if (count == 0) return MOE_OK;
  return check_hip(hipMalloc((void**)p, count * sizeof(T)), "hipMalloc(layer)");
}

// Per-forward scratch is shared by every layer of the process: forwards are
// enqueued on the one library stream under g_layer_mu, so they never overlap
// on the device.  Each buffer grows to the largest need seen (after the
// stream drains) and is kept until the process ends.
struct ScratchBuf {
  void* p = nullptr;
  size_t bytes = 0;
};
struct SharedScratch {
  ScratchBuf logits, idx, p, xtab, htab, h, xn, hpart, xpart, ecount, eoff, perm, y, y16, tasks, ghist, rpart;
  ScratchBuf ftag;                   // tagged words of the one-token gate/up + down launch
  unsigned* sel_counter = nullptr;   // fused selection's block counter, zero between launches
  uint32_t* epoch = nullptr;         // the fused launch's tag, advanced by the router launch
};
SharedScratch g_scratch;
std::mutex g_layer_mu;

moe_status grow(ScratchBuf& b, size_t need, bool* synced) {
  if (need <= b.bytes) return MOE_OK;
  if (!*synced) {
    moe_status st = check_hip(hipStreamSynchronize(stream()), "sync");
    if (st) return st;
    *synced = true;
  }
  dfree(b.p);
  b.p = nullptr;
  b.bytes = 0;
  const size_t cap = need + need / 4;
  moe_status st = check_hip(hipMalloc(&b.p, cap), "hipMalloc(layer scratch)");
  if (st) return st;
  b.bytes = cap;
  return MOE_OK;
}

moe_status ensure_scratch(LayerDev* L, int T) {
  SharedScratch& S = g_scratch;
  bool synced = false;
  moe_status st;
  const size_t np = (size_t)T * L->topk;
  if ((st = grow(S.logits, (size_t)T * L->E * 4, &synced)) || (st = grow(S.idx, np * 4, &synced)) ||
      (st = grow(S.p, np * 4, &synced)) ||
      (st = grow(S.xtab, (size_t)T * act_table_bytes(L->D), &synced)) ||
      (st = grow(S.htab, np * act_table_bytes(L->dff), &synced)) ||
      (st = grow(S.h, np * L->dff * 4, &synced)) || (st = grow(S.xn, (size_t)T * L->D * 4, &synced)) ||
      (st = grow(S.hpart, np * (size_t)((L->dff + 7) / 8) * 8, &synced)) ||
      (st = grow(S.xpart, (size_t)(T > 4 ? 16 : T) * (L->E + 16) * 8, &synced)))
    return st;
  if (grouped_ok(L) &&
      ((st = grow(S.ecount, (size_t)L->E * 4, &synced)) || (st = grow(S.eoff, (size_t)L->E * 4, &synced)) ||
       (st = grow(S.perm, np * 4, &synced)) || (st = grow(S.y, np * L->D * 4, &synced)) ||
       (L->dtype == 3 && (st = grow(S.y16, np * L->D * 2, &synced))) ||
       (st = grow(S.tasks, (np / kMinSplitPairs + L->E + 1) * 8, &synced)) ||
       (st = grow(S.ghist, (size_t)kGroupBlocks * L->E * 4, &synced)) ||
       (st = grow(S.rpart, ((size_t)T / 16 + 1) * ((L->E + 3) / 4) * 16 * 8, &synced))))
    return st;
  L->logits = (float*)S.logits.p; L->idx = (int*)S.idx.p; L->p = (float*)S.p.p;
  L->xtab = (uint8_t*)S.xtab.p; L->htab = (uint8_t*)S.htab.p; L->h = (float*)S.h.p;
  L->xn = (float*)S.xn.p; L->hpart = (uint32_t*)S.hpart.p; L->xpart = (uint32_t*)S.xpart.p;
  L->ecount = (int*)S.ecount.p; L->eoff = (int*)S.eoff.p; L->perm = (int*)S.perm.p;
  L->tasks = (int2*)S.tasks.p;
  L->ghist = (int*)S.ghist.p;
  L->rpart = (uint2*)S.rpart.p;
  if (!S.sel_counter) {
    if ((st = dev_alloc(&S.sel_counter, 1))) return st;
    if ((st = check_hip(hipMemsetAsync(S.sel_counter, 0, 4, stream()), "counter init"))) return st;
  }
  if (T == 1 && L->topk <= kFuseTopK) {
    // zero-filled when (re)allocated: tag 0 is never an epoch
    const size_t words = (size_t)kFuseTopK * (4 * (((size_t)L->dff + 15) / 16 * 4) + L->dff +
                                              2 * (((size_t)L->dff + 7) / 8));
    // (zeroed on every reallocation, even one at the same address)
    const void* old = S.ftag.p;
    const size_t old_bytes = S.ftag.bytes;
    if ((st = grow(S.ftag, words * 8, &synced))) return st;
    if ((S.ftag.p != old || S.ftag.bytes != old_bytes) &&
        (st = check_hip(hipMemsetAsync(S.ftag.p, 0, S.ftag.bytes, stream()), "tag buffer init")))
      return st;
    if (!S.epoch) {
      if ((st = dev_alloc(&S.epoch, 1))) return st;
      if ((st = check_hip(hipMemsetAsync(S.epoch, 0, 4, stream()), "epoch init"))) return st;
    }
    L->ftag = (uint64_t*)S.ftag.p;
    L->epoch = S.epoch;
  } else {
    L->ftag = nullptr;
    L->epoch = nullptr;
  }
  L->y = (float*)S.y.p;
  L->y16 = L->dtype == 3 ? (int16_t*)S.y16.p : nullptr;
  L->sel_counter = S.sel_counter;
  L->capT = T;
  return MOE_OK;
}

void release_scratch_all() {
  std::lock_guard<std::mutex> lk(g_layer_mu);
  SharedScratch& S = g_scratch;
  for (ScratchBuf* b : {&S.logits, &S.idx, &S.p, &S.xtab, &S.htab, &S.h, &S.xn, &S.hpart, &S.xpart,
                        &S.ecount, &S.eoff, &S.perm, &S.y, &S.y16, &S.tasks, &S.ghist, &S.rpart,
                        &S.ftag}) {
    dfree(b->p);
    b->p = nullptr;
    b->bytes = 0;
  }
  dfree(S.sel_counter);
  S.sel_counter = nullptr;
  dfree(S.epoch);
  S.epoch = nullptr;
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

// Rows-per-block targets (tuning knobs, read once): MOEHIP_GATEUP_BLOCKS and
// MOEHIP_DOWN_BLOCKS set the number of blocks a launch aims for.
int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}
int gateup_target_blocks() { static const int v = env_int("MOEHIP_GATEUP_BLOCKS", 1024); return v; }
// Tokens from which the few-token gate/up and down kernels load expert rows
// with ordinary (cache-allocating) loads instead of nontemporal ones: with
// many tokens, pairs that share an expert read its rows again (tuning knobs
// MOEHIP_GATEUP_CACHED_MIN_T, MOEHIP_DOWN_CACHED_MIN_T; 0 = never).
int gateup_cached_min_tokens() { static const int v = env_int("MOEHIP_GATEUP_CACHED_MIN_T", 12); return v; }
int down_cached_min_tokens() { static const int v = env_int("MOEHIP_DOWN_CACHED_MIN_T", 12); return v; }
bool cached_loads(int T, int min_t) { return min_t > 0 && T >= min_t; }

int down_target_blocks() { static const int v = env_int("MOEHIP_DOWN_BLOCKS", 512); return v; }

template <class G>
GateUpArgs gate_up_args(const LayerDev* L, const float* xn, int T, bool sel, int nxpart,
                        int32_t* idx_out, float* p_out, int xp_tok, int xp_slice) {
  // rows per block: a multiple of both the wave-group unit and 8 (whole
  // packed dwords of h), sized for ~1024 blocks
  constexpr int unit0 = kTileWaves * G::WR;
  constexpr int unit = unit0 % 8 == 0 ? unit0 : (unit0 % 4 == 0 ? unit0 * 2 : unit0 * 8);
  const int npairs = T * L->topk;
  const long long total = (long long)L->dff * npairs;
  const int tgt = gateup_target_blocks();
  long long rpb = (total + tgt - 1) / tgt;
  rpb = std::max<long long>(unit, (rpb + unit - 1) / unit * unit);
  rpb = std::min<long long>(rpb, 8 * unit);
  // several tokens: a chunk count that is a multiple of 8, so that every
  // chunk's pairs run on one XCD (xcd_chunk_item) and pairs sharing an
  // expert find its rows in that XCD's L2 -- the nearest such count at or
  // above the target, if its rows per block stay a whole number of units
  if (npairs > L->topk) {
    const long long nc0 = (L->dff + rpb - 1) / rpb;
    const long long nc8 = (nc0 + 7) / 8 * 8;
    const long long r8 = ((L->dff + nc8 - 1) / nc8 + unit - 1) / unit * unit;
    if ((L->dff + r8 - 1) / r8 == nc8) rpb = r8;
  }
  const int nc = (int)((L->dff + rpb - 1) / rpb);
  GateUpArgs a{L->gq, L->gs, L->uq, L->us, L->rbg, L->D, L->dff, L->topk, L->idx,
               L->xtab, act_table_bytes(L->D), xn, L->h, L->htab, act_table_bytes(L->dff),
               L->hpart, nc, (int)rpb};
  a.npairs = npairs;
  if (sel) {
    a.logits = L->logits; a.xpart = L->xpart; a.nxpart = nxpart; a.E = L->E;
    a.xp_tok = xp_tok; a.xp_slice = xp_slice;
    a.idx_w = L->idx; a.p = L->p; a.idx_user = idx_out; a.p_user = p_out;
  }
  return a;
}

template <bool Q4, class G>
void launch_gate_up(const LayerDev* L, const float* xn, int T, int* nchunks, hipStream_t s,
                    bool sel = false, int nxpart = 0, int32_t* idx_out = nullptr,
                    float* p_out = nullptr, int xp_tok = 0, int xp_slice = 1) {
  const GateUpArgs a = gate_up_args<G>(L, xn, T, sel, nxpart, idx_out, p_out, xp_tok, xp_slice);
  const size_t rpb = (size_t)a.rows_per_block;
  *nchunks = a.nchunks;
  dim3 grid((unsigned)(a.nchunks * a.npairs));
  if (sel) {
    if (cached_loads(T, gateup_cached_min_tokens()))
      hipLaunchKernelGGL((gate_up_kernel<Q4, G, true, false>), grid, dim3(kTileBlock), (size_t)rpb * 4, s, a);
    else
      hipLaunchKernelGGL((gate_up_kernel<Q4, G, true, true>), grid, dim3(kTileBlock), (size_t)rpb * 4, s, a);
  } else if (cached_loads(T, gateup_cached_min_tokens())) {
    hipLaunchKernelGGL((gate_up_kernel<Q4, G, false, false>), grid, dim3(kTileBlock), (size_t)rpb * 4, s, a);
  } else {
    hipLaunchKernelGGL((gate_up_kernel<Q4, G, false, true>), grid, dim3(kTileBlock), (size_t)rpb * 4, s, a);
  }
}

template <bool Q4, class G>
void launch_down(const LayerDev* L, int T, int nchunks, const float* resid, float* out,
                 hipStream_t s) {
  constexpr int unit = G::WR;                   // one wave per rank
  const long long total = (long long)L->D * T;
  const int tgt = down_target_blocks();
  long long rpb = (total + tgt - 1) / tgt;
  rpb = std::max<long long>(unit, (rpb + unit - 1) / unit * unit);
  rpb = std::min<long long>(rpb, 16 * unit);
  DownArgs a{L->dq, L->ds, L->rbd, T, L->D, L->dff, L->topk, L->idx, L->p, L->htab,
             act_table_bytes(L->dff), L->h, L->hpart, nchunks, resid, out, (int)rpb};
  a.nrc = (int)((L->D + rpb - 1) / rpb);
  dim3 grid((unsigned)(a.nrc * T));
  if (!cached_loads(T, down_cached_min_tokens()))
    hipLaunchKernelGGL((down_combine_kernel<Q4, G, true>), grid, dim3(kCombineThreads),
                       (size_t)L->topk * rpb * 4, s, a);
  else
    hipLaunchKernelGGL((down_combine_kernel<Q4, G, false>), grid, dim3(kCombineThreads),
                       (size_t)L->topk * rpb * 4, s, a);
}

// Wall-clock ticks a fused launch's down block may wait for its inputs
// (20 ms; the clock rate is the device's, read once).
// MOEHIP_FUSE_WAIT_US (read at every launch; tests set 0 to drive the
// deadline path from the host) overrides the 20 ms.
long long fuse_wait_ticks() {
  static const long long khz = [] {
    int dev = 0, k = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&k, hipDeviceAttributeWallClockRate, dev) != hipSuccess || k <= 0)
      k = 100000;
    return (long long)k;
  }();
  const char* us = getenv("MOEHIP_FUSE_WAIT_US");
  const long long wait_us = us && *us ? atoll(us) : 20000;
  return khz * (wait_us < 0 ? 0 : wait_us) / 1000;
}

size_t fuse_lds(const LayerDev* L, int rpb_gu, int wr) {
  const size_t pw = ((size_t)L->dff + 15) / 16 * 4;
  const size_t dn = ((size_t)kFuseTopK * wr + (size_t)kFuseTopK * 2 * pw + (size_t)L->topk * L->dff) * 4;
  const size_t gu = (size_t)rpb_gu * 4;
  return dn > gu ? dn : gu;
}

template <bool Q4, class GG, class GD>
void launch_gate_up_down(const LayerDev* L, const float* xn, const float* resid, float* out,
                         int nxpart, int32_t* idx_out, float* p_out, int xp_tok, int xp_slice,
                         hipStream_t s) {
  FuseArgs f;
  f.gu = gate_up_args<GG>(L, xn, 1, true, nxpart, idx_out, p_out, xp_tok, xp_slice);
  f.dn = DownArgs{L->dq, L->ds, L->rbd, 1, L->D, L->dff, L->topk, L->idx, L->p, L->htab,
                  act_table_bytes(L->dff), L->h, L->hpart, f.gu.nchunks, resid, out, GD::WR};
  f.dn.nrc = (L->D + GD::WR - 1) / GD::WR;
  const size_t pw = ((size_t)L->dff + 15) / 16 * 4;   // dwords per act-table plane
  f.ft.pw = (int)pw;
  f.ft.pchunks = (L->dff + 7) / 8;
  f.ft.tab = L->ftag;
  f.ft.h = L->ftag + (size_t)kFuseTopK * 4 * pw;
  f.ft.part = f.ft.h + (size_t)kFuseTopK * L->dff;
  f.ft.epoch = L->epoch;
  f.ft.wait_ticks = fuse_wait_ticks();
  f.ngu = f.gu.nchunks * f.gu.npairs;
  hipLaunchKernelGGL((gate_up_down_kernel<Q4, GG, GD>), dim3((unsigned)(f.ngu + f.dn.nrc)),
                     dim3(kTileBlock), fuse_lds(L, f.gu.rows_per_block, GD::WR), s, f);
}

// Row-byte dispatch for the expert GEMVs (same geometries as gemv.hip).
template <bool Q4, class F>
void with_geom(long long rb, F&& f) {
  switch (rb) {
    case 192:  f(TileGeom<3, 4>()); return;
    case 256:  f(TileGeom<4, 4>()); return;
    case 384:  f(TileGeom<3, 8>()); return;
    case 512:  f(TileGeom<4, 8>()); return;
    case 768:  f(TileGeom<3, 16>()); return;
    case 1024: f(TileGeom<4, 16>()); return;
    case 1536: f(TileGeom<3, 32>()); return;
    case 2048: f(TileGeom<4, 32>()); return;
    case 3072: f(TileGeom<3, 64>()); return;
    case 4096: f(TileGeom<4, 64>()); return;
    default: f(GenericGeom()); return;
  }
}

// The fused one-token launch is built for Q4 at D = 2048, d_ff = 768 (the
// model's layers).  Q8 at that shape measured slower fused (29.7 -> 33.6 us
// a layer): its 768 gate/up blocks fill every slot, so the down blocks
// start only as gate/up ends, with their selection still ahead of them.
using FuseGG = TileGeom<4, 16>;
using FuseGD = TileGeom<3, 8>;
bool fuse_geoms(const LayerDev* L) { return L->dtype == 3 && L->rbg == 1024 && L->rbd == 384; }

// The down blocks read two gate/up chunk partials a lane: at most 128 chunks.
bool fuse_chunks_ok(const LayerDev* L) {
  return gate_up_args<FuseGG>(L, nullptr, 1, true, 0, nullptr, nullptr, 0, 1).nchunks <= 2 * kWave;
}

void launch_fused(const LayerDev* L, const float* xn, const float* resid, float* out, int nxpart,
                  int32_t* idx_out, float* p_out, int xp_tok, int xp_slice, hipStream_t s) {
  launch_gate_up_down<true, FuseGG, FuseGD>(L, xn, resid, out, nxpart, idx_out, p_out, xp_tok, xp_slice, s);
}

}  // namespace

// Tokens from which the expert-major kernels replace the per-pair decode
// kernels (layer setting, else MOEHIP_GROUPED_MIN_T, else 32).
int grouped_min_tokens(const LayerDev* L) {
  static const int dflt = env_int("MOEHIP_GROUPED_MIN_T", 32);
  return L->grouped_min_T > 0 ? L->grouped_min_T : dflt;
}

moe_status rmsnorm_dev(const float* x, const float* w, float* y, int T, int D, float eps);

// The MoE block of T tokens on scratch already bound to L (ensure_scratch or
// the no-allocation array).  norm_eps >= 0: `x` is the raw residual stream
// and the block starts with rmsnorm(x, rms2_w) (:461), fused into the router
// product for few tokens; norm_eps < 0: `x` is already x_norm.
// allow_grouped: many tokens may take the expert-major kernels (their
// scratch bound too); otherwise every T runs the per-pair kernels.
moe_status layer_forward_run(LayerDev* L, const float* x, float norm_eps, const float* resid,
                             int T, float* out, int32_t* idx_out, float* p_out,
                             bool allow_grouped) {
  moe_status st = MOE_OK;
  hipStream_t s = stream();
  const bool grouped = allow_grouped && T >= grouped_min_tokens(L) && grouped_ok(L);
  const bool fuse_norm = norm_eps >= 0.0f && !grouped && dense_norm_ok(T, L->D) &&
                         dense_select_ok(T, L->E) && aligned16(x) && aligned16(L->router_w);
  const float* xn = x;
  if (norm_eps >= 0.0f && !fuse_norm) {
    if ((st = rmsnorm_dev(x, L->rms2_w, L->xn, T, L->D, norm_eps))) return st;
    xn = L->xn;
  }
  if (grouped) return layer_forward_grouped(L, xn, resid, T, out, idx_out, p_out);
  const bool q4 = L->dtype == 3;
  DenseArgs ra{xn, L->D, L->router_w, L->D, L->router_b, nullptr, 0, L->logits, L->E, T, L->E, L->D};
  // router logits (+ bias), then top-k and gates (in the router launch's
  // last block for few tokens)
  const bool fuse_sel = dense_select_ok(T, L->E) && aligned16(L->router_w) &&
                        (fuse_norm || aligned16(xn));
  if (fuse_norm) {
    // rmsnorm + x tables + router logits in one launch
    ra.norm = 1; ra.norm_w = L->rms2_w; ra.eps = norm_eps;
    ra.xn_out = L->xn; ra.pack_dtype = L->dtype; ra.pack_tabs = L->xtab; ra.pack_part = L->xpart;
    xn = L->xn;
  } else if (fuse_sel && T <= 4 && dense_row_path(ra)) {
    // up to four given rows: the router's row kernel packs the x tables too
    ra.pack_dtype = L->dtype; ra.pack_tabs = L->xtab; ra.pack_part = L->xpart;
  } else if (!fuse_sel && dense_rows4_path(ra)) {
    // 5-16 given rows: the router's rows kernel packs the x tables too, the
    // selection kernel writes their headers
    ra.pack_dtype = L->dtype; ra.pack_tabs = L->xtab; ra.pack_part = L->xpart;
  } else {
    // x tables for the expert GEMVs
    QShape sh;
    sh.dtype = L->dtype; sh.M = T; sh.N = 1; sh.K = L->D; sh.lda = L->D; sh.ldc = 1; sh.rs = L->rbg;
    QJob one{nullptr, nullptr, xn, nullptr};
    if ((st = check_hip(launch_act_pack(sh, nullptr, one, 1, L->xtab, s), "act pack"))) return st;
  }
  if (fuse_sel) {
    ra.sel_counter = L->sel_counter; ra.sel_topk = L->topk;
    ra.sel_idx = L->idx; ra.sel_p = L->p; ra.sel_idx_user = idx_out; ra.sel_p_user = p_out;
  }
  // up to two tokens the gate/up blocks select themselves (no selection
  // launch) after the row kernel, from each token's x-table partials
  // [token][row]; the same works after the rows kernel (5-16 tokens,
  // partials [row][16 tokens]) with MOEHIP_SEL_GU_MAX_T raised, but from 4
  // tokens on the ranking in every block delays the weight streams by more
  // than the saved launch (measured T = 4 / 8 / 16: +1 / +2 / +2 us)
  static const bool sel_kernel = getenv("MOEHIP_SELECT_KERNEL") != nullptr;
  static const int sel_gu_max_t = env_int("MOEHIP_SEL_GU_MAX_T", 2);
  const bool rows_pack = !fuse_sel && ra.pack_dtype != 0;
  const bool sel_gu = !sel_kernel && T <= sel_gu_max_t && L->E <= kTileBlock &&
                      ((fuse_sel && dense_row_path(ra)) || (rows_pack && T <= 16));
  ra.sel_defer = sel_gu && fuse_sel ? 1 : 0;
  // one token: gate/up and down in one launch, where its geometries are built
  static const bool no_fuse_gd = getenv("MOEHIP_NO_FUSE_GD") != nullptr;
  const bool fuse_gd = !no_fuse_gd && T == 1 && sel_gu && fuse_sel && ra.sel_defer && L->ftag &&
                       L->epoch && L->topk <= kFuseTopK && fuse_geoms(L) && fuse_chunks_ok(L) &&
                       ((size_t)L->dff + 15) / 16 * 4 <= (size_t)kWave * kFusePlaneWords &&
                       fuse_lds(L, 0, 64) <= 64 * 1024;
  if (fuse_gd) ra.epoch_bump = L->epoch;
  if ((st = dense_matmul(ra, s))) return st;
  if (!fuse_sel && !sel_gu &&
      (st = launch_select(L, T, idx_out, p_out, s,
                          rows_pack ? reinterpret_cast<const uint2*>(L->xpart) : nullptr,
                          rows_pack ? L->E : 0)))
    return st;
  const int nxpart = ra.pack_dtype ? L->E : 0;
  const int xp_tok = rows_pack ? 1 : L->E, xp_slice = rows_pack ? 16 : 1;
  if (fuse_gd) {
    launch_fused(L, xn, resid, out, nxpart, idx_out, p_out, xp_tok, xp_slice, s);
    return check_hip(hipGetLastError(), "gate_up/down launch");
  }
  int nchunks = 0;
  if (q4) with_geom<true>(L->rbg, [&](auto g) { launch_gate_up<true, decltype(g)>(L, xn, T, &nchunks, s, sel_gu, nxpart, idx_out, p_out, xp_tok, xp_slice); });
  else with_geom<false>(L->rbg, [&](auto g) { launch_gate_up<false, decltype(g)>(L, xn, T, &nchunks, s, sel_gu, nxpart, idx_out, p_out, xp_tok, xp_slice); });
  if ((st = check_hip(hipGetLastError(), "gate_up launch"))) return st;
  if (q4) with_geom<true>(L->rbd, [&](auto g) { launch_down<true, decltype(g)>(L, T, nchunks, resid, out, s); });
  else with_geom<false>(L->rbd, [&](auto g) { launch_down<false, decltype(g)>(L, T, nchunks, resid, out, s); });
  return check_hip(hipGetLastError(), "down launch");
}

moe_status layer_forward_impl(LayerDev* L, const float* x, float norm_eps, const float* resid,
                              int T, float* out, int32_t* idx_out, float* p_out) {
  if (T <= 0) return MOE_OK;
  moe_status st = ensure_scratch(L, T);
  if (st) return st;
  return layer_forward_run(L, x, norm_eps, resid, T, out, idx_out, p_out, true);
}

moe_status layer_forward(LayerDev* L, const float* xn, const float* resid, int T, float* out,
                         int32_t* idx_out, float* p_out) {
  return layer_forward_impl(L, xn, -1.0f, resid, T, out, idx_out, p_out);
}

// ---- the no-allocation forward ----
//
// Its scratch is this file-scope device array: each GPU holds its own copy
// from module load until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the
// symbol); it uses the device address hipGetSymbolAddress returns, looked up
// once per device.  Every no-allocation call on a GPU shares the array, so
// calls that overlap on one GPU race: the library serialises its own calls
// (one stream, g_layer_mu), callers that enqueue on other streams must not
// overlap two such forwards.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
constexpr int kNoAllocMaxTokens = 32;
constexpr int kNoAllocMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_noalloc_mu;
uint8_t* g_noalloc_ptr[kNoAllocMaxDevices] = {};

__global__ void zero_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Byte offsets of the per-pair path's buffers inside the array (the same
// buffers ensure_scratch sizes for that path); returns the total.
struct NoAllocLayout {
  size_t counter, logits, idx, p, xtab, htab, h, xn, hpart, xpart, total;
};
NoAllocLayout noalloc_layout(const LayerDev* L, int T) {
  NoAllocLayout o{};
  const size_t np = (size_t)T * L->topk;
  size_t at = 0;
  auto take = [&](size_t bytes) { const size_t r = at; at += align256(bytes); return r; };
  o.counter = take(4);
  o.logits = take((size_t)T * L->E * 4);
  o.idx = take(np * 4);
  o.p = take(np * 4);
  o.xtab = take((size_t)T * act_table_bytes(L->D));
  o.htab = take(np * act_table_bytes(L->dff));
  o.h = take(np * L->dff * 4);
  o.xn = take((size_t)T * L->D * 4);
  o.hpart = take(np * (size_t)((L->dff + 7) / 8) * 8);
  o.xpart = take((size_t)(T > 4 ? 16 : T) * (L->E + 16) * 8);
  o.total = at;
  return o;
}

// The array's device address on the current device, looked up (and its
// selection counter zeroed, which every launch that uses it leaves at zero
// again) on the first call on that device.
moe_status noalloc_scratch(uint8_t** out) {
  int dev = 0;
  moe_status st = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (st) return st;
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(MOE_ERR_UNSUPPORTED, "layer_forward_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    if ((st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")))
      return st;
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(64), 0, stream(), (uint32_t*)p, 64);
    if ((st = check_hip(hipGetLastError(), "scratch counter clear"))) return st;
    g_noalloc_ptr[dev] = (uint8_t*)p;
  }
  *out = g_noalloc_ptr[dev];
  return MOE_OK;
}

}  // namespace

moe_status rmsnorm_dev(const float* x, const float* w, float* y, int T, int D, float eps) {
  if (T <= 0) return MOE_OK;
  const int fast = (D % 4 == 0) && aligned16(x) && (size_t)D * 4 <= kMaxLds;
  const size_t lds = fast ? (size_t)D * 4 : 0;
  if (lds > 65536) {
    moe_status st = check_hip(hipFuncSetAttribute((const void*)rmsnorm_kernel,
                                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  (int)lds), "rmsnorm LDS attribute");
    if (st) return st;
  }
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), lds, stream(), x, w, y, D, eps, fast);
  return check_hip(hipGetLastError(), "rmsnorm launch");
}

void release_layer_scratch() { release_scratch_all(); }

}  // namespace moe

using namespace moe;

struct moe_layer {
  LayerDev L;
  moe_layer() { moe::live_objects(1); }
  ~moe_layer() { moe::live_objects(-1); }
};

namespace {

moe_status upload(void* dst, const void* src, size_t bytes, int on_device) {
  if (!bytes) return MOE_OK;
  return check_hip(hipMemcpyAsync(dst, src, bytes, on_device ? hipMemcpyDeviceToDevice
                                                              : hipMemcpyHostToDevice, stream()),
                   "layer upload");
}

void free_layer(LayerDev& L) {
  dfree(L.router_w); dfree(L.router_b); dfree(L.rms2_w);
  dfree(L.gq); dfree(L.gs); dfree(L.uq); dfree(L.us); dfree(L.dq); dfree(L.ds);
  // scratch pointers belong to the shared per-process scratch
}

}  // namespace

extern "C" {

moe_status moe_layer_create_raw(int dtype, int D, int d_ff, int E, int top_k,
                                const float* router_w, const float* router_b, const float* rms2_w,
                                const void* gq, const float* gs, const void* uq, const float* us,
                                const void* dq, const float* ds, int src_on_device,
                                moe_layer** out) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!out) return set_error(MOE_ERR_ARG, "layer_create: null out");
  *out = nullptr;
  if (dtype != 2 && dtype != 3) return set_error(MOE_ERR_ARG, "layer_create: dtype %d", dtype);
  if (D <= 0 || d_ff <= 0 || E <= 0 || top_k <= 0 || top_k > kMaxTopK || top_k > E || E > 1024)
    return set_error(MOE_ERR_ARG, "layer_create: bad dims D=%d d_ff=%d E=%d top_k=%d", D, d_ff, E, top_k);
  if (dtype == 3 && ((D & 1) || (d_ff & 1)))
    return set_error(MOE_ERR_ARG, "layer_create: Q4 needs even D and d_ff");
  if (!router_w || !gq || !gs || !uq || !us || !dq || !ds)
    return set_error(MOE_ERR_ARG, "layer_create: null weight pointer");
  moe_layer* ml = new (std::nothrow) moe_layer();
  if (!ml) return set_error(MOE_ERR_NOMEM, "layer_create: host allocation");
  LayerDev& L = ml->L;
  L.dtype = dtype; L.D = D; L.dff = d_ff; L.E = E; L.topk = top_k;
  L.rbg = dtype == 2 ? D : D / 2;
  L.rbd = dtype == 2 ? d_ff : d_ff / 2;
  const size_t ng = (size_t)E * d_ff * L.rbg, nd = (size_t)E * D * L.rbd;
  if ((st = dev_alloc(&L.router_w, (size_t)E * D)) || (router_b && (st = dev_alloc(&L.router_b, E))) ||
      (rms2_w && (st = dev_alloc(&L.rms2_w, D))) || (st = dev_alloc(&L.gq, ng)) ||
      (st = dev_alloc(&L.uq, ng)) || (st = dev_alloc(&L.dq, nd)) ||
      (st = dev_alloc(&L.gs, (size_t)E * d_ff)) || (st = dev_alloc(&L.us, (size_t)E * d_ff)) ||
      (st = dev_alloc(&L.ds, (size_t)E * D))) {
    free_layer(L);
    delete ml;
    return st;
  }
  const int od = src_on_device;
  if ((st = upload(L.router_w, router_w, (size_t)E * D * 4, od)) ||
      (router_b && (st = upload(L.router_b, router_b, (size_t)E * 4, od))) ||
      (rms2_w && (st = upload(L.rms2_w, rms2_w, (size_t)D * 4, od))) ||
      (st = upload(L.gq, gq, ng, od)) || (st = upload(L.uq, uq, ng, od)) ||
      (st = upload(L.dq, dq, nd, od)) || (st = upload(L.gs, gs, (size_t)E * d_ff * 4, od)) ||
      (st = upload(L.us, us, (size_t)E * d_ff * 4, od)) ||
      (st = upload(L.ds, ds, (size_t)E * D * 4, od)) ||
      (st = check_hip(hipStreamSynchronize(stream()), "layer upload sync"))) {
    free_layer(L);
    delete ml;
    return st;
  }
  *out = ml;
  return MOE_OK;
}

moe_status moe_layer_create(const QwenConfig* cfg, const QwenLayerWeights* lw, moe_layer** out) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!cfg || !lw || !out) return set_error(MOE_ERR_ARG, "layer_create: null argument");
  if (!lw->experts_quantized || !lw->Wg_q || !lw->Wu_q || !lw->Wd_q)
    return set_error(MOE_ERR_UNSUPPORTED, "layer_create: experts are not quantized");
  const int E = cfg->n_experts, D = cfg->d_model, dff = cfg->d_ff;
  if (E <= 0 || D <= 0 || dff <= 0)
    return set_error(MOE_ERR_ARG, "layer_create: bad dims D=%d d_ff=%d E=%d", D, dff, E);
  const int dtype = lw->Wg_q[0].dtype;
  if (dtype != 2 && dtype != 3) return set_error(MOE_ERR_ARG, "layer_create: expert dtype %d", dtype);
  const long long rbg = dtype == 2 ? D : D / 2, rbd = dtype == 2 ? dff : dff / 2;
  // Every expert's descriptor must describe the [d_ff x D] (gate, up) or
  // [D x d_ff] (down) matrix the config implies (model.h:256, 279, 302 set
  // rows / cols from the tensor shapes; cols is the logical column count):
  // the copy below reads that many bytes from each.
  for (int e = 0; e < E; ++e) {
    const QuantizedWeight* ws[3] = {&lw->Wg_q[e], &lw->Wu_q[e], &lw->Wd_q[e]};
    for (int j = 0; j < 3; ++j) {
      const int rows = j < 2 ? dff : D, cols = j < 2 ? D : dff;
      if (!ws[j]->q || !ws[j]->s || ws[j]->rows != rows || ws[j]->cols != cols)
        return set_error(MOE_ERR_ARG,
                         "layer_create: expert %d %s is %d x %d (q %p, s %p), expected %d x %d",
                         e, j == 0 ? "gate" : (j == 1 ? "up" : "down"), ws[j]->rows, ws[j]->cols,
                         (const void*)ws[j]->q, (const void*)ws[j]->s, rows, cols);
    }
  }
  // The reference binds one tensor per expert (model.h:228-305); the device
  // keeps each projection of all experts in one contiguous array.
  std::vector<uint8_t> g((size_t)E * dff * rbg), u((size_t)E * dff * rbg), d((size_t)E * D * rbd);
  std::vector<float> gs((size_t)E * dff), us((size_t)E * dff), ds((size_t)E * D);
  for (int e = 0; e < E; ++e) {
    const QuantizedWeight *wg = &lw->Wg_q[e], *wu = &lw->Wu_q[e], *wd = &lw->Wd_q[e];
    if (wg->dtype != dtype || wu->dtype != dtype || wd->dtype != dtype)
      return set_error(MOE_ERR_ARG, "layer_create: mixed expert dtypes");
    std::memcpy(&g[(size_t)e * dff * rbg], wg->q, (size_t)dff * rbg);
    std::memcpy(&u[(size_t)e * dff * rbg], wu->q, (size_t)dff * rbg);
    std::memcpy(&d[(size_t)e * D * rbd], wd->q, (size_t)D * rbd);
    std::memcpy(&gs[(size_t)e * dff], wg->s, (size_t)dff * 4);
    std::memcpy(&us[(size_t)e * dff], wu->s, (size_t)dff * 4);
    std::memcpy(&ds[(size_t)e * D], wd->s, (size_t)D * 4);
  }
  return moe_layer_create_raw(dtype, D, dff, E, cfg->top_k, lw->router_w, lw->router_b,
                              lw->rms2_w, g.data(), gs.data(), u.data(), us.data(), d.data(),
                              ds.data(), 0, out);
}

moe_status moe_layer_destroy(moe_layer* layer) {
  if (!layer) return MOE_OK;
  moe_status st = check_hip(hipStreamSynchronize(stream()), "sync");
  free_layer(layer->L);
  delete layer;
  return st;
}

moe_status moe_layer_forward(moe_layer* layer, const float* x_norm, const float* x_resid, int T,
                             float* out, int32_t* idx_out, float* p_out) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!layer || !x_norm || !out) return set_error(MOE_ERR_ARG, "layer_forward: null argument");
  if (T < 0) return set_error(MOE_ERR_ARG, "layer_forward: T < 0");
  std::lock_guard<std::mutex> lk(g_layer_mu);
  return layer_forward(&layer->L, x_norm, x_resid, T, out, idx_out, p_out);
}

moe_status moe_layer_forward_noalloc(moe_layer* layer, const float* x_norm, const float* x_resid,
                                     int T, float* out, int32_t* idx_out, float* p_out) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!layer || !x_norm || !out) return set_error(MOE_ERR_ARG, "layer_forward_noalloc: null argument");
  if (T < 0) return set_error(MOE_ERR_ARG, "layer_forward_noalloc: T < 0");
  if (T == 0) return MOE_OK;
  if (T > kNoAllocMaxTokens)
    return set_error(MOE_ERR_ARG, "layer_forward_noalloc: T = %d above the maximum of %d tokens "
                     "(use moe_layer_forward)", T, kNoAllocMaxTokens);
  LayerDev* L = &layer->L;
  const NoAllocLayout o = noalloc_layout(L, T);
  if (o.total > kNoAllocScratchBytes)
    return set_error(MOE_ERR_ARG,
                     "layer_forward_noalloc: %d tokens need %zu scratch bytes, more than the "
                     "%zu-byte no-allocation array (use moe_layer_forward)",
                     T, o.total, kNoAllocScratchBytes);
  std::lock_guard<std::mutex> lk(g_layer_mu);
  uint8_t* base = nullptr;
  if ((st = noalloc_scratch(&base))) return st;
  L->sel_counter = (unsigned*)(base + o.counter);
  L->logits = (float*)(base + o.logits);
  L->idx = (int*)(base + o.idx);
  L->p = (float*)(base + o.p);
  L->xtab = base + o.xtab;
  L->htab = base + o.htab;
  L->h = (float*)(base + o.h);
  L->xn = (float*)(base + o.xn);
  L->hpart = (uint32_t*)(base + o.hpart);
  L->xpart = (uint32_t*)(base + o.xpart);
  L->ecount = L->eoff = L->perm = L->ghist = nullptr;
  L->rpart = nullptr;
  L->tasks = nullptr;
  L->y = nullptr;
  L->y16 = nullptr;
  L->ftag = nullptr;   // the no-allocation forward keeps two launches for gate/up and down
  L->epoch = nullptr;
  L->capT = T;
  return layer_forward_run(L, x_norm, -1.0f, x_resid, T, out, idx_out, p_out, false);
}

moe_status moe_block_forward(moe_layer* layer, const float* x, int T, float* out, float eps) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!layer || !x || !out) return set_error(MOE_ERR_ARG, "block_forward: null argument");
  if (T < 0) return set_error(MOE_ERR_ARG, "block_forward: T < 0");
  LayerDev* L = &layer->L;
  if (T == 0) return MOE_OK;
  if (!(eps >= 0.0f)) return set_error(MOE_ERR_ARG, "block_forward: eps %g < 0", (double)eps);
  std::lock_guard<std::mutex> lk(g_layer_mu);
  return layer_forward_impl(L, x, eps, x, T, out, nullptr, nullptr);
}

moe_status moe_rmsnorm_dev(const float* x, const float* w, float* y, int T, int D, float eps) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!x || !y || T < 0 || D <= 0) return set_error(MOE_ERR_ARG, "rmsnorm: bad argument");
  return rmsnorm_dev(x, w, y, T, D, eps);
}

moe_status moe_layer_set_grouped_min_tokens(moe_layer* layer, int min_tokens) {
  if (!layer) return set_error(MOE_ERR_ARG, "set_grouped_min_tokens: null layer");
  if (min_tokens < 0) return set_error(MOE_ERR_ARG, "set_grouped_min_tokens: %d < 0", min_tokens);
  layer->L.grouped_min_T = min_tokens;
  return MOE_OK;
}

moe_status moe_layer_debug_buffers(moe_layer* layer, const float** logits, const float** h,
                                   const float** y) {
  if (!layer) return set_error(MOE_ERR_ARG, "debug_buffers: null layer");
  if (logits) *logits = layer->L.logits;
  if (h) *h = layer->L.h;
  if (y) *y = nullptr;   // expert outputs stay in LDS (fused with the weighted sum)
  return MOE_OK;
}

}  // extern "C"
