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
#include <mutex>
#include <unordered_set>

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
  // this thread's staging slots: source (float4 units) and LDS offsets
  const float4* srcp[NV];
  int dst[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = tid + 256 * v;
    const int row = i / V4, c4 = i % V4;
    const float* base = row < RX ? a.x + (size_t)min(t0 + row, a.T - 1) * D
                                 : a.W + (size_t)min(e0 + row - RX, a.E - 1) * D;
    srcp[v] = reinterpret_cast<const float4*>(base) + c4;
    dst[v] = row * LD + 4 * c4;
  }
  float4 rg[NV];
  auto load = [&](int c) {
    const size_t o = (size_t)c * V4;
#pragma unroll
    for (int v = 0; v < NV; ++v) rg[v] = srcp[v][o];
  };
  auto store = [&](int bsel) {
    float* b = buf + bsel * R * LD;
#pragma unroll
    for (int v = 0; v < NV; ++v) *reinterpret_cast<float4*>(b + dst[v]) = rg[v];
  };
  float acc[CT][CE];
#pragma unroll
  for (int i = 0; i < CT; ++i)
#pragma unroll
    for (int j = 0; j < CE; ++j) acc[i][j] = 0.0f;
  // loads and stores are unconditional (chunk index clamped; a store past
  // the last chunk fills the idle buffer) so `reg` stays in registers
  load(0);
  store(0);
  load(min(1, nc - 1));
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
    store((c + 1) & 1);
    load(min(c + 2, nc - 1));
    __syncthreads();
  }
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

__global__ __launch_bounds__(kSelectWaves * kWave) void select_kernel(SelectArgs a) {
  __shared__ int sidx[kSelectWaves][kMaxTopK];
  __shared__ float sval[kSelectWaves][kMaxTopK];
  __shared__ float sexp[kSelectWaves][kMaxTopK];
  __shared__ ulonglong2 keys2[kSelectWaves][512];   // E <= 1024 keys per wave
  const int wave = threadIdx.x / kWave;
  const int t = blockIdx.x * kSelectWaves + wave;
  if (t >= a.T) return;
  const size_t q = (size_t)t * a.topk;
  select_token_any(a.logits + (size_t)t * a.E, a.E, a.topk, reinterpret_cast<uint64_t*>(keys2[wave]),
                   sidx[wave], sval[wave], sexp[wave], a.idx + q, a.p + q,
                   a.idx_user ? a.idx_user + q : nullptr, a.p_user ? a.p_user + q : nullptr);
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

// One block: count the pairs of each expert, exclusive prefix sum, then
// scatter the pair ids.  The order of pairs within an expert does not
// affect any result (every pair's outputs are computed independently).
// Also the weight-stationary kernels' tasks, in expert order: expert e's
// pairs in runs of at most kWsSplitPairs, {e | pairs << 16, first pair},
// then {-1, 0} up to ntask_max; and their flags cleared.
__global__ __launch_bounds__(kGroupThreads) void group_kernel(const int* __restrict__ idx,
                                                              int npairs, int E,
                                                              int* __restrict__ ecount,
                                                              int* __restrict__ eoff,
                                                              int* __restrict__ perm,
                                                              int2* __restrict__ tasks,
                                                              int ntask_max,
                                                              int* __restrict__ wsflag) {
  __shared__ int cnt[kGroupThreads];
  __shared__ int wsum[kGroupThreads / kWave];
  const int tid = threadIdx.x;
  cnt[tid] = 0;
  __syncthreads();
  for (int q = tid; q < npairs; q += kGroupThreads) {
    const int e = idx[q];
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  const int c = cnt[tid];   // zero past E
  int total;
  const int start = group_excl_scan(c, wsum, &total);
  if (tid < E) {
    ecount[tid] = c;
    eoff[tid] = start;
    if (wsflag) {
      wsflag[tid] = 0;
      wsflag[E + tid] = 0;
    }
  }
  if (tasks) {
    const int nsplit = (c + kWsSplitPairs - 1) / kWsSplitPairs;
    int ntasks;
    const int t0 = group_excl_scan(nsplit, wsum, &ntasks);
    for (int k = 0; k < nsplit; ++k) {
      const int p0 = k * kWsSplitPairs, n = min(kWsSplitPairs, c - p0);
      tasks[t0 + k] = make_int2(tid | (n << 16), start + p0);
    }
    for (int i = ntasks + tid; i < ntask_max; i += kGroupThreads) tasks[i] = make_int2(-1, 0);
  }
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

// Columns per step, 16-column slices per lane group, and 16-byte B units
// per (pair, limb) and step (see the file header for the column order).
template <bool Q4> struct Step {
  static constexpr int COLS = Q4 ? 256 : 128;
  static constexpr int SL = Q4 ? 4 : 2;
  static constexpr int UPS = 4 * SL;
};

// B (activation) columns live in LDS, for the up to 64 pairs of a pass:
// [slot][limb][16-column unit][16 bytes], slot stride NL * kch + 16 bytes
// (the padding starts consecutive slots 4 banks apart), kch columns at a
// time.  kMmaLds bytes hold all 2048 columns of one limb for 64 slots.
constexpr int kMmaLds = 64 * (2048 + 16);
// Row stride (uint32) of the gate/up dots in LDS: rows 4 apart (the lane
// groups of an MFMA result) land 16 banks apart.
constexpr int kDotRow = 68;
static_assert(2 * kMmaRows * kDotRow * 4 <= kMmaLds, "dots fit the staging area");
// Weight fragment of one step for one matrix: 32 bytes of the lane's row.
struct WFrag {
  u32x4 w[2];
};

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

// 16-byte B unit c (columns 16c .. 16c + 15) of limb l of one activation
// table with K columns: Q8 plane bytes 16c .. 16c + 15; Q4 the 8 even-plane
// bytes at 8c, then the 8 odd-plane bytes of the same columns.
// The table pointers come from LDS, so the compiler cannot tell they are
// global memory; the loads say so (global loads, not flat ones, which would
// also hold up every LDS wait).
typedef __attribute__((address_space(1))) const uint8_t gbyte;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <bool Q4>
__device__ __forceinline__ u32x4 b_unit_load(const uint8_t* tab, int K, int l, int c) {
  gbyte* plane = (gbyte*)(reinterpret_cast<const uint8_t*>(act_plane(tab, K, l)));
  if constexpr (!Q4) {
    return *(__attribute__((address_space(1))) const u32x4*)(plane + (size_t)c * 16);
  } else {
    const u32x2 e = *(__attribute__((address_space(1))) const u32x2*)(plane + (size_t)c * 8);
    const u32x2 o = *(__attribute__((address_space(1))) const u32x2*)(plane + K / 2 + (size_t)c * 8);
    u32x4 r;
    r[0] = e[0]; r[1] = e[1]; r[2] = o[0]; r[3] = o[1];
    return r;
  }
}

// n / d and n % d for n * d < 2^32 (both small here): q = hi32(n * m) with
// m = ceil(2^32 / d), exact in that range.
struct DivMod {
  uint32_t d, m;
  __device__ explicit DivMod(uint32_t dd) : d(dd), m((uint32_t)((0xFFFFFFFFull + dd) / dd)) {}
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return __umulhi(n, m); }
};

// Copies columns [c0, c0 + kch) of the first nlive slots' tables (NL limbs)
// into the LDS layout above; 8 loads in flight per thread.
template <bool Q4, int NL>
__device__ __forceinline__ void stage_b(uint8_t* bbuf, const uint8_t* const* slot_tab, int nlive,
                                        int K, int c0, int kch, int slot_bytes) {
  const int upl = kch / 16;                 // units per limb
  const int ups = NL * upl;                 // units per slot
  const int total = nlive * ups;
  const DivMod by_ups((uint32_t)ups), by_upl((uint32_t)upl);
  for (int base = 0; base < total; base += kMmaThreads * 8) {
    u32x4 r[8];
    int off[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int u = min(base + (int)threadIdx.x + kMmaThreads * i, total - 1);
      const int p = (int)by_ups.div((uint32_t)u), rem = u - p * ups;
      const int l = (int)by_upl.div((uint32_t)rem), c = rem - l * upl;
      r[i] = b_unit_load<Q4>(slot_tab[p], K, l, c0 / 16 + c);
      off[i] = p * slot_bytes + l * kch + c * 16;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (base + (int)threadIdx.x + kMmaThreads * i < total)
        *reinterpret_cast<u32x4*>(bbuf + off[i]) = r[i];
  }
}

// One step (COLS columns) of a pass for ring slot R: at the first step of a
// later chunk, restage B (block-wide, between barriers); issue the weight
// loads of step st + 2 into the slot consumed at step st - 1 (past the last
// step, the last step's bytes again, just loaded and cached, so that every
// step has the same loads in flight); then the MFMAs of step st from slot R
// and the staged B columns.  The ring slot is a template argument so that every
// slot keeps its registers: the only wait before the MFMAs is for slot R's
// own loads.
template <bool Q4, int NM, int NL, int NT, int R>
__device__ __forceinline__ void mma_step(WFrag (&wb)[3][NM], const uint8_t* const W[NM], int st,
                                         int nsteps, int g, const uint8_t* B, int cs,
                                         int slot_bytes, int kch, const uint8_t* const* slot_tab,
                                         int nlive, int K, uint8_t* bbuf, v4i (&acc)[NM][NT][NL]) {
  constexpr int SL = Step<Q4>::SL, UPS = Step<Q4>::UPS, COLS = Step<Q4>::COLS;
  const int sc = st % cs;
  if (sc == 0 && st > 0) {
    __syncthreads();   // the previous chunk is consumed
    stage_b<Q4, NL>(bbuf, slot_tab, nlive, K, st * COLS, kch, slot_bytes);
    __syncthreads();
  }
  const int stl = st + 2 < nsteps ? st + 2 : nsteps - 1;
#pragma unroll
  for (int m = 0; m < NM; ++m) wb[(R + 2) % 3][m] = load_wfrag(W[m], stl, g);
  const uint8_t* Bst = B + sc * UPS * 16;
#pragma unroll
  for (int s = 0; s < SL; ++s) {
    v4i bv[NT][NL];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int l = 0; l < NL; ++l)
        bv[tt][l] = *reinterpret_cast<const v4i*>(Bst + tt * 16 * slot_bytes + l * kch + s * 16);
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const v4i av = a_slice<Q4>(wb[R][m], s);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int l = 0; l < NL; ++l) acc[m][tt][l] = mfma16(av, bv[tt][l], acc[m][tt][l]);
    }
    // keep the next slice's LDS reads after these MFMAs (bounds live B registers)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One pass of a block over up to 16*NT pairs (slot p's activation table at
// slot_tab[p], p < nlive): acc[m][tt][l] = sum over all K columns of
// W_m[lane's row] x table[tt*16 + lane % 16], per limb l.  The activation
// columns are staged in LDS chunk by chunk (as many columns as fit, all K
// of them for one limb); between the two barriers of a chunk the waves run
// free, each streaming its weight rows through a 3-step register ring.
// Every thread of the block calls this.
template <bool Q4, int NM, int NL, int NT>
__device__ __forceinline__ void mma_pass(const uint8_t* const W[NM], int K,
                                         const uint8_t* const* slot_tab, int nlive,
                                         uint8_t* bbuf, v4i (&acc)[NM][NT][NL]) {
  constexpr int COLS = Step<Q4>::COLS, SL = Step<Q4>::SL;
  const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
  const int nsteps = K / COLS;
  // steps per chunk: the largest divisor of nsteps whose columns fit
  int cs = nsteps;
  while (cs > 1 && (nsteps % cs != 0 || 64 * (NL * cs * COLS + 16) > kMmaLds)) --cs;
  const int kch = cs * COLS, slot_bytes = NL * kch + 16;
  const uint8_t* B = bbuf + j * slot_bytes + g * SL * 16;
  // chunk 0 is staged before the weight ring starts, so that waiting for
  // the staging loads does not wait for weight loads
  stage_b<Q4, NL>(bbuf, slot_tab, nlive, K, 0, kch, slot_bytes);
  WFrag wb[3][NM];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    wb[0][m] = load_wfrag(W[m], 0, g);
    wb[1][m] = load_wfrag(W[m], nsteps > 1 ? 1 : 0, g);
  }
  __syncthreads();
  // three steps per iteration, step st reading ring slot st % 3; the loop
  // is left only between steps, so the back edge always sees the same loads
  for (int st = 0;;) {
    mma_step<Q4, NM, NL, NT, 0>(wb, W, st, nsteps, g, B, cs, slot_bytes, kch, slot_tab, nlive, K,
                                bbuf, acc);
    if (++st >= nsteps) break;
    mma_step<Q4, NM, NL, NT, 1>(wb, W, st, nsteps, g, B, cs, slot_bytes, kch, slot_tab, nlive, K,
                                bbuf, acc);
    if (++st >= nsteps) break;
    mma_step<Q4, NM, NL, NT, 2>(wb, W, st, nsteps, g, B, cs, slot_bytes, kch, slot_tab, nlive, K,
                                bbuf, acc);
    if (++st >= nsteps) break;
  }
  __syncthreads();   // LDS free for the next pass
}

template <int NL>
__device__ __forceinline__ uint32_t limb_dot(const v4i* acc_l, int r) {
  int32_t v[4] = {0, 0, 0, 0};
#pragma unroll
  for (int l = 0; l < NL; ++l) v[l] = acc_l[l][r];
  return combine_limbs<NL == 3 ? 4 : NL>(v);
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
  // weight-stationary kernel: flag[e] = 1 for experts left to this kernel
  // (cleared by group_kernel); this kernel: when set, only those experts
  int* flag = nullptr;
  const int* only_flagged = nullptr;
  const int2* tasks = nullptr;  // weight-stationary kernel: its task per blockIdx.y (group_kernel)
};

// Pairs base .. base + n - 1 (n <= 16*NT) of a pass over expert e's pairs
// (tables in slot_tab[]), NT 16-pair tiles: the gate and up dots of this
// block's 128 rows, written to LDS as dots[m][row][pair] (uint32, rows
// kDotRow apart) once the pass has released the staging area.
template <bool Q4, int NL, int NT>
__device__ void gate_up_mma(const GateUpGArgs& a, int e, const uint8_t* const* slot_tab, int base,
                            int n, uint8_t* bbuf) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 16, j = lane % 16;
  const int rowA = blockIdx.x * kMmaRows + wave * 16 + j;   // this lane's A row
  const int rowA_c = rowA < a.dff ? rowA : a.dff - 1;
  const uint8_t* W[2] = {a.gq + ((size_t)e * a.dff + rowA_c) * a.rb,
                         a.uq + ((size_t)e * a.dff + rowA_c) * a.rb};
  v4i acc[2][NT][NL];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int l = 0; l < NL; ++l) acc[m][tt][l] = v4i{0, 0, 0, 0};
  mma_pass<Q4, 2, NL, NT>(W, a.D, slot_tab + base, n, bbuf, acc);
  uint32_t* dots = reinterpret_cast<uint32_t*>(bbuf);
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dots[(m * kMmaRows + wave * 16 + 4 * g + r) * kDotRow + base + tt * 16 + j] =
            limb_dot<NL>(acc[m][tt], r);
}

template <bool Q4>
__device__ void gate_up_epilogue(const GateUpGArgs& a, int e, const int* pass_pair,
                                 const uint32_t* xsum, int base, int n, const uint32_t* dots,
                                 int* red_nl, unsigned* red_sum);

// Live-tile dispatch: 1..4 tiles of 16 pairs; two-limb activations run at
// most two tiles at a time and four-limb ones one tile (the accumulators
// stay in registers).  Each sub-pass's dots go through LDS to the SwiGLU
// epilogue before the next sub-pass restages LDS.
template <bool Q4, int NL>
__device__ __forceinline__ void gate_up_nt(const GateUpGArgs& a, int e, const int* pass_pair,
                                           const uint8_t* const* slot_tab, const uint32_t* xsum,
                                           int n, uint8_t* bbuf, int* red_nl, unsigned* red_sum) {
  constexpr int MAXT = NL == 1 ? 4 : (NL == 2 ? 2 : 1);
  for (int base = 0; base < n; base += 16 * MAXT) {
    const int nb = min(n - base, 16 * MAXT);
    const int nt = (nb + 15) / 16;
    if (nt == 1 || MAXT == 1) gate_up_mma<Q4, NL, 1>(a, e, slot_tab, base, nb, bbuf);
    else if (nt == 2 || MAXT == 2) gate_up_mma<Q4, NL, (MAXT < 2 ? MAXT : 2)>(a, e, slot_tab, base, nb, bbuf);
    else if (nt == 3) gate_up_mma<Q4, NL, (MAXT < 3 ? MAXT : 3)>(a, e, slot_tab, base, nb, bbuf);
    else gate_up_mma<Q4, NL, MAXT>(a, e, slot_tab, base, nb, bbuf);
    __syncthreads();
    gate_up_epilogue<Q4>(a, e, pass_pair, xsum, base, nb, reinterpret_cast<const uint32_t*>(bbuf),
                         red_nl, red_sum);
    __syncthreads();
  }
}

// SwiGLU epilogue of pairs base .. base + n - 1 of a pass (:496-501): wave w
// takes rows 16w .. 16w + 15 of the block, lane p the pass's pair p.  h = (g / (1 + expf(-g))) * u is
// quantized for down, written into the pair's table, and the rows' limb
// count and activation sum go to red_nl / red_sum.
template <bool Q4>
__device__ void gate_up_epilogue(const GateUpGArgs& a, int e, const int* pass_pair,
                                 const uint32_t* xsum, int base, int n, const uint32_t* dots,
                                 int* red_nl, unsigned* red_sum) {
  const int p = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (p < base || p >= base + n) return;
  const int q = pass_pair[p];
  const uint32_t xs = xsum[p];
  const float div = Q4 ? 7.0f : 127.0f;
  uint8_t* tabq = a.htab + (size_t)q * a.htab_bytes;
  int nl = 1;
  uint32_t hs = 0;
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) {
    const int rl = wave * 16 + 4 * r4;                 // local row of 4 consecutive
    const int row0 = blockIdx.x * kMmaRows + rl;
    if (row0 >= a.dff) break;
    uint32_t bytes[4][4];   // [limb][r]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t dg = dots[(rl + r) * kDotRow + p];
      uint32_t du = dots[(kMmaRows + rl + r) * kDotRow + p];
      if (Q4) { dg -= 8u * xs; du -= 8u * xs; }
      const float gv = qdot_epilogue(dg, div, a.gs[(size_t)e * a.dff + row0 + r]);
      const float uv = qdot_epilogue(du, div, a.us[(size_t)e * a.dff + row0 + r]);
      const int32_t hv = f2i_trunc_x86(silu_mul(gv, uv) * div);
      const int nn = limbs_needed(hv);
      nl = nn > nl ? nn : nl;
      hs += (uint32_t)hv;
      uint32_t b[4];
      split_limbs(hv, b);
#pragma unroll
      for (int l = 0; l < 4; ++l) bytes[l][r] = b[l];
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      uint8_t* plane = reinterpret_cast<uint8_t*>(const_cast<uint32_t*>(act_plane(tabq, a.dff, l)));
      if constexpr (!Q4) {
        *reinterpret_cast<uint32_t*>(plane + row0) =
            pack4(bytes[l][0], bytes[l][1], bytes[l][2], bytes[l][3]);
      } else {
        *reinterpret_cast<uint16_t*>(plane + row0 / 2) = (uint16_t)(bytes[l][0] | (bytes[l][2] << 8));
        *reinterpret_cast<uint16_t*>(plane + a.dff / 2 + row0 / 2) =
            (uint16_t)(bytes[l][1] | (bytes[l][3] << 8));
      }
    }
  }
  atomicMax(&red_nl[p], nl);
  atomicAdd(&red_sum[p], hs);
}

template <bool Q4>
__global__ __launch_bounds__(kMmaThreads) void gate_up_grouped_kernel(GateUpGArgs a) {
  extern __shared__ u32x4 lds_b[];
  __shared__ int pass_pair[kPairsPerPass];
  __shared__ const uint8_t* slot_tab[kPairsPerPass];
  __shared__ int red_nl[kPairsPerPass];
  __shared__ unsigned red_sum[kPairsPerPass];
  __shared__ uint32_t pass_xsum[kPairsPerPass];
  uint8_t* bbuf = reinterpret_cast<uint8_t*>(lds_b);
  const int e = blockIdx.y;
  const int n_all = a.ecount[e];
  if (n_all == 0 || (a.only_flagged && !a.only_flagged[e])) return;
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
    if (threadIdx.x < kPairsPerPass) {
      const int i = threadIdx.x;
      const int q = i < n ? a.perm[first + i] : -1;
      pass_pair[i] = q;
      slot_tab[i] = q >= 0 ? a.xtab + (size_t)(q / a.topk) * a.xtab_bytes : nullptr;
      pass_xsum[i] = xsum;
      red_nl[i] = 1;
      red_sum[i] = 0;
    }
    __syncthreads();
    if (nl == 1) gate_up_nt<Q4, 1>(a, e, pass_pair, slot_tab, pass_xsum, n, bbuf, red_nl, red_sum);
    else if (nl == 2) gate_up_nt<Q4, 2>(a, e, pass_pair, slot_tab, pass_xsum, n, bbuf, red_nl, red_sum);
    else gate_up_nt<Q4, 4>(a, e, pass_pair, slot_tab, pass_xsum, n, bbuf, red_nl, red_sum);
    if (threadIdx.x < n) {
      // h segments are 64 rows: this block's 128 rows fill segment 2 bx,
      // segment 2 bx + 1 gets the neutral header
      const int q = pass_pair[threadIdx.x];
      uint32_t* pp = a.hpart + ((size_t)q * a.nseg + 2 * blockIdx.x) * 2;
      pp[0] = (uint32_t)red_nl[threadIdx.x];
      pp[1] = red_sum[threadIdx.x];
      if (2 * (int)blockIdx.x + 1 < a.nseg) {
        pp[2] = 1u;
        pp[3] = 0u;
      }
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
  int* flag = nullptr;               // as in GateUpGArgs
  const int* only_flagged = nullptr;
  const int2* tasks = nullptr;
};

template <bool Q4, int NL, int NT>
__device__ void down_pass(const DownGArgs& a, int e, const int* pass_pair,
                          const uint8_t* const* slot_tab, int base, int n, uint32_t hsum_lane,
                          uint8_t* bbuf) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / 16, j = lane % 16;
  const int rowA = blockIdx.x * kMmaRows + wave * 16 + j;
  const int rowA_c = rowA < a.D ? rowA : a.D - 1;
  const uint8_t* W[1] = {a.dq + ((size_t)e * a.D + rowA_c) * a.rb};
  v4i acc[1][NT][NL];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int l = 0; l < NL; ++l) acc[0][tt][l] = v4i{0, 0, 0, 0};
  mma_pass<Q4, 1, NL, NT>(W, a.dff, slot_tab + base, n, bbuf, acc);
  const float div = Q4 ? 7.0f : 127.0f;
  const int rbase = blockIdx.x * kMmaRows + wave * 16 + 4 * g;
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    const int col = base + tt * 16 + j;
    const int q = tt * 16 + j < n ? pass_pair[col] : -1;
    const uint32_t hs = (uint32_t)__shfl((int)hsum_lane, col, kWave);
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

template <bool Q4, int NL>
__device__ __forceinline__ void down_nt(const DownGArgs& a, int e, const int* pass_pair,
                                        const uint8_t* const* slot_tab, int n, uint32_t hsum,
                                        uint8_t* bbuf) {
  constexpr int MAXT = NL == 4 ? 2 : 4;
  for (int base = 0; base < n; base += 16 * MAXT) {
    const int nb = min(n - base, 16 * MAXT);
    const int nt = (nb + 15) / 16;
    if (nt == 1) down_pass<Q4, NL, 1>(a, e, pass_pair, slot_tab, base, nb, hsum, bbuf);
    else if (nt == 2 || MAXT == 2) down_pass<Q4, NL, 2>(a, e, pass_pair, slot_tab, base, nb, hsum, bbuf);
    else if (nt == 3) down_pass<Q4, NL, 3 < MAXT ? 3 : MAXT>(a, e, pass_pair, slot_tab, base, nb, hsum, bbuf);
    else down_pass<Q4, NL, MAXT>(a, e, pass_pair, slot_tab, base, nb, hsum, bbuf);
  }
}

template <bool Q4>
__global__ __launch_bounds__(kMmaThreads) void down_grouped_kernel(DownGArgs a) {
  extern __shared__ u32x4 lds_b[];
  __shared__ int pass_pair[kPairsPerPass];
  __shared__ const uint8_t* slot_tab[kPairsPerPass];
  uint8_t* bbuf = reinterpret_cast<uint8_t*>(lds_b);
  const int e = blockIdx.y;
  const int n_all = a.ecount[e];
  if (n_all == 0 || (a.only_flagged && !a.only_flagged[e])) return;
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
    if (threadIdx.x < kPairsPerPass) {
      const int i = threadIdx.x;
      const int q = i < n ? a.perm[first + i] : -1;
      pass_pair[i] = q;
      slot_tab[i] = q >= 0 ? a.htab + (size_t)q * a.htab_bytes : nullptr;
    }
    __syncthreads();
    if (nl == 1) down_nt<Q4, 1>(a, e, pass_pair, slot_tab, n, hsum, bbuf);
    else if (nl == 2) down_nt<Q4, 2>(a, e, pass_pair, slot_tab, n, hsum, bbuf);
    else down_nt<Q4, 4>(a, e, pass_pair, slot_tab, n, hsum, bbuf);
    __syncthreads();
  }
}

// ---------------------------------------------------------------- weight-stationary

// The kernels above stream an expert's rows once per pass of up to 64 pairs;
// these keep them in registers instead: each wave owns 16 * RT rows of one
// expert (NM matrices, all K = KS * COLS columns, 8 VGPRs per row tile,
// matrix and step) for the block's whole life, and the expert's pairs
// stream past them through LDS, 16 at a time, double-buffered (the table
// loads of the next pass are in registers while the MFMAs of this one run).
// Every weight byte is read from HBM once per launch.  They take experts
// whose tokens all fit one limb (|x| < 1.0079 for Q8, < 18.3 for Q4, the
// common case) and flag the others (flag[e] = 1), which the streaming
// kernels then process in a second launch.
constexpr int kWsWaves = kMmaWaves;
constexpr int kWsThreads = kWsWaves * kWave;
// Pairs per pass: NT tiles of 16 (each unpacked weight operand feeds NT MFMAs).
template <bool Q4, int KS, int NT>
struct WsShape {
  static constexpr int COLS = Step<Q4>::COLS, SL = Step<Q4>::SL, UPS = Step<Q4>::UPS;
  static constexpr int K = KS * COLS;
  static constexpr int SLOTS = 16 * NT;                     // pairs per pass
  static constexpr int SLOT = K + 16;                       // slot stride (bytes)
  static constexpr int UPL = K / 16;                        // 16-byte units per slot
  static constexpr int U = (SLOTS * UPL + kWsThreads - 1) / kWsThreads;   // per thread
  static constexpr int BUF = SLOTS * SLOT;                  // bytes per staging buffer
  static_assert(2 * BUF <= kMmaLds, "two passes must fit the staging area");
};

// Stores of one pass's table units (loaded into registers) into a staging buffer.
template <bool Q4, int KS, int NT, int U>
__device__ __forceinline__ void ws_commit(const u32x4 (&r)[U], uint8_t* buf, int nlive) {
  using SH = WsShape<Q4, KS, NT>;
  const int total = nlive * SH::UPL;
#pragma unroll
  for (int i = 0; i < SH::U; ++i) {
    const int u = (int)threadIdx.x + kWsThreads * i;
    if (u < total)
      *reinterpret_cast<u32x4*>(buf + (u / SH::UPL) * SH::SLOT + (u % SH::UPL) * 16) = r[i];
  }
}

// acc[m][rt][tt] += W_m[rows of row tile rt] x slots 16 tt .. 16 tt + 15,
// over all K columns, from staging buffer buf.
// PIPE: slice k + 1's B reads and A unpacks are issued before slice k's
// MFMAs, so the LDS latency and the VALU work overlap them (costs registers).
template <bool Q4, int NM, int RT, int KS, int NT, bool PIPE>
__device__ __forceinline__ void ws_mma(const WFrag (&w)[NM][RT][KS], const uint8_t* buf,
                                       v4i (&acc)[NM][RT][NT]) {
  using SH = WsShape<Q4, KS, NT>;
  constexpr int NS = KS * SH::SL;   // slices
  const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
  const uint8_t* B = buf + j * SH::SLOT + g * SH::SL * 16;
  if constexpr (PIPE) {
    v4i bv[NT], av[NM][RT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) bv[tt] = *reinterpret_cast<const v4i*>(B + tt * 16 * SH::SLOT);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) av[m][rt] = a_slice<Q4>(w[m][rt][0], 0);
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      v4i bc[NT], ac[NM][RT];
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) bc[tt] = bv[tt];
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) ac[m][rt] = av[m][rt];
      if (k + 1 < NS) {
        const int st1 = (k + 1) / SH::SL, s1 = (k + 1) % SH::SL;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
          bv[tt] = *reinterpret_cast<const v4i*>(B + tt * 16 * SH::SLOT + (st1 * SH::UPS + s1) * 16);
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) av[m][rt] = a_slice<Q4>(w[m][rt][st1], s1);
      }
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
          for (int tt = 0; tt < NT; ++tt) acc[m][rt][tt] = mfma16(ac[m][rt], bc[tt], acc[m][rt][tt]);
      // bounds the live registers to two slices
      __builtin_amdgcn_sched_barrier(0);
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int st = k / SH::SL, s = k % SH::SL;
    v4i bc[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
      bc[tt] = *reinterpret_cast<const v4i*>(B + tt * 16 * SH::SLOT + (st * SH::UPS + s) * 16);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const v4i av = a_slice<Q4>(w[m][rt][st], s);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) acc[m][rt][tt] = mfma16(av, bc[tt], acc[m][rt][tt]);
      }
    // bounds the live registers to two slices
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The weights become opaque to the compiler at every pass, so that it keeps
// them packed instead of hoisting unpacked copies out of the pass loop.
template <int NM, int RT, int KS>
__device__ __forceinline__ void ws_opaque(WFrag (&w)[NM][RT][KS]) {
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int st = 0; st < KS; ++st)
#pragma unroll
        for (int h = 0; h < 2; ++h) asm volatile("" : "+v"(w[m][rt][st].w[h]));
}

// Pairs of the block's expert, prefetched into LDS at block start (up to
// kWsChunk at a time): pair id and the activation sum of its table; the
// epilogues' limb counts and sums of h (gate/up).
constexpr int kWsChunk = 1024;
struct WsPairs {
  int pair[kWsChunk];
  uint32_t asum[kWsChunk];
  int red_nl[kWsChunk];
  unsigned red_sum[kWsChunk];
  int multi;
};

// The pass loop over pairs [0, n) of the chunk in sp (tables at tab_of(q)):
// epi(acc, i0, nlive) consumes the dots of pairs i0 .. i0 + nlive - 1.  One
// barrier per pass: the next pass's tables are loaded into registers before
// this pass's MFMAs and stored into the other buffer after them.
template <bool Q4, int NM, int RT, int KS, int NT, bool PIPE, class TabOf, class Epi>
__device__ __forceinline__ void ws_passes(WFrag (&w)[NM][RT][KS], int n, const WsPairs& sp,
                                          uint8_t* lds, TabOf&& tab_of, Epi&& epi) {
  using SH = WsShape<Q4, KS, NT>;
  const int npass = (n + SH::SLOTS - 1) / SH::SLOTS;
  auto nlive_of = [&](int P) { return min(SH::SLOTS, n - P * SH::SLOTS); };
  auto issue = [&](u32x4 (&r)[SH::U], int P) {
    const int total = nlive_of(P) * SH::UPL;
#pragma unroll
    for (int i = 0; i < SH::U; ++i) {
      const int u = (int)threadIdx.x + kWsThreads * i;
      if (u < total)
        r[i] = b_unit_load<Q4>(tab_of(sp.pair[P * SH::SLOTS + u / SH::UPL]), SH::K, 0, u % SH::UPL);
    }
  };
  u32x4 r[SH::U];
  issue(r, 0);
  ws_commit<Q4, KS, NT>(r, lds, nlive_of(0));
  __syncthreads();
  for (int P = 0; P < npass; ++P) {
    const int cur = P & 1, nxt = cur ^ 1;
    ws_opaque(w);
    if (P + 1 < npass) issue(r, P + 1);
    v4i acc[NM][RT][NT];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) acc[m][rt][tt] = v4i{0, 0, 0, 0};
    ws_mma<Q4, NM, RT, KS, NT, PIPE>(w, lds + cur * SH::BUF, acc);
    if (P + 1 < npass) ws_commit<Q4, KS, NT>(r, lds + nxt * SH::BUF, nlive_of(P + 1));
    epi(acc, P * SH::SLOTS, nlive_of(P));
    __syncthreads();
  }
}

// This lane's weight fragments: rows row0 + 16 rt + (lane % 16) of the NM
// matrices (rows past nrows read row nrows - 1; their results are dropped).
template <int NM, int RT, int KS>
__device__ __forceinline__ void ws_load_weights(WFrag (&w)[NM][RT][KS], const uint8_t* const* mat,
                                                long long rb, int row0, int nrows) {
  const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = min(row0 + 16 * rt + j, nrows - 1);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int st = 0; st < KS; ++st) w[m][rt][st] = load_wfrag(mat[m] + (size_t)row * rb, st, g);
  }
}

// Prefetch of pairs [c0, c0 + n) of the expert (perm positions first + i):
// info(q) returns {limb count, activation sum} of pair q's table.  Returns
// whether any needs more than one limb (block-wide).
template <class Info>
__device__ __forceinline__ bool ws_prefetch(WsPairs& sp, const int* perm, int first, int c0, int n,
                                            Info&& info) {
  if (threadIdx.x == 0) sp.multi = 0;
  __syncthreads();
  int multi = 0;
  for (int i = threadIdx.x; i < n; i += kWsThreads) {
    const int q = perm[first + c0 + i];
    const int2 v = info(q);
    sp.pair[i] = q;
    sp.asum[i] = (uint32_t)v.y;
    sp.red_nl[i] = 1;
    sp.red_sum[i] = 0;
    multi |= v.x > 1;
  }
  if (multi) atomicOr(&sp.multi, 1);
  __syncthreads();
  return sp.multi != 0;
}

constexpr int kWsDownNT = 1;                      // pair tiles per pass (down)

// gate/up + SwiGLU for the rows 128 * blockIdx.x .. of expert blockIdx.y:
// wave w owns rows 16 w .. 16 w + 15 of the block, both matrices, all K.
template <bool Q4, int KS>
__global__ __launch_bounds__(kWsThreads) void gate_up_ws_kernel(GateUpGArgs a) {
  constexpr int NT = 1;
  extern __shared__ u32x4 lds_b[];
  __shared__ WsPairs sp;
  __shared__ uint64_t exp_tab[32];
  uint8_t* lds = reinterpret_cast<uint8_t*>(lds_b);
  const int2 task = a.tasks[blockIdx.y];
  if (task.x < 0) return;
  const int e = task.x & 0xFFFF, n_all = task.x >> 16, first = task.y;
  if (threadIdx.x < 32) exp_tab[threadIdx.x] = kExp2Tab[threadIdx.x];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, g = lane / 16, j = lane % 16;
  WFrag w[2][1][KS];
  const uint8_t* mats[2] = {a.gq + (size_t)e * a.dff * a.rb, a.uq + (size_t)e * a.dff * a.rb};
  ws_load_weights<2, 1, KS>(w, mats, a.rb, blockIdx.x * kMmaRows + wave * 16, a.dff);
  const int rowq = blockIdx.x * kMmaRows + wave * 16 + 4 * g;   // this lane's 4 result rows
  const bool live_rows = rowq < a.dff;
  float sg[4], su[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = min(rowq + r, a.dff - 1);
    sg[r] = a.gs[(size_t)e * a.dff + row];
    su[r] = a.us[(size_t)e * a.dff + row];
  }
  const float div = Q4 ? 7.0f : 127.0f;
  auto tab_of = [&](int q) { return a.xtab + (size_t)(q / a.topk) * a.xtab_bytes; };
  for (int c0 = 0; c0 < n_all; c0 += kWsChunk) {
    const int n = min(kWsChunk, n_all - c0);
    const bool multi = ws_prefetch(sp, a.perm, first, c0, n, [&](int q) {
      const uint8_t* tb = tab_of(q);
      return make_int2(act_nl(tb), (int)act_asum(tb));
    });
    if (multi) {   // every block of this split sees the same pairs
      if (threadIdx.x == 0) a.flag[e] = 1;
      return;
    }
    auto epi = [&](const v4i (&acc)[2][1][NT], int i0, int nlive) {
      const int i = i0 + (j < nlive ? j : 0);
      int nl = 1;
      uint32_t hs = 0;
      if (j < nlive && live_rows) {
      const int q = sp.pair[i];
      const uint32_t xs = sp.asum[i];
      uint8_t* tabq = a.htab + (size_t)q * a.htab_bytes;
      uint32_t bytes[4][4];   // [limb][r]
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t dg = (uint32_t)acc[0][0][0][r], du = (uint32_t)acc[1][0][0][r];
        if (Q4) { dg -= 8u * xs; du -= 8u * xs; }
        const float gv = qdot_epilogue(dg, div, sg[r]);
        const float uv = qdot_epilogue(du, div, su[r]);
        const int32_t hv = f2i_trunc_x86(silu_mul_t(gv, uv, exp_tab) * div);
        const int nn = limbs_needed(hv);
        nl = nn > nl ? nn : nl;
        hs += (uint32_t)hv;
        uint32_t b[4];
        split_limbs(hv, b);
#pragma unroll
        for (int l = 0; l < 4; ++l) bytes[l][r] = b[l];
      }
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        uint8_t* plane = reinterpret_cast<uint8_t*>(const_cast<uint32_t*>(act_plane(tabq, a.dff, l)));
        if constexpr (!Q4) {
          *reinterpret_cast<uint32_t*>(plane + rowq) =
              pack4(bytes[l][0], bytes[l][1], bytes[l][2], bytes[l][3]);
        } else {
          *reinterpret_cast<uint16_t*>(plane + rowq / 2) = (uint16_t)(bytes[l][0] | (bytes[l][2] << 8));
          *reinterpret_cast<uint16_t*>(plane + a.dff / 2 + rowq / 2) =
              (uint16_t)(bytes[l][1] | (bytes[l][3] << 8));
        }
      }
      }
      // the pair's four row groups (lanes j, j + 16, j + 32, j + 48) combine
      // first: one LDS atomic pair per wave and pair
#pragma unroll
      for (int off = 16; off < kWave; off <<= 1) {
        const int o = __shfl_xor(nl, off, kWave);
        nl = o > nl ? o : nl;
        hs += (uint32_t)__shfl_xor((int)hs, off, kWave);
      }
      if (g == 0 && j < nlive) {
        atomicMax(&sp.red_nl[i], nl);
        atomicAdd(&sp.red_sum[i], hs);
      }
    };
    ws_passes<Q4, 2, 1, KS, NT, true>(w, n, sp, lds, tab_of, epi);
    // this block's two 64-row segments of each pair's h header (the first
    // holds the block's sums, the second the neutral header)
    for (int i = threadIdx.x; i < n; i += kWsThreads) {
      uint32_t* pp = a.hpart + ((size_t)sp.pair[i] * a.nseg + 2 * blockIdx.x) * 2;
      pp[0] = (uint32_t)sp.red_nl[i];
      pp[1] = sp.red_sum[i];
      if (2 * (int)blockIdx.x + 1 < a.nseg) {
        pp[2] = 1u;
        pp[3] = 0u;
      }
    }
    __syncthreads();
  }
}

constexpr int kWsDownRT = 2;                      // row tiles per wave (down)
constexpr int kWsDownRows = kWsWaves * kWsDownRT * 16;

// down for the rows kWsDownRows * blockIdx.x .. of expert blockIdx.y: y per pair.
template <bool Q4, int KS>
__global__ __launch_bounds__(kWsThreads) void down_ws_kernel(DownGArgs a) {
  constexpr int RT = kWsDownRT;
  extern __shared__ u32x4 lds_b[];
  __shared__ WsPairs sp;
  uint8_t* lds = reinterpret_cast<uint8_t*>(lds_b);
  const int2 task = a.tasks[blockIdx.y];
  if (task.x < 0) return;
  const int e = task.x & 0xFFFF, n_all = task.x >> 16, first = task.y;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, g = lane / 16, j = lane % 16;
  WFrag w[1][RT][KS];
  const uint8_t* mats[1] = {a.dq + (size_t)e * a.D * a.rb};
  const int row0 = blockIdx.x * kWsDownRows + wave * RT * 16;
  ws_load_weights<1, RT, KS>(w, mats, a.rb, row0, a.D);
  float sd[RT][4];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int r = 0; r < 4; ++r) sd[rt][r] = a.ds[(size_t)e * a.D + min(row0 + rt * 16 + 4 * g + r, a.D - 1)];
  const float div = Q4 ? 7.0f : 127.0f;
  auto tab_of = [&](int q) { return a.htab + (size_t)q * a.htab_bytes; };
  for (int c0 = 0; c0 < n_all; c0 += kWsChunk) {
    const int n = min(kWsChunk, n_all - c0);
    const bool multi = ws_prefetch(sp, a.perm, first, c0, n, [&](int q) {
      int nl = 1;
      uint32_t hs = 0;
      for (int s = 0; s < a.nseg; ++s) {
        const uint32_t* pp = a.hpart + ((size_t)q * a.nseg + s) * 2;
        nl = (int)pp[0] > nl ? (int)pp[0] : nl;
        hs += pp[1];
      }
      return make_int2(nl, (int)hs);
    });
    if (multi) {
      if (threadIdx.x == 0) a.flag[e] = 1;
      return;
    }
    auto epi = [&](const v4i (&acc)[1][RT][kWsDownNT], int i0, int nlive) {
#pragma unroll
     for (int tt = 0; tt < kWsDownNT; ++tt) {
      if (tt * 16 + j >= nlive) break;
      const int q = sp.pair[i0 + tt * 16 + j];
      const uint32_t hs = sp.asum[i0 + tt * 16 + j];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int row = row0 + rt * 16 + 4 * g;
        if (row >= a.D) continue;
        float yv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          uint32_t d = (uint32_t)acc[0][rt][tt][r];
          if (Q4) d -= 8u * hs;
          yv[r] = qdot_epilogue(d, div, sd[rt][r]);
        }
        *reinterpret_cast<float4*>(a.y + (size_t)q * a.D + row) = make_float4(yv[0], yv[1], yv[2], yv[3]);
      }
     }
    };
    ws_passes<Q4, 1, RT, KS, kWsDownNT, false>(w, n, sp, lds, tab_of, epi);
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

// Dynamic LDS above 64 KB needs the per-kernel attribute (set once per kernel).
std::mutex g_attr_mu;
std::unordered_set<const void*> g_attr_set;

moe_status grouped_lds_attribute(const void* fn) {
  std::lock_guard<std::mutex> lk(g_attr_mu);
  if (g_attr_set.count(fn)) return MOE_OK;
  moe_status st = check_hip(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kMmaLds),
                            "grouped LDS attribute");
  if (st == MOE_OK) g_attr_set.insert(fn);
  return st;
}

using GroupedFn = const void*;

// Weight-stationary kernels exist for 1..8 steps of K (Q4: 256 columns a
// step, Q8: 128); longer rows use the streaming kernels.
template <bool Q4, bool GU>
GroupedFn ws_fn(int ks) {
  switch (ks) {
#define WS_CASE(n) \
  case n: return GU ? (GroupedFn)gate_up_ws_kernel<Q4, n> : (GroupedFn)down_ws_kernel<Q4, n>;
    WS_CASE(1) WS_CASE(2) WS_CASE(3) WS_CASE(4) WS_CASE(5) WS_CASE(6) WS_CASE(7) WS_CASE(8)
#undef WS_CASE
    default: return nullptr;
  }
}

GroupedFn pick_ws(bool q4, bool gate_up, int ks) {
  if (q4) return gate_up ? ws_fn<true, true>(ks) : ws_fn<true, false>(ks);
  return gate_up ? ws_fn<false, true>(ks) : ws_fn<false, false>(ks);
}

template <class Args>
moe_status launch_grouped(GroupedFn fn, dim3 grid, const Args& args, size_t lds, hipStream_t s) {
  moe_status st = grouped_lds_attribute(fn);
  if (st) return st;
  hipLaunchKernelGGL(((void (*)(Args))fn), grid, dim3(kMmaThreads), lds, s, args);
  return check_hip(hipGetLastError(), "grouped launch");
}

// Dynamic LDS of a weight-stationary kernel: two staging buffers.
size_t ws_lds(int nt, int K) { return 2 * (size_t)16 * nt * (K + 16); }

// MOEHIP_GROUPED_WS=0 selects the streaming kernels everywhere.
bool ws_enabled() {
  static const bool v = !(getenv("MOEHIP_GROUPED_WS") && atoi(getenv("MOEHIP_GROUPED_WS")) == 0);
  return v;
}

}  // namespace

moe_status launch_select(const LayerDev* L, int T, int32_t* idx_out, float* p_out, hipStream_t s) {
  SelectArgs sa{L->logits, T, L->E, L->topk, L->idx, L->p, idx_out, p_out};
  dim3 sg((unsigned)((T + kSelectWaves - 1) / kSelectWaves));
  hipLaunchKernelGGL(select_kernel, sg, dim3(kSelectWaves * kWave), 0, s, sa);
  return check_hip(hipGetLastError(), "select launch");
}

bool grouped_ok(const LayerDev* L) {
  const int step = L->dtype == 3 ? 256 : 128;
  return L->D % step == 0 && L->dff % step == 0 && L->D % 128 == 0 && L->E <= kGroupThreads &&
         is16(L->router_w);
}

constexpr int kPackOverlapTokens = 1024;

moe_status layer_forward_grouped(LayerDev* L, const float* xn, const float* resid, int T,
                                 float* out, int32_t* idx_out, float* p_out) {
  hipStream_t s = stream();
  const bool q4 = L->dtype == 3;
  moe_status st;
  if (!is16(xn) || !is16(out) || (resid && !is16(resid)))
    return set_error(MOE_ERR_ARG, "grouped forward: arrays must be 16-byte aligned");
  // 1. x tables; for many tokens on the side stream, where they overlap the
  // router, the selection and the grouping and are joined before gate/up
  // (the fork and join cost ~8 us: more than the packing saves below ~1024
  // tokens, measured)
  QShape sh;
  sh.dtype = L->dtype; sh.M = T; sh.N = 1; sh.K = L->D; sh.lda = L->D; sh.ldc = 1;
  sh.rs = L->rbg;
  QJob one{nullptr, nullptr, xn, nullptr};
  const bool overlap = T >= kPackOverlapTokens;
  if (overlap) {
    hipStream_t s2 = side_stream();
    if ((st = check_hip(hipEventRecord(fork_event(), s), "fork record")) ||
        (st = check_hip(hipStreamWaitEvent(s2, fork_event(), 0), "fork wait")) ||
        (st = check_hip(launch_act_pack(sh, nullptr, one, 1, L->xtab, s2), "act pack")) ||
        (st = check_hip(hipEventRecord(join_event(), s2), "join record")))
      return st;
  } else if ((st = check_hip(launch_act_pack(sh, nullptr, one, 1, L->xtab, s), "act pack"))) {
    return st;
  }
  // 2. router logits
  RouterTileArgs ra{xn, L->router_w, L->router_b, L->logits, T, L->D, L->E};
  // one chain per lane below 2048 tokens (2x2 chains per lane left three
  // quarters of the SIMDs idle at T = 512; 256-column chunks were no
  // faster); from 2048 tokens two token chains per lane (512 blocks at E =
  // 128, a third fewer LDS reads per product: T = 2048 layer 449 -> 437 us,
  // no gain at 1024), measured
  st = T >= 2048 ? launch_router_tile<2, 1, 128>(ra, s) : launch_router_tile<1, 1, 128>(ra, s);
  if (st) return st;
  // 3. top-k and gates
  if ((st = launch_select(L, T, idx_out, p_out, s))) return st;
  // 4. group pairs by expert
  const int npairs = T * L->topk;
  const int ntask_max = npairs / kWsSplitPairs + L->E + 1;
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(kGroupThreads), 0, s, L->idx, npairs, L->E,
                     L->ecount, L->eoff, L->perm, L->tasks, ntask_max, L->wsflag);
  if ((st = check_hip(hipGetLastError(), "group launch"))) return st;
  if (overlap && (st = check_hip(hipStreamWaitEvent(s, join_event(), 0), "join wait"))) return st;
  // 5. gate/up + SwiGLU
  const int nseg = 2 * ((L->dff + kMmaRows - 1) / kMmaRows);   // h header segments of 64 rows
  GateUpGArgs ga{L->gq, L->gs, L->uq, L->us, L->rbg, L->D, L->dff, L->topk,
                 L->ecount, L->eoff, L->perm, L->xtab, act_table_bytes(L->D),
                 L->htab, act_table_bytes(L->dff), L->hpart, nseg};
  dim3 gg((unsigned)((L->dff + kMmaRows - 1) / kMmaRows), (unsigned)L->E);
  // weight-stationary kernels where the rows fit registers; experts with
  // multi-limb activations (flagged by them) go to the streaming kernels
  const int cols = q4 ? 256 : 128;
  const bool ws = ws_enabled();
  const GroupedFn gu_stream =
      q4 ? (GroupedFn)gate_up_grouped_kernel<true> : (GroupedFn)gate_up_grouped_kernel<false>;
  const GroupedFn gu_ws = ws ? pick_ws(q4, true, L->D / cols) : nullptr;
  if (gu_ws) {
    ga.flag = L->wsflag;
    ga.tasks = L->tasks;
    const dim3 ggw(gg.x, (unsigned)ntask_max);
    if ((st = launch_grouped(gu_ws, ggw, ga, ws_lds(1, L->D), s))) return st;
    ga.flag = nullptr;
    ga.tasks = nullptr;
    ga.only_flagged = L->wsflag;
  }
  if ((st = launch_grouped(gu_stream, gg, ga, kMmaLds, s))) return st;
  // 6. down
  DownGArgs da{L->dq, L->ds, L->rbd, L->D, L->dff, L->ecount, L->eoff, L->perm,
               L->htab, act_table_bytes(L->dff), L->hpart, nseg, L->y};
  const GroupedFn dn_stream =
      q4 ? (GroupedFn)down_grouped_kernel<true> : (GroupedFn)down_grouped_kernel<false>;
  const GroupedFn dn_ws = ws ? pick_ws(q4, false, L->dff / cols) : nullptr;
  if (dn_ws) {
    da.flag = L->wsflag + L->E;
    da.tasks = L->tasks;
    dim3 dgw((unsigned)((L->D + kWsDownRows - 1) / kWsDownRows), (unsigned)ntask_max);
    if ((st = launch_grouped(dn_ws, dgw, da, ws_lds(kWsDownNT, L->dff), s))) return st;
    da.flag = nullptr;
    da.tasks = nullptr;
    da.only_flagged = L->wsflag + L->E;
  }
  dim3 dg((unsigned)((L->D + kMmaRows - 1) / kMmaRows), (unsigned)L->E);
  if ((st = launch_grouped(dn_stream, dg, da, kMmaLds, s))) return st;
  // 7. ordered combine + residual
  dim3 cg((unsigned)((L->D / 4 + 255) / 256), (unsigned)T);
  hipLaunchKernelGGL(combine_kernel, cg, dim3(256), 0, s, L->y, L->idx, L->p, resid, out, L->D,
                     L->topk);
  return check_hip(hipGetLastError(), "combine launch");
}

}  // namespace moe
