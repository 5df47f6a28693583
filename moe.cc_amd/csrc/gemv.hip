// gemv.hip - rowwise Q8 / Q4 matrix-times-vectors kernels for gfx950.
//
// Semantics: kernels.c:51-74 (Q8) and kernels.c:96-128 (Q4), bit for bit.
//   a_k  = (int32)(A[m,k] * 127.0f)        (Q8; 7.0f for Q4), x86 truncation
//   dot  = sum_k a_k * w[n,k]               wrapping int32, any order (exact)
//   C    = ((float)dot / 127.0f) * s[n]     (7.0f for Q4)
//
// Two launches per call:
//   1. act_pack: every activation row -> packed limb table (moe_qtile.h),
//      once, into a workspace;
//   2. qgemv_tiled: each block owns a chunk of rows of one job; its waves
//      load their slice of the activation table into registers once, then
//      stream rows with double-buffered dwordx4 loads (LPR lanes per row, a
//      row = LPR*P*16 bytes), dot on v_dot4_i32_i8 and reduce across the
//      row's lanes with DPP.  No LDS, no block barriers in the main loop.
// Shapes without a tiled geometry (row bytes not LPR*P*16, unaligned rows,
// odd-K Q4) and Q4 activations that need 4 limbs use a one-wave-per-row
// kernel with plain int32 arithmetic on the fp32 activations.
#include <cstdlib>

#include "moe_device.h"
#include "moe_internal.h"
#include "moe_qtile.h"

namespace moe {
namespace {

constexpr int kBlock = kTileBlock;
constexpr int kWaves = kTileWaves;
// LDS for the fused kernel's activation tables at most (four token slots of
// K = 2048 take 32.8 KiB; larger products pack into a workspace first).
constexpr size_t kFusedTableLds = 40 * 1024;

struct TiledArgs {
  QShape sh;
  const QJob* jobs;     // device array, or nullptr -> `one`
  QJob one;
  const uint8_t* tabs;  // packed activations, [job][m] tables of tab_bytes
  size_t tab_bytes;
  int shared_tabs;      // 1: every job uses job 0's tables
  int blocks_per_job;
  int rows_per_block;
};

__device__ __forceinline__ QJob get_job(const TiledArgs& a, int j) {
  return a.jobs ? a.jobs[j] : a.one;
}

template <bool Q4>
__global__ __launch_bounds__(kBlock) void act_pack_kernel(QShape sh, const QJob* __restrict__ jobs,
                                                          QJob one, uint8_t* __restrict__ tabs,
                                                          size_t tab_bytes) {
  __shared__ int scratch[2];
  const int j = blockIdx.x, m = blockIdx.y;
  const QJob job = jobs ? jobs[j] : one;
  if (j > 0 && job.A == jobs[0].A) return;   // shares job 0's activations and tables
  pack_act_row<Q4>(job.A + (size_t)m * sh.lda, sh.K, tabs + ((size_t)j * sh.M + m) * tab_bytes,
                   scratch);
}

// Epilogue of the plain GEMV: y = ((float)dot / div) * S[row], staged in
// the block's LDS buffer Y[t][row - r0] (t = token slot of the block) and
// written to C by the whole block at the end (gemv_write_outputs): one
// coalesced, nontemporal burst per block instead of a 4-byte store per row
// group in the middle of the weight stream (measured ~1.5% faster; the
// output writes, ~1% of the bytes, still cost ~8% of the streaming rate on
// the box, wherever in the launch they are placed).
constexpr int kYRows = 512;   // rows per block, at most
constexpr int kLdsPerCU = 160 * 1024;

struct GemvEpiMaker {
  const float* S;
  float* Y;
  int ldy, M, mbase, r0;
  float div;
  template <int MTI>
  struct Epi {
    const float* S;
    float* Y;
    int ldy, M, m0, tb, r0;   // token m0 + t lives in slot tb + t
    float div;
    using Pre = float;
    __device__ Pre pre(int row) const { return S[row]; }
    template <class Tot>
    __device__ void operator()(int row, const Tot& tot, float sc) const {
#pragma unroll
      for (int t = 0; t < MTI; ++t)
        if (m0 + t < M) Y[(tb + t) * ldy + (row - r0)] = qdot_epilogue(tot[0][t], div, sc);
    }
    template <class Tot>
    __device__ void operator()(int row, const Tot& tot) const { (*this)(row, tot, S[row]); }
  };
  template <int MTI>
  __device__ Epi<MTI> at(int t0) const { return Epi<MTI>{S, Y, ldy, M, mbase + t0, t0, r0, div}; }
};

// The block's staged outputs to C (after every wave has finished its rows).
__device__ __forceinline__ void gemv_write_outputs(const float* Y, int ldy, float* C, int ldc,
                                                   int mbase, int ntok, int r0, int r1) {
  __syncthreads();
  const int n = r1 - r0;
  for (int t = 0; t < ntok; ++t) {
    float* c = C + (size_t)(mbase + t) * ldc + r0;
    for (int i = (int)threadIdx.x; i < n; i += (int)blockDim.x) __builtin_nontemporal_store(Y[t * ldy + i], c + i);
  }
}

template <bool Q4, class G, int MT>
__global__ __launch_bounds__(kBlock) void qgemv_tiled(TiledArgs a) {
  const int job_id = blockIdx.x / a.blocks_per_job;
  const int r0 = (blockIdx.x % a.blocks_per_job) * a.rows_per_block;
  const int r1 = r0 + a.rows_per_block < a.sh.N ? r0 + a.rows_per_block : a.sh.N;
  const QJob job = get_job(a, job_id);
  const int mbase = blockIdx.y * MT;
  const int ntok = a.sh.M - mbase < MT ? a.sh.M - mbase : MT;
  // jobs whose activations are job 0's use job 0's packed tables
  const int tab_job =
      (a.shared_tabs || (a.jobs && job_id > 0 && job.A == a.jobs[0].A)) ? 0 : job_id;
  const uint8_t* tabs[MT];
  const float* xs[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int m = mbase + (t < ntok ? t : ntok - 1);
    tabs[t] = a.tabs + ((size_t)tab_job * a.sh.M + m) * a.tab_bytes;
    xs[t] = job.A + (size_t)m * a.sh.lda;
  }
  const uint8_t* W[1] = {job.W};
  __shared__ float ybuf[MT * kYRows];
  GemvEpiMaker mk{job.S, ybuf, kYRows, a.sh.M, mbase, r0, Q4 ? 7.0f : 127.0f};
  stream_tokens<Q4, G, 1, MT>(W, a.sh.rs, a.sh.K, tabs, xs, ntok, r0, r1, mk);
  gemv_write_outputs(ybuf, kYRows, job.C, a.sh.ldc, mbase, ntok, r0, r1);
}

// The reads of a batch-1 tiled launch and nothing else: the same blocks,
// rows per block, wave walk (row groups wave, wave + 4, ..., two groups of
// loads in flight), nontemporal 16-byte weight loads, per-row scale loads and
// LDS-capped blocks per CU as qgemv_tiled<Q4, G, 1>, with the words folded
// into one XOR per wave instead of the dots.  Its rate is what the GEMV's own
// access order allows on the same pool.
template <class G>
__global__ __launch_bounds__(kBlock) void rows_read_kernel(TiledArgs a, uint32_t* sink) {
  const int job_id = blockIdx.x / a.blocks_per_job;
  const int r0 = (blockIdx.x % a.blocks_per_job) * a.rows_per_block;
  const int r1 = r0 + a.rows_per_block < a.sh.N ? r0 + a.rows_per_block : a.sh.N;
  const QJob job = get_job(a, job_id);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int g = lane / G::LPR;
  const int ngroups = (r1 - r0 + G::WR - 1) / G::WR;
  constexpr int PF = 2;
  uint32_t w[PF][G::DW];
  uint32_t sc[PF];
  uint32_t acc = 0;
  auto load = [&](int gi, uint32_t (&d)[G::DW], uint32_t& s) {
    const int row = r0 + gi * G::WR + g;
    s = __float_as_uint(job.S[row < r1 ? row : r0]);
    if (row < r1) {
      load_row_regs<G>(job.W + (size_t)row * (size_t)a.sh.rs, d);
    } else {
#pragma unroll
      for (int i = 0; i < G::DW; ++i) d[i] = 0;
    }
  };
#pragma unroll
  for (int i = 0; i < PF; ++i)
    if (wave + i * kWaves < ngroups) load(wave + i * kWaves, w[i], sc[i]);
  for (int base = 0;; base += PF) {
    bool done = false;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int gi = wave + (base + i) * kWaves;
      if (gi >= ngroups) { done = true; break; }
      // the row's scale once (lane 0 of its lane group), past-the-end rows none
      if (lane % G::LPR == 0 && r0 + gi * G::WR + g < r1) acc ^= sc[i];
#pragma unroll
      for (int j = 0; j < G::DW; ++j) acc ^= w[i][j];
      const int gn = gi + PF * kWaves;
      if (gn < ngroups) load(gn, w[i], sc[i]);
    }
    if (done) break;
  }
  // one atomic a block, on one of the sink's four words (tens of thousands
  // of atomics on one address would serialise behind the loads)
  __shared__ uint32_t wx[kWaves];
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, kWave);
  if (lane == 0) wx[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t b = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) b ^= wx[i];
    if (b != 0u) atomicXor(sink + (blockIdx.x & 3), b);
  }
}

// One activation row into an LDS table (the layout act_pack writes): a
// first pass over x for the limb count and sum (block reduction), a second
// that writes the planes those values need -- all four when `all_planes`
// (a block of several rows reads as many planes as its largest count).
// Whole block; barriers.
template <bool Q4>
__device__ void pack_act_row_lds(const float* __restrict__ x, int K, uint8_t* tab, int* scratch,
                                 bool all_planes) {
  const float mult = Q4 ? 7.0f : 127.0f;
  constexpr int V = Q4 ? 8 : 4;
  const size_t plane = (((size_t)K + 15) / 16) * 16;
  uint32_t* p0 = reinterpret_cast<uint32_t*>(tab + 16);
  const int nd = (K + V - 1) / V;
  if (threadIdx.x == 0) { scratch[0] = 1; scratch[1] = 0; }
  __syncthreads();
  int32_t lo = 0, hi = 0;
  uint32_t part = 0;
  for (int d = threadIdx.x; d < nd; d += blockDim.x)
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int k = V * d + i;
      const int32_t v = k < K ? f2i_trunc_x86(x[k] * mult) : 0;
      lo = v < lo ? v : lo;
      hi = v > hi ? v : hi;
      part += (uint32_t)v;
    }
  block_max_sum(max(limbs_needed(lo), limbs_needed(hi)), part, scratch);
  __syncthreads();
  const int nl = scratch[0];
  const int nw = all_planes ? 4 : nl;
  if (threadIdx.x == 0) {
    reinterpret_cast<int*>(tab)[0] = nl;
    reinterpret_cast<uint32_t*>(tab)[1] = (uint32_t)scratch[1];
  }
  for (int d = threadIdx.x; d < nd; d += blockDim.x) {
    uint32_t b[V][4];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int k = V * d + i;
      split_limbs(k < K ? f2i_trunc_x86(x[k] * mult) : 0, b[i]);
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      if (l >= nw) break;
      uint32_t* pl = p0 + (size_t)l * (plane / 4);
      if constexpr (!Q4) {
        pl[d] = pack4(b[0][l], b[1][l], b[2][l], b[3][l]);
      } else {
        const int KW = (K + 7) / 8;
        pl[d] = pack4(b[0][l], b[2][l], b[4][l], b[6][l]);
        pl[KW + d] = pack4(b[1][l], b[3][l], b[5][l], b[7][l]);
      }
    }
  }
}

// qgemv_tiled with the activation tables built by each block in its own LDS
// (dynamic, ntok tables of tab_bytes) from the fp32 rows: one launch for a
// product instead of act_pack + qgemv_tiled.  x (K floats) is re-read from
// cache by every block; only the planes the values need are written.
template <bool Q4, class G, int MT>
__global__ __launch_bounds__(kBlock) void qgemv_fused(TiledArgs a) {
  extern __shared__ u32x4 lds_tabs[];
  __shared__ int scratch[2];
  const int job_id = blockIdx.x / a.blocks_per_job;
  const int r0 = (blockIdx.x % a.blocks_per_job) * a.rows_per_block;
  const int r1 = r0 + a.rows_per_block < a.sh.N ? r0 + a.rows_per_block : a.sh.N;
  const QJob job = get_job(a, job_id);
  const int mbase = blockIdx.y * MT;
  const int ntok = a.sh.M - mbase < MT ? a.sh.M - mbase : MT;
  uint8_t* lt = reinterpret_cast<uint8_t*>(lds_tabs);
  for (int t = 0; t < ntok; ++t) {
    pack_act_row_lds<Q4>(job.A + (size_t)(mbase + t) * a.sh.lda, a.sh.K, lt + (size_t)t * a.tab_bytes,
                         scratch, ntok > 1);
    __syncthreads();
  }
  const uint8_t* tabs[MT];
  const float* xs[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int tt = t < ntok ? t : ntok - 1;
    tabs[t] = lt + (size_t)tt * a.tab_bytes;
    xs[t] = job.A + (size_t)(mbase + tt) * a.sh.lda;
  }
  const uint8_t* W[1] = {job.W};
  __shared__ float ybuf[MT * kYRows];
  GemvEpiMaker mk{job.S, ybuf, kYRows, a.sh.M, mbase, r0, Q4 ? 7.0f : 127.0f};
  stream_tokens<Q4, G, 1, MT>(W, a.sh.rs, a.sh.K, tabs, xs, ntok, r0, r1, mk);
  gemv_write_outputs(ybuf, kYRows, job.C, a.sh.ldc, mbase, ntok, r0, r1);
}

template <bool Q4>
__global__ __launch_bounds__(kBlock) void qgemv_generic(QShape sh, const QJob* __restrict__ jobs,
                                                        QJob one, int blocks_per_job) {
  const int job_id = blockIdx.x / blocks_per_job;
  const int r0 = (blockIdx.x % blocks_per_job) * kWaves;
  const int r1 = r0 + kWaves < sh.N ? r0 + kWaves : sh.N;
  const QJob job = jobs ? jobs[job_id] : one;
  const int m0 = blockIdx.y * 16;
  const int m1 = m0 + 16 < sh.M ? m0 + 16 : sh.M;
  const uint8_t* W[1] = {job.W};
  __shared__ float ybuf[16 * kWaves];
  GemvEpiMaker mk{job.S, ybuf, kWaves, sh.M, m0, r0, Q4 ? 7.0f : 127.0f};
  for (int m = m0; m < m1; ++m) {
    auto epi = mk.at<1>(m - m0);
    generic_rows_fp32<Q4, 1>(W, sh.rs, sh.K, job.A + (size_t)m * sh.lda, r0, r1, epi);
  }
  gemv_write_outputs(ybuf, kWaves, job.C, sh.ldc, m0, m1 - m0, r0, r1);
}

// fp32 path: one thread per output, k ascending, unfused multiply then add.
__global__ __launch_bounds__(kBlock) void f32gemv_seq(const float* __restrict__ A,
                                                      const float* __restrict__ W,
                                                      float* __restrict__ C, int M, int N, int K,
                                                      int lda, int ldw, int ldc) {
  const long long i = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (i >= (long long)M * N) return;
  const int m = (int)(i / N), n = (int)(i % N);
  const float* a = A + (size_t)m * lda;
  const float* w = W + (size_t)n * ldw;
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    const float p = a[k] * w[k];
    acc = acc + p;
  }
  C[(size_t)m * ldc + n] = acc;
}

__global__ void zero_fill(float* p, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// Read-only stream of n16 16-byte words: the plain HBM read rate on a pass
// over data that no cache holds, reported beside the GEMV's.  The blocks
// sweep the span together, tile t (8 words a thread, eight
// nontemporal 16-byte loads in flight: the GEMV's load kind) by block t mod
// the grid, and the words fold into one XOR per wave (so that no load is
// dead), combined into *sink.
constexpr int kStreamUnroll = 8;
__global__ __launch_bounds__(kBlock) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                             uint32_t* sink) {
  constexpr size_t tile = (size_t)kStreamUnroll * kBlock;
  const size_t ntiles = n16 / tile;
  uint32_t acc = 0;
  for (size_t t = blockIdx.x; t < ntiles; t += gridDim.x) {
    const u32x4* q = p + t * tile + threadIdx.x;
    u32x4 v[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) v[u] = __builtin_nontemporal_load(q + u * kBlock);
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (size_t i = ntiles * tile + (size_t)blockIdx.x * kBlock + threadIdx.x; i < n16;
       i += (size_t)gridDim.x * kBlock) {
    const u32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, kWave);
  if (threadIdx.x % kWave == 0 && acc != 0u) atomicXor(sink, acc);
}

// ---- host-side variant selection ----
using TiledFn = void (*)(TiledArgs);

using ReadFn = void (*)(TiledArgs, uint32_t*);

struct Variant {
  TiledFn fn;
  TiledFn fused;   // the same with the activation tables built in LDS
  ReadFn read;     // its reads alone (rows_read_kernel)
  int wr;          // rows per wave group
  int mt;
  const char* name;
};

template <bool Q4, class G, int MT>
Variant make_variant(const char* name) {
  return Variant{qgemv_tiled<Q4, G, MT>, qgemv_fused<Q4, G, MT>, rows_read_kernel<G>, G::WR, MT, name};
}

// Row byte counts with a tiled geometry: LPR lanes x P dwordx4 x 16 bytes.
template <bool Q4, int MT>
bool pick_tiled(long long rb, Variant* v) {
  switch (rb) {
    case 192:  *v = make_variant<Q4, TileGeom<3, 4>, MT>("tiled_p3l4"); return true;
    case 256:  *v = make_variant<Q4, TileGeom<4, 4>, MT>("tiled_p4l4"); return true;
    case 384:  *v = make_variant<Q4, TileGeom<3, 8>, MT>("tiled_p3l8"); return true;
    case 512:  *v = make_variant<Q4, TileGeom<4, 8>, MT>("tiled_p4l8"); return true;
    case 768:  *v = make_variant<Q4, TileGeom<3, 16>, MT>("tiled_p3l16"); return true;
    case 1024: *v = make_variant<Q4, TileGeom<4, 16>, MT>("tiled_p4l16"); return true;
    case 1536: *v = make_variant<Q4, TileGeom<3, 32>, MT>("tiled_p3l32"); return true;
    case 2048: *v = make_variant<Q4, TileGeom<4, 32>, MT>("tiled_p4l32"); return true;
    case 3072: *v = make_variant<Q4, TileGeom<3, 64>, MT>("tiled_p3l64"); return true;
    case 4096: *v = make_variant<Q4, TileGeom<4, 64>, MT>("tiled_p4l64"); return true;
    default: return false;
  }
}

bool select_tiled(const QShape& sh, const void* w_base, Variant* v) {
  const bool q4 = sh.dtype == 3;
  if (q4 && (sh.K & 1)) return false;
  if (sh.K <= 0) return false;
  const long long rb = q4 ? sh.K / 2 : sh.K;
  if (sh.rs != rb) return false;
  if (w_base && ((uintptr_t)w_base % 16) != 0) return false;
  const int mt = sh.M == 1 ? 1 : (sh.M == 2 ? 2 : 4);
  if (q4) {
    if (mt == 1) return pick_tiled<true, 1>(rb, v);
    if (mt == 2) return pick_tiled<true, 2>(rb, v);
    return pick_tiled<true, 4>(rb, v);
  }
  if (mt == 1) return pick_tiled<false, 1>(rb, v);
  if (mt == 2) return pick_tiled<false, 2>(rb, v);
  return pick_tiled<false, 4>(rb, v);
}

// Workspace for packed activation tables (grown on demand; freed never).
uint8_t* g_ws = nullptr;
size_t g_ws_bytes = 0;

hipError_t ensure_ws(size_t need) {
  if (need <= g_ws_bytes) return hipSuccess;
  if (g_ws) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    (void)hipFree(g_ws);
  }
  g_ws = nullptr;
  g_ws_bytes = 0;
  size_t cap = need < ((size_t)1 << 20) ? ((size_t)1 << 20) : need + need / 2;
  hipError_t e = hipMalloc(&g_ws, cap);
  if (e == hipSuccess) g_ws_bytes = cap;
  return e;
}

}  // namespace

void release_gemv_workspace() {
  if (g_ws) (void)hipFree(g_ws);
  g_ws = nullptr;
  g_ws_bytes = 0;
}

const char* qgemv_variant_name(const QShape& sh, const void* w_base) {
  Variant v;
  if (select_tiled(sh, w_base, &v)) return v.name;
  return "generic";
}

hipError_t launch_act_pack(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                           uint8_t* tabs, hipStream_t stream) {
  const size_t tb = act_table_bytes(sh.K);
  if (sh.dtype == 3)
    hipLaunchKernelGGL(act_pack_kernel<true>, dim3(njobs, sh.M), dim3(kBlock), 0, stream, sh,
                       jobs_dev, one, tabs, tb);
  else
    hipLaunchKernelGGL(act_pack_kernel<false>, dim3(njobs, sh.M), dim3(kBlock), 0, stream, sh,
                       jobs_dev, one, tabs, tb);
  return hipGetLastError();
}

// The geometry of a tiled launch: arguments, grid and (batch-1 launches from
// tables) the dynamic LDS that caps the blocks a CU holds.
struct TiledPlan {
  Variant v;
  TiledArgs a;
  dim3 grid;
  size_t pad;
};

static bool plan_tiled(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                       const uint8_t* tabs, int shared_tabs, TiledPlan* pl) {
  Variant& v = pl->v;
  if (!select_tiled(sh, jobs_dev ? nullptr : one.W, &v)) return false;
  // rows per block: a multiple of (waves x rows per wave group), large
  // enough to amortise the activation loads, small enough for >= target
  // blocks (tuning knobs MOEHIP_GEMV_BLOCKS, MOEHIP_GEMV_MAX_GROUPS)
  static const int target = getenv("MOEHIP_GEMV_BLOCKS") ? atoi(getenv("MOEHIP_GEMV_BLOCKS")) : 2048;
  static const int max_groups = getenv("MOEHIP_GEMV_MAX_GROUPS") ? atoi(getenv("MOEHIP_GEMV_MAX_GROUPS")) : 8;
  const int unit = kWaves * v.wr;
  const long long total_rows = (long long)sh.N * njobs;
  long long rpb = (total_rows + target - 1) / target;
  rpb = (rpb + unit - 1) / unit * unit;
  if (rpb < unit) rpb = unit;
  if (rpb > (long long)max_groups * unit) rpb = (long long)max_groups * unit;
  if (rpb > kYRows) rpb = kYRows / unit * unit;   // the staging buffer's rows
  if (rpb > sh.N) rpb = (sh.N + unit - 1) / unit * unit;
  TiledArgs& a = pl->a;
  a.sh = sh;
  a.jobs = jobs_dev;
  a.one = one;
  a.tabs = tabs;
  a.tab_bytes = act_table_bytes(sh.K);
  a.shared_tabs = shared_tabs;
  a.rows_per_block = (int)rpb;
  a.blocks_per_job = (int)((sh.N + rpb - 1) / rpb);
  pl->grid = dim3((unsigned)((long long)a.blocks_per_job * njobs), (unsigned)((sh.M + v.mt - 1) / v.mt));
  // Batch-1 launches from tables cap the blocks a CU holds through dynamic
  // LDS that the kernel does not use: measured on 1 GiB pools (alternating
  // runs), fewer resident blocks read HBM faster -- 5 a CU for rows under 1
  // KB (Q4 down [2048 x 768]: 6.43-6.51 uncapped, 6.48-6.58 with 4 a CU,
  // 6.59-6.60 with 5, 6.24-6.27 with 3), 3 for longer rows (Q4 gate [768 x
  // 2048]: 6.67-6.72 -> 6.71-6.78, Q8 gate 6.57-6.63 -> 6.68-6.76; 2 a CU
  // alike).
  pl->pad = 0;
  if (tabs && sh.M == 1) {
    const int cap = sh.rs >= 1024 ? 3 : 5;
    pl->pad = ((size_t)kLdsPerCU / cap - (size_t)v.mt * kYRows * 4 - 256) / 512 * 512;
  }
  return true;
}

// tabs == nullptr: the fused kernel (tables in LDS, lds bytes per block).
static hipError_t launch_tiled(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                        const uint8_t* tabs, int shared_tabs, size_t lds, hipStream_t stream) {
  TiledPlan pl;
  if (!plan_tiled(sh, jobs_dev, one, njobs, tabs, shared_tabs, &pl)) return hipErrorInvalidValue;
  if (tabs)
    hipLaunchKernelGGL(pl.v.fn, pl.grid, dim3(kBlock), pl.pad, stream, pl.a);
  else
    hipLaunchKernelGGL(pl.v.fused, pl.grid, dim3(kBlock), lds, stream, pl.a);
  return hipGetLastError();
}

hipError_t launch_rows_read(const QShape& sh, const QJob* jobs_dev, int njobs, int blocks_per_cu,
                            uint32_t* sink, hipStream_t stream) {
  if (sh.M != 1 || blocks_per_cu < 0 || blocks_per_cu > 8) return hipErrorInvalidValue;
  TiledPlan pl;
  const QJob none{nullptr, nullptr, nullptr, nullptr};
  // any non-null tables pointer: the plan of a launch from packed tables
  if (!plan_tiled(sh, jobs_dev, none, njobs, reinterpret_cast<const uint8_t*>(sink), 1, &pl))
    return hipErrorInvalidValue;
  // the GEMV's LDS per block (its output staging plus the cap's padding),
  // or the padding of another cap
  size_t lds = pl.pad + (size_t)pl.v.mt * kYRows * 4;
  if (blocks_per_cu > 0) lds = ((size_t)kLdsPerCU / blocks_per_cu - 256) / 512 * 512;
  hipLaunchKernelGGL(pl.v.read, pl.grid, dim3(kBlock), lds, stream, pl.a, sink);
  return hipGetLastError();
}

hipError_t launch_qgemv_tables(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                               const uint8_t* tabs, int shared_tabs, hipStream_t stream) {
  if (!tabs) return hipErrorInvalidValue;
  return launch_tiled(sh, jobs_dev, one, njobs, tabs, shared_tabs, 0, stream);
}

size_t act_table_size(int K) { return act_table_bytes(K); }

bool qgemv_tiled_ok(const QShape& sh, const void* w_base) {
  Variant v;
  return select_tiled(sh, w_base, &v);
}

hipError_t launch_qgemv(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                        hipStream_t stream) {
  if (sh.M <= 0 || sh.N <= 0 || njobs <= 0) return hipSuccess;
  if (sh.dtype != 2 && sh.dtype != 3) return hipErrorInvalidValue;
  // With a device job array the host cannot see the pointers; callers of the
  // batched entry point guarantee 16-byte aligned packed rows (capi.cpp).
  if (qgemv_tiled_ok(sh, jobs_dev ? nullptr : one.W)) {
    const size_t tb = act_table_bytes(sh.K);
    // one product whose token slots' tables fit in LDS: one fused launch
    // (for many products packing once first is faster: measured 175 against
    // 189 us for 1366 batch-1 GEMVs of [2048 x 768])
    const int slots = sh.M == 1 ? 1 : (sh.M == 2 ? 2 : 4);   // select_tiled's token slots per block
    const size_t lds = tb * (size_t)(sh.M < slots ? sh.M : slots);
    if (njobs == 1 && lds <= kFusedTableLds)
      return launch_tiled(sh, jobs_dev, one, njobs, nullptr, 0, lds, stream);
    hipError_t e = ensure_ws(tb * (size_t)njobs * (size_t)sh.M);
    if (e != hipSuccess) return e;
    e = launch_act_pack(sh, jobs_dev, one, njobs, g_ws, stream);
    if (e != hipSuccess) return e;
    return launch_qgemv_tables(sh, jobs_dev, one, njobs, g_ws, 0, stream);
  }
  const int bpj = (sh.N + kWaves - 1) / kWaves;
  dim3 grid((unsigned)((long long)bpj * njobs), (unsigned)((sh.M + 15) / 16));
  if (sh.dtype == 3)
    hipLaunchKernelGGL(qgemv_generic<true>, grid, dim3(kBlock), 0, stream, sh, jobs_dev, one, bpj);
  else
    hipLaunchKernelGGL(qgemv_generic<false>, grid, dim3(kBlock), 0, stream, sh, jobs_dev, one, bpj);
  return hipGetLastError();
}

hipError_t launch_f32gemv(const float* A, const float* W, float* C, int M, int N, int K, int lda,
                          int ldw, int ldc, hipStream_t stream) {
  const long long total = (long long)M * N;
  if (total <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)((total + kBlock - 1) / kBlock);
  hipLaunchKernelGGL(f32gemv_seq, dim3(blocks), dim3(kBlock), 0, stream, A, W, C, M, N, K, lda,
                     ldw, ldc);
  return hipGetLastError();
}

hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream) {
  const size_t n16 = bytes / 16;
  if (n16 == 0) return hipSuccess;
  // four blocks a CU (256 CUs; measured on quantized weights: 6.0 TB/s, 5.6
  // with eight, 4.3 with sixteen), fewer for small spans
  const size_t tile = (size_t)kStreamUnroll * kBlock;
  const size_t want = (n16 + tile - 1) / tile;
  const unsigned blocks = (unsigned)(want < 1024 ? want : 1024);
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(kBlock), 0, stream,
                     reinterpret_cast<const u32x4*>(src), n16, sink);
  return hipGetLastError();
}

hipError_t launch_zero(float* C, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((n + kBlock - 1) / kBlock);
  hipLaunchKernelGGL(zero_fill, dim3(blocks), dim3(kBlock), 0, stream, C, n);
  return hipGetLastError();
}

}  // namespace moe
