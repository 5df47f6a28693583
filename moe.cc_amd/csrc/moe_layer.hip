// moe_layer.hip - the MoE block of one Qwen3-MoE layer on gfx950
// (test_model_trace.c:460-517), bit-identical to the reference.
//
// Launch sequence of one forward (T tokens):
//   [rmsnorm]   x_norm = rmsnorm(x, rms2_w)          (block forward only; :461)
//   router      logits[t,e] = sum_k x_norm[t,k] * Wr[e,k], k ascending,
//               separate roundings (:465 -> :213-227), + bias (:466-468);
//               top-k by the insertion rule (:480 -> :275-288), softmax over
//               the selected logits (:482-487); packs x_norm[t] for the
//               expert GEMVs.  One block of 1024 threads per token.
//   tasks       groups the T*k (token, rank) pairs by expert, ascending
//               (token, rank) inside an expert: one task per routed expert,
//               so an expert's weights are read once for all its tokens.
//   gate_up     per task and row chunk: g = Q(x Wg), u = Q(x Wu), both exact
//               integer dots; h = (g / (1 + expf(-g))) * u  (:496-501)
//   pack_h      packs every h row for the down GEMV
//   down        per task and row chunk: y = Q(h Wd)  (:502-503)
//   combine     out[t] = x_resid[t] + (((0 + p0 y0) + p1 y1) + ...), ranks in
//               order, each product and sum rounded on its own (:513, :517)
// The router's sequential sum runs as one add chain per (token, expert):
// 8 lanes hold 32 consecutive products and lane 0 of the group adds them in
// k order through DPP row shifts (v_add_f32_dpp), so a wave carries 8 chains.
#include <algorithm>
#include <cstring>
#include <new>
#include <type_traits>
#include <vector>

#include "moe_device.h"
#include "moe_lib.h"
#include "moe_qtile.h"

namespace moe {

struct LayerDev {
  int dtype = 2, D = 0, dff = 0, E = 0, topk = 0;
  long long rbg = 0, rbd = 0;          // row bytes of gate/up and of down
  float* router_w = nullptr;           // [E][D]
  float* router_b = nullptr;           // [E] or null
  float* rms2_w = nullptr;             // [D] or null
  uint8_t* gq = nullptr; float* gs = nullptr;   // [E][dff][rbg], [E][dff]
  uint8_t* uq = nullptr; float* us = nullptr;
  uint8_t* dq = nullptr; float* ds = nullptr;   // [E][D][rbd], [E][D]
  // per-forward scratch, grown to the largest T seen
  int capT = 0;
  float* logits = nullptr;   // [T][E]
  int* idx = nullptr;        // [T][topk]
  float* p = nullptr;        // [T][topk]
  uint8_t* xtab = nullptr;   // [T] packed x_norm rows
  uint8_t* htab = nullptr;   // [T*topk] packed h rows
  float* h = nullptr;        // [T*topk][dff]
  float* y = nullptr;        // [T*topk][D]
  float* xn = nullptr;       // [T][D] normed input (block forward)
  int* tasks = nullptr;      // [0]=U, expert[E], start[E], count[E], pairs[T*topk]
};

namespace {

constexpr int kRouterThreads = 1024;
constexpr int kRouterWaves = kRouterThreads / kWave;
constexpr int kMaxTopK = 32;

template <int J>
__device__ __forceinline__ float shl8(float v) {
  if constexpr (J == 0) return v;
  else return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + J, 0xF, 0xF, true));
}

// acc + p_m(lane+J), m = 0..3, in that order
template <int J>
__device__ __forceinline__ float chain4(float acc, float p0, float p1, float p2, float p3) {
  acc = acc + shl8<J>(p0);
  acc = acc + shl8<J>(p1);
  acc = acc + shl8<J>(p2);
  acc = acc + shl8<J>(p3);
  return acc;
}

// Sequential fp32 dot of x[0..D) with row w (test_model_trace.c:221-222):
// lanes 8g..8g+7 of a wave cooperate on one row; the result is valid in lane
// 8g.  Requires D % 32 == 0 and 16-byte aligned x and w.
__device__ __forceinline__ float seq_dot_group8(const float* __restrict__ x,
                                                const float* __restrict__ w, int D, bool live) {
  const int j = threadIdx.x % 8;
  float acc = 0.0f;
  float4 wa = live ? *reinterpret_cast<const float4*>(w + 4 * j) : make_float4(0, 0, 0, 0);
  float4 xa = *reinterpret_cast<const float4*>(x + 4 * j);
  for (int k0 = 0; k0 < D; k0 += 32) {
    float4 wn = make_float4(0, 0, 0, 0), xn = make_float4(0, 0, 0, 0);
    if (k0 + 32 < D) {
      if (live) wn = *reinterpret_cast<const float4*>(w + k0 + 32 + 4 * j);
      xn = *reinterpret_cast<const float4*>(x + k0 + 32 + 4 * j);
    }
    const float p0 = xa.x * wa.x, p1 = xa.y * wa.y, p2 = xa.z * wa.z, p3 = xa.w * wa.w;
    acc = chain4<0>(acc, p0, p1, p2, p3);
    acc = chain4<1>(acc, p0, p1, p2, p3);
    acc = chain4<2>(acc, p0, p1, p2, p3);
    acc = chain4<3>(acc, p0, p1, p2, p3);
    acc = chain4<4>(acc, p0, p1, p2, p3);
    acc = chain4<5>(acc, p0, p1, p2, p3);
    acc = chain4<6>(acc, p0, p1, p2, p3);
    acc = chain4<7>(acc, p0, p1, p2, p3);
    wa = wn;
    xa = xn;
  }
  return acc;
}

template <bool Q4>
__global__ __launch_bounds__(kRouterThreads) void router_topk_kernel(
    const float* __restrict__ xn, int D, int E, int topk, const float* __restrict__ Wr,
    const float* __restrict__ rb, float* __restrict__ logits_out, int* __restrict__ idx_out,
    float* __restrict__ p_out, uint8_t* __restrict__ xtab, size_t tab_bytes, int fast) {
  extern __shared__ float lds[];
  float* lg = lds;                                   // [E]
  int* rank = reinterpret_cast<int*>(lds + E);       // [E]
  __shared__ int slot_idx[kMaxTopK];
  __shared__ float slot_val[kMaxTopK];
  __shared__ float slot_exp[kMaxTopK];
  __shared__ float inv_sum;
  __shared__ int scratch[2];
  const int t = blockIdx.x;
  const float* x = xn + (size_t)t * D;
  const int tid = threadIdx.x;

  // 1. logits
  if (fast) {
    const int wave = tid / kWave, g = (tid % kWave) / 8;
    for (int e0 = 0; e0 < E; e0 += kRouterWaves * 8) {
      const int e = e0 + wave * 8 + g;
      const bool live = e < E;
      const float acc = seq_dot_group8(x, Wr + (size_t)(live ? e : 0) * D, D, live);
      if (live && (tid % 8) == 0) lg[e] = rb ? acc + rb[e] : acc;
    }
  } else {
    for (int e = tid; e < E; e += blockDim.x) {
      const float* w = Wr + (size_t)e * D;
      float acc = 0.0f;
      for (int k = 0; k < D; ++k) {
        const float pk = x[k] * w[k];
        acc = acc + pk;
      }
      lg[e] = rb ? acc + rb[e] : acc;
    }
  }
  for (int e = tid; e < E; e += blockDim.x) rank[e] = 0;
  if (tid < topk) { slot_idx[tid] = -1; slot_val[tid] = -__builtin_inff(); }
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) logits_out[(size_t)t * E + e] = lg[e];

  // 2. top-k: rank of e = #{c : v_c > v_e} + #{c < e : v_c == v_e}; NaN and
  //    -inf are never selected (insertion rule of test_model_trace.c:275-288)
  const int tpe = E <= (int)blockDim.x ? (int)blockDim.x / E : 1;
  for (int i = tid; i < tpe * E; i += blockDim.x) {
    const int e = i / tpe, part = i % tpe;
    const float v = lg[e];
    int cnt = 0;
    for (int c = part; c < E; c += tpe) {
      const float vc = lg[c];
      cnt += (vc > v) || (vc == v && c < e);
    }
    atomicAdd(&rank[e], cnt);
  }
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    const float v = lg[e];
    const int r = rank[e];
    if (v > -__builtin_inff() && r < topk) { slot_idx[r] = e; slot_val[r] = v; }
  }
  __syncthreads();

  // 3. softmax over the selected logits (:482-487)
  if (tid < topk) {
    float mx = slot_val[0];
    for (int i = 1; i < topk; ++i) if (slot_val[i] > mx) mx = slot_val[i];
    slot_exp[tid] = expf_glibc(slot_val[tid] - mx);
  }
  __syncthreads();
  if (tid == 0) {
    float sum = 0.0f;
    for (int i = 0; i < topk; ++i) sum = sum + slot_exp[i];
    inv_sum = 1.0f / (sum + 1e-9f);
  }
  __syncthreads();
  if (tid < topk) {
    idx_out[(size_t)t * topk + tid] = slot_idx[tid];
    p_out[(size_t)t * topk + tid] = slot_exp[tid] * inv_sum;
  }

  // 4. packed activations of x_norm[t] for the gate/up GEMVs
  pack_act_row<Q4>(x, D, xtab + (size_t)t * tab_bytes, scratch);
}

// Groups the (token, rank) pairs by expert: task u = u-th routed expert in
// ascending id; its pairs in ascending pair id = t*topk + j.
__global__ __launch_bounds__(256) void build_tasks_kernel(const int* __restrict__ idx, int npairs,
                                                          int E, int* __restrict__ tasks) {
  extern __shared__ int cnt[];   // [E] counts then [E] starts
  int* start = cnt + E;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
    for (int q = 0; q < npairs; ++q) c += idx[q] == e;
    cnt[e] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int u = 0, s = 0;
    for (int e = 0; e < E; ++e) {
      start[e] = s;
      if (cnt[e] > 0) {
        tasks[1 + u] = e;
        tasks[1 + E + u] = s;
        tasks[1 + 2 * E + u] = cnt[e];
        ++u;
      }
      s += cnt[e];
    }
    tasks[0] = u;
  }
  __syncthreads();
  int* pairs = tasks + 1 + 3 * E;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    if (cnt[e] == 0) continue;
    int o = start[e];
    for (int q = 0; q < npairs; ++q)
      if (idx[q] == e) pairs[o++] = q;
  }
}

constexpr int kMTok = 4;   // token slots per block pass in the expert kernels

// Marks the untiled expert path: one wave per row, int32 arithmetic on the
// fp32 activations (any row size; used for small or irregular layers).
struct GenericGeom {
  static constexpr int WR = 1;
};

// Epilogue of gate/up: h[pair, row] = silu(g) * u
struct GateUpEpiMaker {
  const float* gs;
  const float* us;
  float* h;
  const int* pairs;   // this task's pairs
  int n, dff;
  float div;
  template <int MTI>
  struct Epi {
    const float* gs;
    const float* us;
    float* h;
    const int* pairs;
    int n, dff;
    float div;
    int t0;
    template <class Tot>
    __device__ void operator()(int row, const Tot& tot) const {
      const float sg = gs[row], su = us[row];
#pragma unroll
      for (int t = 0; t < MTI; ++t) {
        if (t0 + t >= n) break;
        const float g = qdot_epilogue(tot[0][t], div, sg);
        const float u = qdot_epilogue(tot[1][t], div, su);
        h[(size_t)pairs[t0 + t] * dff + row] = silu_mul(g, u);
      }
    }
  };
  template <int MTI>
  __device__ Epi<MTI> at(int t0) const { return Epi<MTI>{gs, us, h, pairs, n, dff, div, t0}; }
};

// Epilogue of down: y[pair, row] = Q(h Wd)
struct DownEpiMaker {
  const float* ds;
  float* y;
  const int* pairs;
  int n, D;
  float div;
  template <int MTI>
  struct Epi {
    const float* ds;
    float* y;
    const int* pairs;
    int n, D;
    float div;
    int t0;
    template <class Tot>
    __device__ void operator()(int row, const Tot& tot) const {
      const float sc = ds[row];
#pragma unroll
      for (int t = 0; t < MTI; ++t) {
        if (t0 + t >= n) break;
        y[(size_t)pairs[t0 + t] * D + row] = qdot_epilogue(tot[0][t], div, sc);
      }
    }
  };
  template <int MTI>
  __device__ Epi<MTI> at(int t0) const { return Epi<MTI>{ds, y, pairs, n, D, div, t0}; }
};

struct GateUpArgs {
  const uint8_t* gq; const float* gs; const uint8_t* uq; const float* us;
  long long rb; int D, dff, E, topk;
  const int* tasks; const uint8_t* xtab; size_t tab_bytes; const float* xn;
  float* h; int rows_per_block;
};

template <bool Q4, class G>
__global__ __launch_bounds__(kTileBlock) void gate_up_kernel(GateUpArgs a) {
  const int u = blockIdx.y;
  if (u >= a.tasks[0]) return;
  const int e = a.tasks[1 + u], st = a.tasks[1 + a.E + u], n = a.tasks[1 + 2 * a.E + u];
  const int* pairs = a.tasks + 1 + 3 * a.E + st;
  const int r0 = blockIdx.x * a.rows_per_block;
  const int r1 = r0 + a.rows_per_block < a.dff ? r0 + a.rows_per_block : a.dff;
  const uint8_t* W[2] = {a.gq + (size_t)e * a.dff * a.rb, a.uq + (size_t)e * a.dff * a.rb};
  for (int c0 = 0; c0 < n; c0 += kMTok) {
    const int nt = n - c0 < kMTok ? n - c0 : kMTok;
    const uint8_t* tabs[kMTok];
    const float* xs[kMTok];
#pragma unroll
    for (int t = 0; t < kMTok; ++t) {
      const int tok = pairs[c0 + (t < nt ? t : nt - 1)] / a.topk;
      tabs[t] = a.xtab + (size_t)tok * a.tab_bytes;
      xs[t] = a.xn + (size_t)tok * a.D;
    }
    GateUpEpiMaker mk{a.gs + (size_t)e * a.dff, a.us + (size_t)e * a.dff, a.h, pairs + c0, nt,
                      a.dff, Q4 ? 7.0f : 127.0f};
    if constexpr (std::is_same<G, GenericGeom>::value) {
      for (int t = 0; t < nt; ++t) {
        auto epi = mk.template at<1>(t);
        generic_rows_fp32<Q4, 2>(W, a.rb, a.D, xs[t], r0, r1, epi);
      }
    } else {
      stream_tokens<Q4, G, 2, kMTok>(W, a.rb, a.D, tabs, xs, nt, r0, r1, mk);
    }
  }
}

template <bool Q4>
__global__ __launch_bounds__(256) void pack_h_kernel(const float* __restrict__ h, int dff,
                                                     const int* __restrict__ idx,
                                                     uint8_t* __restrict__ htab, size_t tab_bytes) {
  __shared__ int scratch[2];
  const int q = blockIdx.x;
  if (idx[q] < 0) return;
  pack_act_row<Q4>(h + (size_t)q * dff, dff, htab + (size_t)q * tab_bytes, scratch);
}

struct DownArgs {
  const uint8_t* dq; const float* ds; long long rb; int D, dff, E;
  const int* tasks; const uint8_t* htab; size_t tab_bytes; const float* h;
  float* y; int rows_per_block;
};

template <bool Q4, class G>
__global__ __launch_bounds__(kTileBlock) void down_kernel(DownArgs a) {
  const int u = blockIdx.y;
  if (u >= a.tasks[0]) return;
  const int e = a.tasks[1 + u], st = a.tasks[1 + a.E + u], n = a.tasks[1 + 2 * a.E + u];
  const int* pairs = a.tasks + 1 + 3 * a.E + st;
  const int r0 = blockIdx.x * a.rows_per_block;
  const int r1 = r0 + a.rows_per_block < a.D ? r0 + a.rows_per_block : a.D;
  const uint8_t* W[1] = {a.dq + (size_t)e * a.D * a.rb};
  for (int c0 = 0; c0 < n; c0 += kMTok) {
    const int nt = n - c0 < kMTok ? n - c0 : kMTok;
    const uint8_t* tabs[kMTok];
    const float* xs[kMTok];
#pragma unroll
    for (int t = 0; t < kMTok; ++t) {
      const int q = pairs[c0 + (t < nt ? t : nt - 1)];
      tabs[t] = a.htab + (size_t)q * a.tab_bytes;
      xs[t] = a.h + (size_t)q * a.dff;
    }
    DownEpiMaker mk{a.ds + (size_t)e * a.D, a.y, pairs + c0, nt, a.D, Q4 ? 7.0f : 127.0f};
    if constexpr (std::is_same<G, GenericGeom>::value) {
      for (int t = 0; t < nt; ++t) {
        auto epi = mk.template at<1>(t);
        generic_rows_fp32<Q4, 1>(W, a.rb, a.dff, xs[t], r0, r1, epi);
      }
    } else {
      stream_tokens<Q4, G, 1, kMTok>(W, a.rb, a.dff, tabs, xs, nt, r0, r1, mk);
    }
  }
}

__global__ void combine_kernel(const float* __restrict__ y, const float* __restrict__ p,
                               const int* __restrict__ idx, const float* __restrict__ resid,
                               float* __restrict__ out, int T, int D, int topk) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)T * D) return;
  const int t = (int)(i / D), o = (int)(i % D);
  float acc = 0.0f;
  for (int j = 0; j < topk; ++j) {
    const int q = t * topk + j;
    if (idx[q] < 0) continue;
    const float py = p[q] * y[(size_t)q * D + o];
    acc = acc + py;
  }
  out[i] = resid ? resid[i] + acc : acc;
}

// rmsnorm (test_model_trace.c:241-255): one wave per token; the sum of
// squares is one sequential chain in lane 0 (8 lanes feed it through DPP).
__global__ __launch_bounds__(64) void rmsnorm_kernel(const float* __restrict__ x,
                                                     const float* __restrict__ w,
                                                     float* __restrict__ y, int D, float eps,
                                                     int fast) {
  __shared__ float inv_s;
  const int t = blockIdx.x;
  const float* xt = x + (size_t)t * D;
  if (fast) {
    // 8 chains would be computed by the 8 groups of the wave; only group 0's
    // lane 0 carries the real one (D-long), the others are idle copies.
    const float acc = seq_dot_group8(xt, xt, D, true);
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
moe_status dev_alloc(T** p, size_t count) {
  *p = nullptr;
  if (count == 0) return MOE_OK;
  return check_hip(hipMalloc((void**)p, count * sizeof(T)), "hipMalloc(layer)");
}

moe_status ensure_scratch(LayerDev* L, int T) {
  if (T <= L->capT) return MOE_OK;
  moe_status st = check_hip(hipStreamSynchronize(stream()), "sync");
  if (st) return st;
  hipFree(L->logits); hipFree(L->idx); hipFree(L->p); hipFree(L->xtab); hipFree(L->htab);
  hipFree(L->h); hipFree(L->y); hipFree(L->xn); hipFree(L->tasks);
  L->capT = 0;
  const size_t np = (size_t)T * L->topk;
  if ((st = dev_alloc(&L->logits, (size_t)T * L->E))) return st;
  if ((st = dev_alloc(&L->idx, np))) return st;
  if ((st = dev_alloc(&L->p, np))) return st;
  if ((st = dev_alloc(&L->xtab, (size_t)T * act_table_bytes(L->D)))) return st;
  if ((st = dev_alloc(&L->htab, np * act_table_bytes(L->dff)))) return st;
  if ((st = dev_alloc(&L->h, np * L->dff))) return st;
  if ((st = dev_alloc(&L->y, np * L->D))) return st;
  if ((st = dev_alloc(&L->xn, (size_t)T * L->D))) return st;
  if ((st = dev_alloc(&L->tasks, 1 + 3 * (size_t)L->E + np))) return st;
  L->capT = T;
  return MOE_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

template <bool Q4, class G>
void launch_gate_up(const LayerDev* L, const float* xn, int T, int U_max, hipStream_t s) {
  constexpr int unit = kTileWaves * G::WR;
  const long long total = (long long)L->dff * std::min(U_max, T * L->topk);
  long long rpb = (total + 1023) / 1024;
  rpb = std::max<long long>(unit, (rpb + unit - 1) / unit * unit);
  rpb = std::min<long long>(rpb, 8 * unit);
  GateUpArgs a{L->gq, L->gs, L->uq, L->us, L->rbg, L->D, L->dff, L->E, L->topk, L->tasks,
               L->xtab, act_table_bytes(L->D), xn, L->h, (int)rpb};
  dim3 grid((unsigned)((L->dff + rpb - 1) / rpb), (unsigned)U_max);
  hipLaunchKernelGGL((gate_up_kernel<Q4, G>), grid, dim3(kTileBlock), 0, s, a);
}

template <bool Q4, class G>
void launch_down(const LayerDev* L, int T, int U_max, hipStream_t s) {
  constexpr int unit = kTileWaves * G::WR;
  const long long total = (long long)L->D * std::min(U_max, T * L->topk);
  long long rpb = (total + 1023) / 1024;
  rpb = std::max<long long>(unit, (rpb + unit - 1) / unit * unit);
  rpb = std::min<long long>(rpb, 8 * unit);
  DownArgs a{L->dq, L->ds, L->rbd, L->D, L->dff, L->E, L->tasks, L->htab,
             act_table_bytes(L->dff), L->h, L->y, (int)rpb};
  dim3 grid((unsigned)((L->D + rpb - 1) / rpb), (unsigned)U_max);
  hipLaunchKernelGGL((down_kernel<Q4, G>), grid, dim3(kTileBlock), 0, s, a);
}

// Row-byte dispatch for the expert GEMVs (same geometries as gemv.hip).
template <bool Q4, class F>
bool with_geom(long long rb, F&& f) {
  switch (rb) {
    case 192:  f(TileGeom<3, 4>()); return true;
    case 256:  f(TileGeom<4, 4>()); return true;
    case 384:  f(TileGeom<3, 8>()); return true;
    case 512:  f(TileGeom<4, 8>()); return true;
    case 768:  f(TileGeom<3, 16>()); return true;
    case 1024: f(TileGeom<4, 16>()); return true;
    case 1536: f(TileGeom<3, 32>()); return true;
    case 2048: f(TileGeom<4, 32>()); return true;
    case 3072: f(TileGeom<3, 64>()); return true;
    case 4096: f(TileGeom<4, 64>()); return true;
    default: f(GenericGeom()); return true;
  }
}

}  // namespace

moe_status layer_forward(LayerDev* L, const float* xn, const float* resid, int T, float* out,
                         int32_t* idx_out, float* p_out) {
  if (T <= 0) return MOE_OK;
  moe_status st = ensure_scratch(L, T);
  if (st) return st;
  hipStream_t s = stream();
  const bool q4 = L->dtype == 3;
  const int fast = (L->D % 32 == 0) && aligned16(xn) && aligned16(L->router_w);
  const size_t lds = 2 * (size_t)L->E * sizeof(float);
  if (q4)
    hipLaunchKernelGGL(router_topk_kernel<true>, dim3(T), dim3(kRouterThreads), lds, s, xn, L->D,
                       L->E, L->topk, L->router_w, L->router_b, L->logits, L->idx, L->p, L->xtab,
                       act_table_bytes(L->D), fast);
  else
    hipLaunchKernelGGL(router_topk_kernel<false>, dim3(T), dim3(kRouterThreads), lds, s, xn, L->D,
                       L->E, L->topk, L->router_w, L->router_b, L->logits, L->idx, L->p, L->xtab,
                       act_table_bytes(L->D), fast);
  if ((st = check_hip(hipGetLastError(), "router launch"))) return st;
  const int npairs = T * L->topk;
  hipLaunchKernelGGL(build_tasks_kernel, dim3(1), dim3(256), 2 * (size_t)L->E * sizeof(int), s,
                     L->idx, npairs, L->E, L->tasks);
  if ((st = check_hip(hipGetLastError(), "tasks launch"))) return st;
  const int U_max = std::min(L->E, npairs);
  bool ok = q4 ? with_geom<true>(L->rbg, [&](auto g) { launch_gate_up<true, decltype(g)>(L, xn, T, U_max, s); })
               : with_geom<false>(L->rbg, [&](auto g) { launch_gate_up<false, decltype(g)>(L, xn, T, U_max, s); });
  if (!ok) return set_error(MOE_ERR_UNSUPPORTED, "gate/up row bytes %lld have no tiled geometry", L->rbg);
  if ((st = check_hip(hipGetLastError(), "gate_up launch"))) return st;
  if (q4)
    hipLaunchKernelGGL(pack_h_kernel<true>, dim3(npairs), dim3(256), 0, s, L->h, L->dff, L->idx,
                       L->htab, act_table_bytes(L->dff));
  else
    hipLaunchKernelGGL(pack_h_kernel<false>, dim3(npairs), dim3(256), 0, s, L->h, L->dff, L->idx,
                       L->htab, act_table_bytes(L->dff));
  if ((st = check_hip(hipGetLastError(), "pack_h launch"))) return st;
  ok = q4 ? with_geom<true>(L->rbd, [&](auto g) { launch_down<true, decltype(g)>(L, T, U_max, s); })
          : with_geom<false>(L->rbd, [&](auto g) { launch_down<false, decltype(g)>(L, T, U_max, s); });
  if (!ok) return set_error(MOE_ERR_UNSUPPORTED, "down row bytes %lld have no tiled geometry", L->rbd);
  if ((st = check_hip(hipGetLastError(), "down launch"))) return st;
  const size_t n = (size_t)T * L->D;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, L->y,
                     L->p, L->idx, resid, out, T, L->D, L->topk);
  if ((st = check_hip(hipGetLastError(), "combine launch"))) return st;
  if (idx_out)
    if ((st = check_hip(hipMemcpyAsync(idx_out, L->idx, (size_t)npairs * 4, hipMemcpyDeviceToDevice, s), "idx copy"))) return st;
  if (p_out)
    if ((st = check_hip(hipMemcpyAsync(p_out, L->p, (size_t)npairs * 4, hipMemcpyDeviceToDevice, s), "p copy"))) return st;
  return MOE_OK;
}

moe_status rmsnorm_dev(const float* x, const float* w, float* y, int T, int D, float eps) {
  if (T <= 0) return MOE_OK;
  const int fast = (D % 32 == 0) && aligned16(x);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(64), 0, stream(), x, w, y, D, eps, fast);
  return check_hip(hipGetLastError(), "rmsnorm launch");
}

}  // namespace moe

using namespace moe;

struct moe_layer { LayerDev L; };

namespace {

moe_status upload(void* dst, const void* src, size_t bytes, int on_device) {
  if (!bytes) return MOE_OK;
  return check_hip(hipMemcpyAsync(dst, src, bytes, on_device ? hipMemcpyDeviceToDevice
                                                              : hipMemcpyHostToDevice, stream()),
                   "layer upload");
}

void free_layer(LayerDev& L) {
  hipFree(L.router_w); hipFree(L.router_b); hipFree(L.rms2_w);
  hipFree(L.gq); hipFree(L.gs); hipFree(L.uq); hipFree(L.us); hipFree(L.dq); hipFree(L.ds);
  hipFree(L.logits); hipFree(L.idx); hipFree(L.p); hipFree(L.xtab); hipFree(L.htab);
  hipFree(L.h); hipFree(L.y); hipFree(L.xn); hipFree(L.tasks);
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
  const int dtype = lw->Wg_q[0].dtype;
  const long long rbg = dtype == 2 ? D : D / 2, rbd = dtype == 2 ? dff : dff / 2;
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
  return layer_forward(&layer->L, x_norm, x_resid, T, out, idx_out, p_out);
}

moe_status moe_block_forward(moe_layer* layer, const float* x, int T, float* out, float eps) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!layer || !x || !out) return set_error(MOE_ERR_ARG, "block_forward: null argument");
  if (T < 0) return set_error(MOE_ERR_ARG, "block_forward: T < 0");
  LayerDev* L = &layer->L;
  if (T == 0) return MOE_OK;
  if ((st = ensure_scratch(L, T))) return st;
  if ((st = rmsnorm_dev(x, L->rms2_w, L->xn, T, L->D, eps))) return st;
  return layer_forward(L, L->xn, x, T, out, nullptr, nullptr);
}

moe_status moe_rmsnorm_dev(const float* x, const float* w, float* y, int T, int D, float eps) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!x || !y || T < 0 || D <= 0) return set_error(MOE_ERR_ARG, "rmsnorm: bad argument");
  return rmsnorm_dev(x, w, y, T, D, eps);
}

moe_status moe_layer_debug_buffers(moe_layer* layer, const float** logits, const float** h,
                                   const float** y) {
  if (!layer) return set_error(MOE_ERR_ARG, "debug_buffers: null layer");
  if (logits) *logits = layer->L.logits;
  if (h) *h = layer->L.h;
  if (y) *y = layer->L.y;
  return MOE_OK;
}

}  // extern "C"
