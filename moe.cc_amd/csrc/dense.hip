// dense.hip - the fp32 (non-expert) half of the Qwen3-MoE forward on gfx950:
// the projections, q/k norm, RoPE, causal attention with a KV cache,
// embedding, greedy choice and the vocabulary softmax of
// test_model_trace.c:213-430 and :526-579, bit-identical to the reference.
//
// Every fp32 sum the reference forms is a sequential chain (k ascending,
// each product and sum rounded on its own; the library is compiled with
// -ffp-contract=off).  The kernels keep each chain in one lane and make the
// lanes plentiful: a lane per output row (and token) for the products, a
// lane per score for attention, a lane per head dimension for the weighted V
// sum.  Operands are staged through LDS with coalesced 16-byte loads issued
// a chunk ahead, so that the chain, not the memory, sets the pace (a
// dependent v_add_f32 every ~8 clocks).  Order-free steps (max, expf, the
// products of the softmax) run across lanes.
#include <climits>
#include <cstdlib>
#include <math.h>

#include <mutex>
#include <unordered_map>

#include "dense.h"
#include "moe_device.h"
#include "moe_layer.h"
#include "moe_qtile.h"

namespace moe {
namespace {

__device__ __forceinline__ float4 zero4() { return make_float4(0.0f, 0.0f, 0.0f, 0.0f); }

// acc = (((acc + x0 w0) + x1 w1) + ...) over 4*n4 columns of two LDS rows;
// 16 float4 of each row are read before their 64 dependent adds.
__device__ __forceinline__ float chain_dot(float acc, const float* x, const float* w, int n4) {
  const float4* x4 = reinterpret_cast<const float4*>(x);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  int k4 = 0;
  for (; k4 + 16 <= n4; k4 += 16) {
    float4 xv[16], wv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) { xv[i] = x4[k4 + i]; wv[i] = w4[k4 + i]; }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p0 = xv[i].x * wv[i].x, p1 = xv[i].y * wv[i].y;
      const float p2 = xv[i].z * wv[i].z, p3 = xv[i].w * wv[i].w;
      acc = acc + p0;
      acc = acc + p1;
      acc = acc + p2;
      acc = acc + p3;
    }
  }
  for (; k4 < n4; ++k4) {
    const float4 xv = x4[k4], wv = w4[k4];
    const float p0 = xv.x * wv.x, p1 = xv.y * wv.y, p2 = xv.z * wv.z, p3 = xv.w * wv.w;
    acc = acc + p0;
    acc = acc + p1;
    acc = acc + p2;
    acc = acc + p3;
  }
  return acc;
}

// max(a, b), NaN when either is NaN
__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : (a > b ? a : b);
}

__device__ __forceinline__ float dense_epilogue(const DenseArgs& a, int m, int n, float acc) {
  float c = acc;
  if (a.bias) c = c + a.bias[n];
  if (a.resid) c = a.resid[(size_t)m * a.ldr + n] + c;
  return c;
}

// ---------------------------------------------------------------- products

// Few tokens (M <= MM = 64 / RW): a block owns RW output rows; wave 0 is the
// consumer, waves 1..NP are producers.  The weight rows and the M token rows
// stream in chunks of KC columns with coalesced 16-byte loads; producer p
// owns chunks p, p + NP, ... and keeps its next chunk in registers, so each
// load has NP chunk-times to arrive (HBM latency, not bandwidth, limits a
// GEMV with this few bytes in flight).  A producer writes its chunk's
// products x[m][k] * w[r][k] into one of NP + 1 LDS buffers; the consumer
// lane m * RW + r sums token m's products with row n0 + r in column order.
// Splitting the roles keeps multiplies and loads out of the chain's wave: a
// pure add chain issues an add every 8 clocks, a chain that also multiplies
// every 12-13 (measured on gfx950).  Columns past K are zero in both
// operands: 0 * 0 = +0 and adding +0 leaves a chain unchanged (a chain that
// starts at +0 and adds round-to-nearest sums is never -0).  Rows past N read
// row N - 1 and are not stored.  K % 4 == 0, 16-byte aligned rows.  Dynamic
// LDS: NP + 1 buffers of M*RW rows of KC + 4 floats, then (NORM) the rows.
//
// NORM: the token rows are staged whole in LDS and rmsnorm'ed first
// (test_model_trace.c:241-255): squares x*x by all threads, their
// sequential sum by the whole block (block_seq_sum), msq / K,
// 1 / sqrtf(msq + eps), then x = (x * inv) * w; the producers' first weight
// chunks load meanwhile.
// Each block also writes a column slice of the normalized rows and
// (PACK = 2 / 3) packs the slice into the activation tables; the last block
// (fused selection) writes the tables' headers.
template <int RW, bool NORM, int PACK, int NP, int MMX = 64 / RW>
__global__ __launch_bounds__(64 * (NP + 1)) void dense_gemv_kernel(DenseArgs a) {
  constexpr int KC = RW >= 16 ? 4096 / RW : 256;
  constexpr int MM = MMX;                    // token rows one block can chain (<= 64 / RW)
  static_assert(MM * RW <= 64, "one consumer lane per chain");
  constexpr int V4 = KC / 4;                 // float4 per row chunk (<= 64)
  constexpr int LD = KC + 4;                 // padded LDS row (floats)
  constexpr int RPL = 64 / V4;               // rows one load instruction covers
  constexpr int NW = RW / RPL;               // W float4 per producer lane per chunk
  constexpr int NB = NP + 1;                 // LDS product buffers
  constexpr int NT = 64 * (NP + 1);
  extern __shared__ float4 pl4[];
  float* pl = reinterpret_cast<float*>(pl4);
  __shared__ float inv_s[MM];
  __shared__ int pack_scratch[2];
  __shared__ SeqSumScratch seq;
  __shared__ int ring_full[NP + 1], ring_done;
  if (threadIdx.x <= NP) ring_full[threadIdx.x] = 0;
  if (threadIdx.x == 0) ring_done = 0;
  const int M = a.M, N = a.N, K = a.K;
  const int nc = (K + KC - 1) / KC;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int prod = wave - 1;                 // producer index, -1 for the consumer
  const int n0 = blockIdx.x * RW;
  const int bufsz = M * RW * LD;
  float* xs = pl + NB * bufsz;               // NORM: [M][K] token rows
  const int c4 = lane % V4, r0 = lane / V4;
  float4 rw[NW], rx[MM];
  const float* wsrc[NW];
#pragma unroll
  for (int v = 0; v < NW; ++v)
    wsrc[v] = a.W + (size_t)min(n0 + r0 + v * RPL, N - 1) * a.ldw + 4 * c4;
  auto loadW = [&](int c) {
    const bool in = c * KC + 4 * c4 < K;
#pragma unroll
    for (int v = 0; v < NW; ++v)
      rw[v] = in ? *reinterpret_cast<const float4*>(wsrc[v] + (size_t)c * KC) : zero4();
  };
  auto loadX = [&](int c) {
    const int k = c * KC + 4 * c4;
    const bool in = k < K;
#pragma unroll
    for (int m = 0; m < MM; ++m)
      if (m < M) {
        if constexpr (NORM)
          rx[m] = in ? *reinterpret_cast<const float4*>(xs + (size_t)m * K + k) : zero4();
        else
          rx[m] = in ? *reinterpret_cast<const float4*>(a.A + (size_t)m * a.lda + k) : zero4();
      }
  };
  auto produce = [&](int c) {
    float* P = pl + (c % NB) * bufsz;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      if (m >= M) break;
#pragma unroll
      for (int v = 0; v < NW; ++v) {
        const float4 w = rw[v], x = rx[m];
        *reinterpret_cast<float4*>(P + (m * RW + r0 + v * RPL) * LD + 4 * c4) =
            make_float4(x.x * w.x, x.y * w.y, x.z * w.z, x.w * w.w);
      }
    }
  };
  if constexpr (NORM) {
    const int k4 = K / 4;
    // The token rows first, alone: issued with the weight chunks of every
    // block they would return behind that burst.  Producer 0 requests chunk
    // 0 once the rows are in (after the staging barrier), so that it arrives
    // while the squares are summed; the other producers' first chunks, needed
    // a chunk-time later, wait until the norm is done.
    constexpr int XR = 2, NWR = 2;
    const bool x_regs = M * k4 <= XR * NT;
    const bool nw_regs = k4 <= NWR * NT;
    float4 xr[XR], nwr[NWR];
#pragma unroll
    for (int u = 0; u < XR; ++u) {
      const int i = (int)threadIdx.x + u * NT;
      xr[u] = (x_regs && i < M * k4)
                  ? *reinterpret_cast<const float4*>(a.A + (size_t)(i / k4) * a.lda + 4 * (i % k4))
                  : zero4();
    }
#pragma unroll
    for (int u = 0; u < NWR; ++u) {
      const int j = (int)threadIdx.x + u * NT;
      nwr[u] = (nw_regs && a.norm_w && j < k4) ? reinterpret_cast<const float4*>(a.norm_w)[j]
                                              : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
    if (x_regs) {
#pragma unroll
      for (int u = 0; u < XR; ++u) {
        const int i = (int)threadIdx.x + u * NT;
        if (i < M * k4) {
          const float4 v = xr[u];
          reinterpret_cast<float4*>(xs)[i] = v;
          reinterpret_cast<float4*>(pl)[i] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
        }
      }
    } else {
      for (int i = threadIdx.x; i < M * k4; i += NT) {
        const int m = i / k4, j = i % k4;
        const float4 v = *reinterpret_cast<const float4*>(a.A + (size_t)m * a.lda + 4 * j);
        reinterpret_cast<float4*>(xs)[i] = v;
        reinterpret_cast<float4*>(pl)[i] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
      }
    }
    __syncthreads();
    if (prod == 0 && nc > 0) loadW(0);
    for (int m = 0; m < M; ++m) {
      const float msq = block_seq_sum<NT>(pl + (size_t)m * K, K, seq);
      if (threadIdx.x == 0) inv_s[m] = 1.0f / sqrtf(msq / (float)K + a.eps);
    }
    __syncthreads();
    if (prod > 0 && prod < nc) loadW(prod);
    if (nw_regs) {
      // (a missing weight is 1: the reference multiplies by 1.0f)
#pragma unroll
      for (int u = 0; u < NWR; ++u) {
        const int j = (int)threadIdx.x + u * NT;
        if (j < k4)
          for (int m = 0; m < M; ++m) {
            float4* xp = reinterpret_cast<float4*>(xs + (size_t)m * K) + j;
            const float4 x = *xp, w = nwr[u];
            const float iv = inv_s[m];
            const float v0 = x.x * iv, v1 = x.y * iv, v2 = x.z * iv, v3 = x.w * iv;
            *xp = make_float4(v0 * w.x, v1 * w.y, v2 * w.z, v3 * w.w);
          }
      }
    } else {
      for (int i = threadIdx.x; i < M * K; i += NT) {
        const float v = xs[i] * inv_s[i / K];
        xs[i] = a.norm_w ? v * a.norm_w[i % K] : v * 1.0f;
      }
    }
    __syncthreads();
    // this block's column slice [c0, c1) (a multiple of 8 columns)
    const int sl = ((K + 7) / 8 + (int)gridDim.x - 1) / (int)gridDim.x * 8;
    const int c0 = min(K, (int)blockIdx.x * sl), c1 = min(K, c0 + sl);
    if (a.xn_out)
      for (int m = 0; m < M; ++m)
        for (int i = c0 + threadIdx.x; i < c1; i += NT) a.xn_out[(size_t)m * K + i] = xs[(size_t)m * K + i];
    if constexpr (PACK != 0) {
      const size_t tb = act_table_bytes(K);
      for (int m = 0; m < M; ++m) {
        if (threadIdx.x == 0) { pack_scratch[0] = 1; pack_scratch[1] = 0; }
        __syncthreads();
        int nl;
        uint32_t sum;
        pack_act_cols<PACK == 3>(xs + (size_t)m * K, K, c0, c1, a.pack_tabs + m * tb, threadIdx.x, NT,
                                 nl, sum);
        // wave reductions, then one LDS atomic per wave
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
          const int on = __shfl_xor(nl, off, kWave);
          nl = on > nl ? on : nl;
          sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
        }
        if (lane == 0) {
          atomicMax(&pack_scratch[0], nl);
          atomicAdd(reinterpret_cast<unsigned*>(&pack_scratch[1]), sum);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
          uint32_t* pp = a.pack_part + ((size_t)m * gridDim.x + blockIdx.x) * 2;
          pp[0] = (uint32_t)pack_scratch[0];
          pp[1] = (uint32_t)pack_scratch[1];
        }
      }
    }
  }
  if constexpr (!NORM) {
    if (prod >= 0 && prod < nc) loadW(prod);
    if constexpr (PACK != 0) {
      // up to 16 given rows: this block's column slice [c0, c1) of each
      // token row into its activation table, V columns a thread, while the
      // first chunks load; the slice's partial header {limbs, sum} goes to
      // pack_part[block][token] (select_kernel writes the headers)
      static_assert(MM <= 16, "partial headers of up to 16 tokens a block");
      constexpr int V = PACK == 3 ? 8 : 4;
      __shared__ unsigned pk[16][2];
      if (threadIdx.x < 16) { pk[threadIdx.x][0] = 1u; pk[threadIdx.x][1] = 0u; }
      __syncthreads();
      const int sl = ((K + 7) / 8 + (int)gridDim.x - 1) / (int)gridDim.x * 8;
      const int c0 = min(K, (int)blockIdx.x * sl), c1 = min(K, c0 + sl);
      const int G = (c1 - c0 + V - 1) / V;
      const size_t tb = act_table_bytes(K);
      for (int i = threadIdx.x; i < M * G; i += NT) {
        const int m = i / G, g0 = c0 + (i % G) * V;
        int nl;
        uint32_t sum;
        pack_act_cols<PACK == 3>(a.A + (size_t)m * a.lda, K, g0, min(c1, g0 + V), a.pack_tabs + m * tb, 0, 1,
                                 nl, sum);
        atomicMax(&pk[m][0], (unsigned)nl);
        atomicAdd(&pk[m][1], sum);
      }
      __syncthreads();
      if (threadIdx.x < M)
        reinterpret_cast<uint2*>(a.pack_part)[(size_t)blockIdx.x * 16 + threadIdx.x] =
            make_uint2(pk[threadIdx.x][0], pk[threadIdx.x][1]);
    }
  }
  // The ring's hand-over: a producer stores k + 1 into ring_full[k % NB]
  // after writing chunk k, the consumer the number of chunks it has summed
  // into ring_done; a producer waits for ring_done >= k - NB + 1 before
  // reusing a buffer, the consumer for ring_full[c % NB] >= c + 1.  Neither
  // side waits on itself, so every wait ends.
  __syncthreads();   // the ring counters are zero
  if (prod >= 0) {
    if (prod < nc) loadX(prod);
    for (int k = prod; k < nc; k += NP) {
      if (k >= NB) ring_wait(&ring_done, k - NB + 1, true);
      produce(k);
      ring_post(&ring_full[k % NB], k + 1);
      if (k + NP < nc) {
        loadW(k + NP);
        loadX(k + NP);
      }
    }
  } else {
    const int m = lane / RW, r = lane % RW;
    const bool live = m < M;
    float acc = 0.0f;
    for (int c = 0; c < nc; ++c) {
      ring_wait(&ring_full[c % NB], c + 1, false);
      if (live) acc = chain_sum(acc, pl + (c % NB) * bufsz + lane * LD, V4);
      ring_post(&ring_done, c + 1);
    }
    const int n = n0 + r;
    float c = -__builtin_inff();
    if (live && n < N) {
      c = dense_epilogue(a, m, n, acc);
      a.C[(size_t)m * a.ldc + n] = c;
    }
    if (a.amax_part) {   // M == 1: the block's largest output, NaN if any is NaN
      float v = c;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v = nan_max(v, __shfl_xor(v, off, kWave));
      if (lane == 0) a.amax_part[blockIdx.x] = v;
    }
  }
  if constexpr (RW == 16) {
    if (a.sel_counter) {
      // the last block to finish selects the experts of every token (and
      // writes the activation tables' headers from the slices' partials)
      __shared__ int last;
      __shared__ int sidx[NP + 1][kMaxTopK];
      __shared__ float sval[NP + 1][kMaxTopK], sexp[NP + 1][kMaxTopK];
      __threadfence();
      __syncthreads();
      if (threadIdx.x == 0) {
        const unsigned prev = atomicAdd(a.sel_counter, 1u);
        last = prev == gridDim.x - 1;
        if (last) *a.sel_counter = 0u;
      }
      __syncthreads();
      if (last) {
        __threadfence();
        if constexpr (PACK != 0) {
          if (threadIdx.x < M) {
            const int m = threadIdx.x;
            uint32_t nl = 1, sum = 0;
            for (unsigned b = 0; b < gridDim.x; ++b) {
              const uint32_t* pp = a.pack_part + ((size_t)m * gridDim.x + b) * 2;
              nl = pp[0] > nl ? pp[0] : nl;
              sum += pp[1];
            }
            uint32_t* hh = reinterpret_cast<uint32_t*>(a.pack_tabs + m * act_table_bytes(K));
            hh[0] = nl;
            hh[1] = sum;
          }
        }
        // one wave per token; keys in the product buffers (free now)
        uint64_t* keys = reinterpret_cast<uint64_t*>(pl) + (size_t)wave * 1024;
        for (int m = wave; m < M; m += NP + 1) {
          const size_t o = (size_t)m * a.sel_topk;
          select_token_any(a.C + (size_t)m * a.ldc, N, a.sel_topk, keys, sidx[wave], sval[wave],
                           sexp[wave], a.sel_idx + o, a.sel_p + o,
                           a.sel_idx_user ? a.sel_idx_user + o : nullptr,
                           a.sel_p_user ? a.sel_p_user + o : nullptr);
        }
      }
    }
  }
}

// Few tokens, few rows (the router): one block per (output row, token); with
// NORM one token.  The token row is staged in LDS (normalized first
// when NORM, the sum of squares by block_seq_sum), the products x[k] *
// W[n][k] are formed into LDS and summed in order by block_seq_sum, so a row
// costs about K / 8 dependent adds instead of K.  With PACK each block packs its column slice of its
// token's (normalized) row into that token's activation table (row_finish_kernel writes the
// header and, with a fused selection, picks the experts).
// 512 threads: two waves per SIMD.  A wave issues a VALU instruction about
// every 8 clocks whether or not it depends on the previous one, so the
// candidate chains of block_seq_sum fill a SIMD only with two waves on it.
constexpr int kRowThreads = 512;
constexpr int kRowMaxK = 8192;

template <bool NORM, int PACK>
__global__ __launch_bounds__(kRowThreads) void dense_row_kernel(DenseArgs a) {
  extern __shared__ float4 rl4[];
  const int K = a.K, k4 = K / 4, n = blockIdx.x, m = blockIdx.y;
  float* xs = reinterpret_cast<float*>(rl4);   // [K] the token row
  float* pv = xs + K;                          // [K] squares, then products, then keys
  float4* xs4 = rl4;
  float4* pv4 = rl4 + k4;
  __shared__ SeqSumScratch seq;
  __shared__ int pack_scratch[2];
  __shared__ float inv_s;
  const int tid = threadIdx.x, lane = tid % kWave;
  if (a.epoch_bump && n == 0 && m == 0 && tid == 0) {
    const uint32_t e = *a.epoch_bump + 1u;
    *a.epoch_bump = e ? e : 1u;
  }
  constexpr int WV = kRowMaxK / 4 / kRowThreads;
  // the token row (and norm weights) into registers first, then the weight
  // row (a wave's loads complete in order: the LDS staging waits only for
  // the token row)
  const float4* x4 = reinterpret_cast<const float4*>(a.A + (size_t)m * a.lda);
  const float4* nw4g = reinterpret_cast<const float4*>(a.norm_w);
  float4 xv[WV], nv[WV];
#pragma unroll
  for (int u = 0; u < WV; ++u) {
    const int i = tid + kRowThreads * u;
    xv[u] = i < k4 ? x4[i] : zero4();
    nv[u] = (NORM && a.norm_w && i < k4) ? nw4g[i] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
  }
  const float4* wr = reinterpret_cast<const float4*>(a.W + (size_t)n * a.ldw);
  float4 w[WV];
#pragma unroll
  for (int u = 0; u < WV; ++u) {
    const int i = tid + kRowThreads * u;
    w[u] = i < k4 ? wr[i] : zero4();
  }
#pragma unroll
  for (int u = 0; u < WV; ++u) {
    const int i = tid + kRowThreads * u;
    if (i < k4) {
      const float4 v = xv[u];
      xs4[i] = v;
      if (NORM) pv4[i] = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
    }
  }
  __syncthreads();
  if constexpr (NORM) {
    const float msq = block_seq_sum<kRowThreads>(pv, K, seq);
    if (tid == 0) inv_s = 1.0f / sqrtf(msq / (float)K + a.eps);
    __syncthreads();
    // (a missing weight is 1: the reference multiplies by 1.0f)
    const float iv = inv_s;
#pragma unroll
    for (int u = 0; u < WV; ++u) {
      const int i = tid + kRowThreads * u;
      if (i < k4) {
        const float4 x = xv[u], g = nv[u];
        const float v0 = x.x * iv, v1 = x.y * iv, v2 = x.z * iv, v3 = x.w * iv;
        xs4[i] = make_float4(v0 * g.x, v1 * g.y, v2 * g.z, v3 * g.w);
      }
    }
    __syncthreads();
  }
  // this block's column slice [c0, c1) (a multiple of 8 columns) of the
  // (normalized) row: to xn_out, and packed into the x tables' planes
  const int sl = ((K + 7) / 8 + (int)gridDim.x - 1) / (int)gridDim.x * 8;
  const int c0 = min(K, (int)blockIdx.x * sl), c1 = min(K, c0 + sl);
  if (NORM && a.xn_out)
    for (int i = c0 + tid; i < c1; i += kRowThreads) a.xn_out[i] = xs[i];
  if constexpr (PACK != 0) {
    if (tid == 0) { pack_scratch[0] = 1; pack_scratch[1] = 0; }
    __syncthreads();
    int nl;
    uint32_t sum;
    pack_act_cols<PACK == 3>(xs, K, c0, c1, a.pack_tabs + (size_t)m * act_table_bytes(K), tid, kRowThreads,
                             nl, sum);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int on = __shfl_xor(nl, off, kWave);
      nl = on > nl ? on : nl;
      sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
    }
    if (lane == 0) {
      atomicMax(&pack_scratch[0], nl);
      atomicAdd(reinterpret_cast<unsigned*>(&pack_scratch[1]), sum);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t* pp = a.pack_part + ((size_t)m * gridDim.x + blockIdx.x) * 2;
      pp[0] = (uint32_t)pack_scratch[0];
      pp[1] = (uint32_t)pack_scratch[1];
    }
  }
  // products x[k] * W[n][k], then their sum in column order
#pragma unroll
  for (int u = 0; u < WV; ++u) {
    const int i = tid + kRowThreads * u;
    if (i < k4) {
      const float4 x = xs4[i];
      pv4[i] = make_float4(x.x * w[u].x, x.y * w[u].y, x.z * w[u].z, x.w * w[u].w);
    }
  }
  __syncthreads();
  const float acc = block_seq_sum<kRowThreads>(pv, K, seq);
  if (tid == 0) a.C[(size_t)m * a.ldc + n] = dense_epilogue(a, m, n, acc);
}

// 5-16 tokens, few rows: a block per (output row, four tokens), its 512
// threads four groups of 128 side by side, each the row kernel on its own
// token -- products x[k] * W[n][k] into its LDS slice, summed in order by
// group_seq_sum (four candidate chains per thread).  No norm.  With PACK
// each group also packs the block's column slice of its token's row into
// the token's activation table and leaves the slice's partial header at
// pack_part[slice][token] (uint2 {limbs, sum}; select_kernel combines them).
constexpr int kRowGroups = 4;
constexpr int kRowGroupThreads = kRowThreads / kRowGroups;
constexpr int kRowsMaxK = 4096;

template <int PACK>
__global__ __launch_bounds__(kRowThreads) void dense_rows4_kernel(DenseArgs a) {
  extern __shared__ float4 rg4[];   // [kRowGroups][K] products
  __shared__ SeqSumScratch seq[kRowGroups];
  __shared__ int pk[kRowGroups][2];
  const int K = a.K, k4 = K / 4, n = blockIdx.x;
  const int g = threadIdx.x / kRowGroupThreads, gt = threadIdx.x % kRowGroupThreads;
  const int mg = blockIdx.y * kRowGroups + g;   // this group's token (past M: a repeat, not written)
  const int m = min(mg, a.M - 1);
  float4* pv4 = rg4 + (size_t)g * k4;
  const float4* x4 = reinterpret_cast<const float4*>(a.A + (size_t)m * a.lda);
  const float4* w4 = reinterpret_cast<const float4*>(a.W + (size_t)n * a.ldw);
  constexpr int WV = kRowsMaxK / 4 / kRowGroupThreads;
  float4 xv[WV], wv[WV];
#pragma unroll
  for (int u = 0; u < WV; ++u) {
    const int i = gt + kRowGroupThreads * u;
    xv[u] = i < k4 ? x4[i] : zero4();
  }
#pragma unroll
  for (int u = 0; u < WV; ++u) {
    const int i = gt + kRowGroupThreads * u;
    wv[u] = i < k4 ? w4[i] : zero4();
  }
  if constexpr (PACK != 0) {
    // the block's column slice [c0, c1) (a multiple of 8 columns)
    const int sl = ((K + 7) / 8 + (int)gridDim.x - 1) / (int)gridDim.x * 8;
    const int c0 = min(K, (int)blockIdx.x * sl), c1 = min(K, c0 + sl);
    if (gt == 0) { pk[g][0] = 1; pk[g][1] = 0; }
    int nl = 1;
    uint32_t sum = 0;
    if (mg < a.M)
      pack_act_cols<PACK == 3>(a.A + (size_t)m * a.lda, K, c0, c1, a.pack_tabs + (size_t)m * act_table_bytes(K),
                               gt, kRowGroupThreads, nl, sum);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const int on = __shfl_xor(nl, off, kWave);
      nl = on > nl ? on : nl;
      sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
    }
    __syncthreads();
    if (threadIdx.x % kWave == 0) {
      atomicMax(&pk[g][0], nl);
      atomicAdd(reinterpret_cast<unsigned*>(&pk[g][1]), sum);
    }
  }
#pragma unroll
  for (int u = 0; u < WV; ++u) {
    const int i = gt + kRowGroupThreads * u;
    if (i < k4)
      pv4[i] = make_float4(xv[u].x * wv[u].x, xv[u].y * wv[u].y, xv[u].z * wv[u].z, xv[u].w * wv[u].w);
  }
  __syncthreads();
  if constexpr (PACK != 0) {
    if (gt == 0 && mg < a.M)
      reinterpret_cast<uint2*>(a.pack_part)[(size_t)n * 16 + mg] = make_uint2((unsigned)pk[g][0], (unsigned)pk[g][1]);
  }
  const float acc = group_seq_sum<kRowGroupThreads>(reinterpret_cast<const float*>(pv4), K, seq[g], gt);
  if (gt == 0 && mg < a.M) a.C[(size_t)m * a.ldc + n] = dense_epilogue(a, m, n, acc);
}

// After dense_row_kernel (a kernel boundary instead of a fence in each of
// its blocks): each token's activation-table header from its slices'
// partials and its expert selection, one wave per token (M <= 4).
constexpr int kRowFinishWaves = 4;
__global__ __launch_bounds__(kRowFinishWaves * kWave) void row_finish_kernel(DenseArgs a) {
  __shared__ uint64_t keys[kRowFinishWaves][1024];
  __shared__ int sidx[kRowFinishWaves][kMaxTopK];
  __shared__ float sval[kRowFinishWaves][kMaxTopK], sexp[kRowFinishWaves][kMaxTopK];
  const int lane = threadIdx.x % kWave, m = threadIdx.x / kWave;
  if (a.pack_dtype && m < a.M) {
    uint32_t nl = 1, sum = 0;
    for (int b = lane; b < a.N; b += kWave) {
      const uint32_t* pp = a.pack_part + ((size_t)m * a.N + b) * 2;
      nl = pp[0] > nl ? pp[0] : nl;
      sum += pp[1];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint32_t on = (uint32_t)__shfl_xor((int)nl, off, kWave);
      nl = on > nl ? on : nl;
      sum += (uint32_t)__shfl_xor((int)sum, off, kWave);
    }
    if (lane == 0) {
      uint32_t* hh = reinterpret_cast<uint32_t*>(a.pack_tabs + (size_t)m * act_table_bytes(a.K));
      hh[0] = nl;
      hh[1] = sum;
    }
  }
  if (m >= a.M) return;
  const size_t o = (size_t)m * a.sel_topk;
  select_token_any(a.C + (size_t)m * a.ldc, a.N, a.sel_topk, keys[m], sidx[m], sval[m], sexp[m],
                   a.sel_idx + o, a.sel_p + o, a.sel_idx_user ? a.sel_idx_user + o : nullptr,
                   a.sel_p_user ? a.sel_p_user + o : nullptr);
}

// Many tokens: a block computes a tile of 16*CT tokens x 16*CE rows; thread
// (ti, ei) owns tokens t0 + ti + 16i and rows n0 + ei + 16j, CT*CE chains.
// Token and weight rows stream through two LDS chunk buffers of KC columns.
// Same zero padding and clamping as above.
template <int CT, int CE, int KC>
__global__ __launch_bounds__(256) void dense_tile_kernel(DenseArgs a) {
  constexpr int RX = 16 * CT, RW = 16 * CE, R = RX + RW;
  constexpr int LD = KC + 4;
  constexpr int V4 = KC / 4;
  constexpr int NV = R * V4 / 256;
  static_assert(R * V4 % 256 == 0, "chunk must split evenly over the block");
  extern __shared__ float4 lds4[];
  float* buf = reinterpret_cast<float*>(lds4);   // [2][R][LD]
  const int tid = threadIdx.x;
  const int ti = tid / 16, ei = tid % 16;
  const int t0 = blockIdx.y * RX, n0 = blockIdx.x * RW;
  const int nc = (a.K + KC - 1) / KC;
  const float* src[NV];
  int dst[NV], col[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = tid + 256 * v;
    const int row = i / V4, c4 = i % V4;
    src[v] = row < RX ? a.A + (size_t)min(t0 + row, a.M - 1) * a.lda + 4 * c4
                      : a.W + (size_t)min(n0 + row - RX, a.N - 1) * a.ldw + 4 * c4;
    dst[v] = row * LD + 4 * c4;
    col[v] = 4 * c4;
  }
  float4 rg[NV];
  auto load = [&](int c) {
#pragma unroll
    for (int v = 0; v < NV; ++v)
      rg[v] = c * KC + col[v] < a.K ? *reinterpret_cast<const float4*>(src[v] + (size_t)c * KC)
                                    : zero4();
  };
  auto store = [&](int b) {
#pragma unroll
    for (int v = 0; v < NV; ++v) *reinterpret_cast<float4*>(buf + b * R * LD + dst[v]) = rg[v];
  };
  float acc[CT][CE];
#pragma unroll
  for (int i = 0; i < CT; ++i)
#pragma unroll
    for (int j = 0; j < CE; ++j) acc[i][j] = 0.0f;
  load(0);
  store(0);
  if (nc > 1) load(1);
  for (int c = 0; c < nc; ++c) {
    __syncthreads();
    if (c + 1 < nc) {
      store((c + 1) & 1);
      if (c + 2 < nc) load(c + 2);
    }
    const float* B = buf + (c & 1) * R * LD;
#pragma unroll 2
    for (int k = 0; k < KC; k += 4) {
      float4 xv[CT], wv[CE];
#pragma unroll
      for (int i = 0; i < CT; ++i) xv[i] = *reinterpret_cast<const float4*>(B + (ti + 16 * i) * LD + k);
#pragma unroll
      for (int j = 0; j < CE; ++j) wv[j] = *reinterpret_cast<const float4*>(B + (RX + ei + 16 * j) * LD + k);
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
  }
#pragma unroll
  for (int i = 0; i < CT; ++i)
#pragma unroll
    for (int j = 0; j < CE; ++j) {
      const int t = t0 + ti + 16 * i, n = n0 + ei + 16 * j;
      if (t < a.M && n < a.N) a.C[(size_t)t * a.ldc + n] = dense_epilogue(a, t, n, acc[i][j]);
    }
}

// Any shape or alignment: one thread per output, plain loads.
__global__ __launch_bounds__(256) void dense_generic_kernel(DenseArgs a) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)a.M * a.N) return;
  const int m = (int)(i / a.N), n = (int)(i % a.N);
  const float* x = a.A + (size_t)m * a.lda;
  const float* w = a.W + (size_t)n * a.ldw;
  float acc = 0.0f;
  for (int k = 0; k < a.K; ++k) {
    const float p = x[k] * w[k];
    acc = acc + p;
  }
  a.C[(size_t)m * a.ldc + n] = dense_epilogue(a, m, n, acc);
}

// ---------------------------------------------------------------- heads

constexpr int kMaxHd = 512;

// Up to two head rows (v0 and, if v1, v1; LDS, hd values each) through the
// per-head RMSNorm of test_model_trace.c:381-402 (when the weight is given:
// squares by all lanes, the sequential sum in lane 0 (row 0) and lane 1
// (row 1) side by side, inv = 1/sqrtf(msq/hd + eps), v = (v*inv)*w) and
// RoPE (:326-336: the pair (i, i + hd/2) turned by cos/sin of the row's
// position, each product rounded, then one subtraction / addition) into
// out0 / out1 (global or LDS).  Everything the rows need (weights, cos/sin)
// is read from LDS or registers, so no global load sits between the steps.
// Called by all 64 threads of a one-wave block; sq: LDS scratch [2][hd].
__device__ void heads_prep(float* v0, float* v1, const float* w0, const float* w1, float eps,
                           int hd, const float* cs, const float* sn, float* sq, float* inv_s,
                           float* out0, float* out1) {
  const int lane = threadIdx.x, d2 = hd / 2;
  const bool n0 = w0 != nullptr, n1 = v1 && w1;
  if (n0 || n1) {
    for (int d = lane; d < hd; d += 64) {
      if (n0) sq[d] = v0[d] * v0[d];
      if (n1) sq[hd + d] = v1[d] * v1[d];
    }
    __syncthreads();
    if ((lane == 0 && n0) || (lane == 1 && n1)) {
      const float msq = chain_sum(0.0f, sq + lane * hd, hd / 4);
      const float mean = msq / (float)hd;
      inv_s[lane] = 1.0f / sqrtf(mean + eps);
    }
    __syncthreads();
    for (int d = lane; d < hd; d += 64) {
      if (n0) {
        const float s = v0[d] * inv_s[0];
        v0[d] = s * w0[d];
      }
      if (n1) {
        const float s = v1[d] * inv_s[1];
        v1[d] = s * w1[d];
      }
    }
    __syncthreads();
  }
  for (int i = lane; i < d2; i += 64) {
    const float c = cs[i], s = sn[i];
    {
      const float e = v0[i], o = v0[i + d2];
      const float ec = e * c, os = o * s, oc = o * c, es = e * s;
      out0[i] = ec - os;
      out0[i + d2] = oc + es;
    }
    if (v1) {
      const float e = v1[i], o = v1[i + d2];
      const float ec = e * c, os = o * s, oc = o * c, es = e * s;
      out1[i] = ec - os;
      out1[i + d2] = oc + es;
    }
  }
}

// Block (t, h) over the heads of row t of [Q | K | V] (each head hd wide, so
// head h starts at h * hd): q/k heads through heads_prep at position
// pos0 + t (Q stays in place, K goes to the cache), V rows to the cache.
__global__ __launch_bounds__(64) void heads_kernel(HeadArgs a) {
  __shared__ float4 v4[kMaxHd / 4];
  __shared__ float4 sq4[2 * kMaxHd / 4];
  __shared__ float4 w4[kMaxHd / 4];
  __shared__ float4 cs4[kMaxHd / 8], sn4[kMaxHd / 8];
  __shared__ float inv_s[2];
  const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int hd = a.hd, d2 = hd / 2, pos = a.pos0 + t;
  float* row = a.qkv + (size_t)t * a.ld + (size_t)h * hd;
  if (h >= a.nq + a.nkv) {   // V head: into the cache unchanged
    float* dst = a.vc + ((size_t)(h - a.nq - a.nkv) * a.max_seq + pos) * hd;
    for (int d = lane; d < hd; d += 64) dst[d] = row[d];
    return;
  }
  const bool isq = h < a.nq;
  const float* wg = isq ? a.q_norm : a.k_norm;
  float* v = reinterpret_cast<float*>(v4);
  float* w = reinterpret_cast<float*>(w4);
  float* cs = reinterpret_cast<float*>(cs4);
  float* sn = reinterpret_cast<float*>(sn4);
  for (int d = lane; d < hd; d += 64) {
    v[d] = row[d];
    if (wg) w[d] = wg[d];
  }
  for (int i = lane; i < d2; i += 64) {
    cs[i] = a.rope_cos[(size_t)pos * d2 + i];
    sn[i] = a.rope_sin[(size_t)pos * d2 + i];
  }
  __syncthreads();
  float* out = isq ? row : a.kc + ((size_t)(h - a.nq) * a.max_seq + pos) * hd;
  heads_prep(v, nullptr, wg ? w : nullptr, nullptr, a.eps, hd, cs, sn, reinterpret_cast<float*>(sq4),
             inv_s, out, nullptr);
}

// ---------------------------------------------------------------- attention

// Scores of query row t, head h against cache positions tk0 .. tk0 + 63
// (<= pos0 + t): lane i runs the chain dot = (((0 + q0 k0) + q1 k1) + ...)
// over hd for position tk0 + i and stores dot * scale.  REG (hd <= 128):
// each lane loads its K row straight into registers (one round trip);
// otherwise the 64 K rows are staged in LDS.  fuse_heads (T == 1, position
// P = pos0): q is normed and rotated here; the block holding position P
// computes K's row P the same way (the cache does not have it yet) and, for
// the first query head of each KV group, writes K and V row P into the
// caches.  All global loads are issued first.
constexpr int kRegHd = 128;

// (x, y) work indices of this block in a 2-D grid, permuted so that blocks
// with consecutive y (heads of one KV group) share an XCD: blocks are dealt
// to the 8 XCDs in turn, so XCD k runs the blocks whose linear index is k
// mod 8, and those get logical indices k n/8 .. k n/8 + n/8 - 1 (x fastest).
// The K and V rows a KV head's blocks read then come from one XCD's L2
// instead of every XCD's.  The identity when n is not a multiple of 8 or
// with MOEHIP_ATTN_NO_XCD set.
__device__ __forceinline__ void attn_xcd_map(bool on, int* bx, int* by) {
  const int gx = (int)gridDim.x, n = gx * (int)gridDim.y;
  const int L = (int)blockIdx.x + gx * (int)blockIdx.y;
  if (!on || n % 8) {
    *bx = (int)blockIdx.x;
    *by = (int)blockIdx.y;
    return;
  }
  const int Lg = (L % 8) * (n / 8) + L / 8;
  *bx = Lg % gx;
  *by = Lg / gx;
}

template <bool REG>
__global__ __launch_bounds__(64) void attn_scores_kernel(AttnArgs a) {
  extern __shared__ float lds[];
  const int hd = a.hd, LD = hd + 4, d2 = hd / 2;
  const int hdp = (hd + 3) & ~3;
  float* q = lds;                       // [hd] the query (rotated)
  float* kt = q + hdp;                  // REG: [hd] K row P; else [64][LD] K rows
  float* qraw = kt + (REG ? hdp : 64 * LD);   // [hd]
  float* kraw = qraw + hdp;             // [hd]
  float* wq = kraw + hdp;               // [hd]
  float* wk = wq + hdp;                 // [hd]
  float* cs = wk + hdp;                 // [hd/2]
  float* sn = cs + hdp;                 // [hd/2]
  float* sq = sn + hdp;                 // [2][hd]
  __shared__ float inv_s[2];
  int bx, h;
  attn_xcd_map(a.xcd_map, &bx, &h);
  const int t = blockIdx.z, lane = threadIdx.x;
  const int P = a.pos0 + t;
  const int tk0 = bx * 64;
  if (tk0 > P) return;
  const int group = a.nq / a.nkv;
  const int kvh = h / group;
  const float* qrow = a.qkv + (size_t)t * a.ld + (size_t)h * hd;
  const float* kbase = a.kc + ((size_t)kvh * a.max_seq + tk0) * hd;
  const int rows = min(64, P + 1 - tk0);
  const bool own_new = a.fuse_heads && P - tk0 < 64;   // this block holds row P
  const int cached = own_new ? rows - 1 : rows;        // rows read from the cache
  const int h4 = hd / 4;
  const int total = cached * h4;
  // fuse_heads: the head rows, norm weights and cos/sin into registers first
  // (a wave's loads complete in order: heads_prep below then waits for these
  // alone, not for the K rows requested after them)
  constexpr int SR = (REG ? kRegHd : kMaxHd) / 64, SC = SR / 2;
  float rq[SR], rwq[SR], rk[SR], rwk[SR], rv[SR], rcs[SC], rsn[SC];
  const bool write_v = own_new && h % group == 0;
  if (a.fuse_heads) {
    const float* krow = a.qkv + (size_t)t * a.ld + (size_t)(a.nq + kvh) * hd;
    const float* vraw = a.qkv + (size_t)t * a.ld + (size_t)(a.nq + a.nkv + kvh) * hd;
#pragma unroll
    for (int u = 0; u < SR; ++u) {
      const int d = lane + 64 * u;
      const bool in = d < hd;
      rq[u] = in ? qrow[d] : 0.0f;
      rwq[u] = in && a.q_norm ? a.q_norm[d] : 0.0f;
      rk[u] = in && own_new ? krow[d] : 0.0f;
      rwk[u] = in && own_new && a.k_norm ? a.k_norm[d] : 0.0f;
      rv[u] = in && write_v ? vraw[d] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < SC; ++u) {
      const int i = lane + 64 * u;
      rcs[u] = i < d2 ? a.rope_cos[(size_t)P * d2 + i] : 0.0f;
      rsn[u] = i < d2 ? a.rope_sin[(size_t)P * d2 + i] : 0.0f;
    }
  }
  float4 kr[REG ? kRegHd / 4 : 1];
  if constexpr (REG) {
    // this lane's K row (position tk0 + lane) into registers
    // (columns past hd: the row's last float4 again; their products are not summed)
    const float4* src = reinterpret_cast<const float4*>(kbase + (size_t)(lane < cached ? lane : 0) * hd);
#pragma unroll
    for (int i = 0; i < kRegHd / 4; ++i) kr[i] = src[i < h4 ? i : h4 - 1];
  } else {
    // 16 loads in flight per lane, then their stores
    for (int base = 0; base < total; base += 64 * 16) {
      float4 r[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int i = base + lane + 64 * u;
        r[u] = i < total ? *reinterpret_cast<const float4*>(kbase + (size_t)(i / h4) * hd + 4 * (i % h4))
                         : zero4();
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int i = base + lane + 64 * u;
        if (i < total) *reinterpret_cast<float4*>(kt + (i / h4) * LD + 4 * (i % h4)) = r[u];
      }
    }
  }
  if (a.fuse_heads) {
#pragma unroll
    for (int u = 0; u < SR; ++u) {
      const int d = lane + 64 * u;
      if (d < hd) {
        qraw[d] = rq[u];
        wq[d] = rwq[u];
        kraw[d] = rk[u];
        wk[d] = rwk[u];
      }
    }
#pragma unroll
    for (int u = 0; u < SC; ++u) {
      const int i = lane + 64 * u;
      if (i < d2) {
        cs[i] = rcs[u];
        sn[i] = rsn[u];
      }
    }
    if (write_v) {   // V row P into the cache unchanged
      float* vd = a.vc + ((size_t)kvh * a.max_seq + P) * hd;
#pragma unroll
      for (int u = 0; u < SR; ++u)
        if (lane + 64 * u < hd) vd[lane + 64 * u] = rv[u];
    }
    __syncthreads();
    float* knew = REG ? kt : kt + (P - tk0) * LD;
    heads_prep(qraw, own_new ? kraw : nullptr, a.q_norm ? wq : nullptr, a.k_norm ? wk : nullptr,
               a.eps, hd, cs, sn, sq, inv_s, q, knew);
    if (own_new && h % group == 0) {
      __syncthreads();
      float* kd = a.kc + ((size_t)kvh * a.max_seq + P) * hd;
      for (int d = lane; d < hd; d += 64) kd[d] = knew[d];
    }
  } else {
    for (int d = lane; d < hd; d += 64) q[d] = qrow[d];
  }
  __syncthreads();
  if (lane < rows) {
    float dot;
    if constexpr (REG) {
      if (own_new && lane == P - tk0) {   // row P: computed above, in LDS
        const float4* kn4 = reinterpret_cast<const float4*>(kt);
#pragma unroll
        for (int i = 0; i < kRegHd / 4; ++i) kr[i] = kn4[i < h4 ? i : h4 - 1];
      }
      const float4* q4 = reinterpret_cast<const float4*>(q);
      dot = 0.0f;
      // the query (an LDS broadcast) is read 8 float4 ahead of its adds
#pragma unroll
      for (int ib = 0; ib < kRegHd / 4; ib += 8) {
        float4 qv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) qv[u] = q4[ib + u < h4 ? ib + u : h4 - 1];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (ib + u < h4) {
            const float p0 = qv[u].x * kr[ib + u].x, p1 = qv[u].y * kr[ib + u].y;
            const float p2 = qv[u].z * kr[ib + u].z, p3 = qv[u].w * kr[ib + u].w;
            dot = dot + p0;
            dot = dot + p1;
            dot = dot + p2;
            dot = dot + p3;
          }
        }
      }
    } else {
      dot = chain_dot(0.0f, q, kt + lane * LD, h4);
    }
    a.S[((size_t)t * a.nq + h) * a.max_seq + tk0 + lane] = dot * a.scale;
  }
}

constexpr int kPvThreads = 256;

// Softmax of the n = pos0 + t + 1 scores of (t, h) and the weighted V sum
// for head dimensions DPB*g .. DPB*g + DPB - 1 (test_model_trace.c:408-426):
//   m = S[0], then every larger score (a NaN S[0] stays; later NaNs never
//   win); e_i = expf(S_i - m); sum = (((0 + e_0) + e_1) + ...) (the
//   sequential sum: one chain, or block_seq_sum for the long rows of
//   prefill);
//   p_i = e_i * (1 / (sum + 1e-9)); out_d = (((0 + p_0 v_0d) + p_1 v_1d) + ...).
// The weighted sum runs over chunks of CH positions: every thread forms
// products p_i * v_id of the chunk into a transposed LDS tile [d][i] (the
// next chunk's V loads already in flight), then lanes d < DPB sum their row
// with pure dependent adds.  Products past n are 0 * 0 = +0 (no-ops).
template <int DPB>
__global__ __launch_bounds__(kPvThreads) void attn_softmax_pv_kernel(AttnArgs a) {
  constexpr int CH = 16384 / DPB;                  // positions per chunk
  constexpr int Q4 = DPB / 4;                      // float4 per position
  constexpr int NL = CH * Q4 / kPvThreads;         // float4 per thread per chunk
  constexpr int LDT = CH + 4;
  extern __shared__ float lds[];
  const int hd = a.hd;
  int bx, h;
  attn_xcd_map(a.xcd_map, &bx, &h);
  const int t = blockIdx.z;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int n = a.pos0 + t + 1;
  float* es = lds;                                  // [max_seq, rounded up to 4]
  float* pt = lds + ((a.max_seq + 3) & ~3);         // [DPB][LDT]
  __shared__ float red[kPvThreads / kWave];
  __shared__ SeqSumScratch seq;
  const int kvh = h / (a.nq / a.nkv);
  const int d0 = DPB * bx;
  const int dl = min(DPB, hd - d0);
  const float* vbase = a.vc + (size_t)kvh * a.max_seq * hd + d0;
  const int nch = (n + CH - 1) / CH;
  float4 rg[NL];
  auto load = [&](int c) {
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int i = tid + kPvThreads * u;
      const int pos = c * CH + i / Q4, q4 = i % Q4;
      rg[u] = (pos < n && 4 * q4 < dl) ? *reinterpret_cast<const float4*>(vbase + (size_t)pos * hd + 4 * q4)
                                       : zero4();
    }
  };
  auto store = [&](int c) {
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int i = tid + kPvThreads * u;
      const int lp = i / Q4, q4 = i % Q4, pos = c * CH + lp;
      const float pk = pos < n ? es[pos] : 0.0f;
      float* col = pt + 4 * q4 * LDT + lp;
      col[0] = pk * rg[u].x;
      col[LDT] = pk * rg[u].y;
      col[2 * LDT] = pk * rg[u].z;
      col[3 * LDT] = pk * rg[u].w;
    }
  };
  // the scores first (into registers when they fit), then the first V
  // tile, which loads while the softmax runs (a thread's loads complete in
  // order, so the max waits for the scores alone)
  const float* Srow = a.S + ((size_t)t * a.nq + h) * a.max_seq;
  constexpr int SR = 8;
  const bool s_regs = n <= SR * kPvThreads;
  float sr[SR];
  if (s_regs) {
#pragma unroll
    for (int u = 0; u < SR; ++u) {
      const int i = tid + kPvThreads * u;
      sr[u] = i < n ? Srow[i] : 0.0f;
    }
  }
  load(0);
  float mx = -__builtin_inff();
  if (s_regs) {
#pragma unroll
    for (int u = 0; u < SR; ++u) {
      const int i = tid + kPvThreads * u;
      if (i < n) {
        const float s = sr[u];
        es[i] = s;
        if (s == s && s > mx) mx = s;
      }
    }
  } else {
    for (int i = tid; i < n; i += kPvThreads) {
      const float s = Srow[i];
      es[i] = s;
      if (s == s && s > mx) mx = s;
    }
  }
  // order-free max over the non-NaN scores (-inf when there is none)
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off, kWave);
    mx = o > mx ? o : mx;
  }
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < kPvThreads / kWave; ++w) m = red[w] > m ? red[w] : m;
  const float s0 = es[0];
  if (s0 != s0) m = s0;
  for (int i = tid; i < n; i += kPvThreads) es[i] = expf_glibc(es[i] - m);
  for (int i = n + tid; i < ((n + 3) & ~3); i += kPvThreads) es[i] = 0.0f;
  __syncthreads();
  // the sum: by the whole block for long rows (prefill), else one chain in
  // thread 0 (block_seq_sum's fixed cost exceeds a chain of a few hundred)
  float esum;
  if constexpr (DPB >= 128) {
    esum = block_seq_sum<kPvThreads>(es, n, seq);
  } else {
    if (tid == 0) seq.result = chain_sum(0.0f, es, (n + 3) / 4);
    __syncthreads();
    esum = seq.result;
  }
  const float inv = 1.0f / (esum + 1e-9f);
  for (int i = tid; i < n; i += kPvThreads) es[i] = es[i] * inv;
  __syncthreads();
  float out = 0.0f;
  // the next product's first chunks toward the memory-side cache (values
  // unused), requested once the V tile is in LDS so that no wait for V or
  // the scores counts them
  constexpr int PFN = kAttnPfRows * kAttnPfCols / 4 / kPvThreads;
  float4 pfv[PFN];
  const bool pf = a.pf_w && t == 0 && DPB == 16;
  for (int c = 0; c < nch; ++c) {
    store(c);
    if (c + 1 < nch) load(c + 1);
    if (c == 0 && pf) {
      const int b = (int)blockIdx.x + (int)gridDim.x * (int)blockIdx.y;
#pragma unroll
      for (int u = 0; u < PFN; ++u) {
        const int i = tid + kPvThreads * u;
        const int row = kAttnPfRows * b + i / (kAttnPfCols / 4), c4 = i % (kAttnPfCols / 4);
        pfv[u] = row < a.pf_n && 4 * c4 + 4 <= a.pf_ld
                     ? *reinterpret_cast<const float4*>(a.pf_w + (size_t)row * a.pf_ld + 4 * c4)
                     : zero4();
      }
    }
    __syncthreads();
    const int np = min(CH, n - c * CH);
    if (tid < dl) out = chain_sum(out, pt + tid * LDT, (np + 3) / 4);
    __syncthreads();
  }
  if (tid < dl) a.H[(size_t)t * a.nq * hd + (size_t)h * hd + d0 + tid] = out;
  if (pf) {
#pragma unroll
    for (int u = 0; u < PFN; ++u) asm volatile("" ::"v"(pfv[u].x));   // keeps the requests
  }
}

// ---- many query rows (prefill): several rows share each staged K / V tile ----
//
// The one-row kernels above read the whole key / value prefix once per
// query row (T^2/2 rows of hd floats for T new rows); these read it once per
// kSq (scores) or kQt (softmax and V sums) rows.  Same chains, same order:
// bit-identical results.
constexpr int kQt = 8;

// Scores of query rows t0 .. t0 + kSq - 1 (t0 = kSq blockIdx.z) of head
// blockIdx.y against keys tk0 .. tk0 + 63 (tk0 = 64 blockIdx.x): K rows and
// queries staged in LDS with coalesced loads; wave w runs the chains of rows
// w, w + 4, w + 8, w + 12 side by side, lane = key.  q must already be
// normed and rotated (heads_kernel).  S as attn_scores_kernel, key <= pos0 +
// t only.
constexpr int kSq = 16;                 // query rows per block
constexpr int kSqPerWave = kSq / 4;     // chains per lane

__global__ __launch_bounds__(256) void attn_scores_qt_kernel(AttnArgs a) {
  extern __shared__ float lds[];
  const int hd = a.hd, h4 = hd / 4, LD = hd + 4;
  float* kt = lds;             // [64][LD]
  float* qs = kt + 64 * LD;    // [kSq][hd]
  const int h = blockIdx.y, t0 = blockIdx.z * kSq, tk0 = blockIdx.x * 64;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nt = min(kSq, a.T - t0);
  const int Pmax = a.pos0 + t0 + nt - 1;
  if (tk0 > Pmax) return;   // every key of the block is masked (uniform)
  const int kvh = h / (a.nq / a.nkv);
  const int rows = min(64, Pmax + 1 - tk0);
  const float* kbase = a.kc + ((size_t)kvh * a.max_seq + tk0) * hd;
  // K rows (rows past `rows` read row rows - 1; never used), then the queries
  // (rows past nt read row nt - 1)
  for (int base = 0; base < 64 * h4; base += 256 * 8) {
    float4 r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + tid + 256 * u, rr = min(i / h4, rows - 1);
      r[u] = i < 64 * h4 ? *reinterpret_cast<const float4*>(kbase + (size_t)rr * hd + 4 * (i % h4)) : zero4();
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + tid + 256 * u;
      if (i < 64 * h4) *reinterpret_cast<float4*>(kt + (i / h4) * LD + 4 * (i % h4)) = r[u];
    }
  }
  for (int i = tid; i < kSq * h4; i += 256) {
    const int qr = min(i / h4, nt - 1);
    *reinterpret_cast<float4*>(qs + (i / h4) * hd + 4 * (i % h4)) =
        *reinterpret_cast<const float4*>(a.qkv + (size_t)(t0 + qr) * a.ld + (size_t)h * hd + 4 * (i % h4));
  }
  __syncthreads();
  const int key = tk0 + lane;
  if (lane >= rows) return;
  const float4* k4 = reinterpret_cast<const float4*>(kt + lane * LD);
  float dot[kSqPerWave];
#pragma unroll
  for (int u = 0; u < kSqPerWave; ++u) dot[u] = 0.0f;
  for (int c = 0; c < h4; ++c) {
    const float4 k = k4[c];
    float4 x[kSqPerWave];
#pragma unroll
    for (int u = 0; u < kSqPerWave; ++u) x[u] = reinterpret_cast<const float4*>(qs + (wave + 4 * u) * hd)[c];
    float p[kSqPerWave][4];
#pragma unroll
    for (int u = 0; u < kSqPerWave; ++u) {
      p[u][0] = x[u].x * k.x;
      p[u][1] = x[u].y * k.y;
      p[u][2] = x[u].z * k.z;
      p[u][3] = x[u].w * k.w;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int u = 0; u < kSqPerWave; ++u) dot[u] = dot[u] + p[u][e];
  }
#pragma unroll
  for (int u = 0; u < kSqPerWave; ++u) {
    const int q = wave + 4 * u;
    if (q < nt && key <= a.pos0 + t0 + q) a.S[((size_t)(t0 + q) * a.nq + h) * a.max_seq + key] = dot[u] * a.scale;
  }
}

// Softmax of the score rows of the query-tiled path, in place, once per
// (query row, head): one wave each, row t of head h (n = pos0 + t + 1
// scores) staged in LDS; its max by the wave (order-free; a NaN first score
// wins, as in attn_softmax_pv_kernel), e = expf(s - m), the sum chain in
// lane 0, p = e * (1 / (sum + 1e-9)) written back over the scores
// (test_model_trace.c:411-420).  attn_pv_qt_kernel then reads p.
constexpr int kSmRowWaves = 4;

size_t attn_softmax_rows_lds(int pos0, int T) {
  return (size_t)kSmRowWaves * (size_t)((pos0 + T + 3) & ~3) * 4;
}

__global__ __launch_bounds__(kSmRowWaves * kWave) void attn_softmax_rows_kernel(AttnArgs a) {
  extern __shared__ float smr[];   // [kSmRowWaves][ES]
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int h = blockIdx.x * kSmRowWaves + wave, t = blockIdx.y;
  if (h >= a.nq) return;   // (no block barriers below)
  const int ES = (a.pos0 + a.T + 3) & ~3;
  float* er = smr + (size_t)wave * ES;
  const int n = a.pos0 + t + 1;
  float* Srow = a.S + ((size_t)t * a.nq + h) * a.max_seq;
  float mx = -__builtin_inff();
  for (int i = lane; i < n; i += kWave) {
    const float v = Srow[i];
    er[i] = v;
    if (v == v && v > mx) mx = v;
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off, kWave);
    mx = o > mx ? o : mx;
  }
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
  const float s0 = er[0];
  const float m = s0 != s0 ? s0 : mx;
  for (int i = lane; i < n; i += kWave) er[i] = expf_glibc(er[i] - m);
  for (int i = n + lane; i < ((n + 3) & ~3); i += kWave) er[i] = 0.0f;
  __threadfence_block();
  __builtin_amdgcn_wave_barrier();
  float inv = 0.0f;
  if (lane == 0) inv = 1.0f / (chain_sum(0.0f, er, (n + 3) / 4) + 1e-9f);
  inv = __shfl(inv, 0, kWave);
  for (int i = lane; i < n; i += kWave) Srow[i] = er[i] * inv;
}

// Weighted V sum of query rows t0 .. t0 + kQt - 1 of head blockIdx.y for
// dimensions d0 .. d0 + kPvDpb - 1: thread (qi, dd) = (tid / kPvDpb, tid %
// kPvDpb).  Row qi's probabilities (n = pos0 + t0 + qi + 1, from
// attn_softmax_rows_kernel) in LDS; V staged kPvCh positions at a time and
// out = (((0 + p_0 v_0) + p_1 v_1) + ...) over the row's positions in order.
constexpr int kPvDpb = 32;
constexpr int kPvCh = 128;
static_assert(kQt * kPvDpb == 256, "one thread per (row, dimension)");

size_t attn_pv_qt_lds(int pos0, int T) {
  const size_t es = (size_t)((pos0 + T + 3) & ~3);
  return ((size_t)kQt * es + (size_t)kPvCh * kPvDpb) * 4;
}

__global__ __launch_bounds__(256) void attn_pv_qt_kernel(AttnArgs a) {
  extern __shared__ float lds[];
  const int hd = a.hd;
  const int h = blockIdx.y, t0 = blockIdx.z * kQt, d0 = blockIdx.x * kPvDpb;
  const int tid = threadIdx.x, qi = tid / kPvDpb, dd = tid % kPvDpb;
  const int ES = (a.pos0 + a.T + 3) & ~3;            // row stride of es
  float* es = lds;                                    // [kQt][ES]
  float* vt = es + (size_t)kQt * ES;                  // [kPvCh][kPvDpb]
  const int nt = min(kQt, a.T - t0);
  const int nmax = a.pos0 + t0 + nt;                  // positions of the last row
  const bool row_live = qi < nt;
  const int n = row_live ? a.pos0 + t0 + qi + 1 : 0;
  const int kvh = h / (a.nq / a.nkv);
  float* er = es + (size_t)qi * ES;
  // 1. the row's probabilities (attn_softmax_rows_kernel)
  const float* Srow = a.S + ((size_t)(t0 + qi) * a.nq + h) * a.max_seq;
  for (int i = dd; i < n; i += kPvDpb) er[i] = Srow[i];
  for (int i = n + dd; i < ((n + 3) & ~3); i += kPvDpb) er[i] = 0.0f;
  // 2. the weighted V sums
  const float* vbase = a.vc + (size_t)kvh * a.max_seq * hd + d0;
  const int dl = min(kPvDpb, hd - d0);
  float out = 0.0f;
  for (int c0 = 0; c0 < nmax; c0 += kPvCh) {
    __syncthreads();   // the previous chunk's readers are done (and p is complete)
    constexpr int PER = kPvCh * kPvDpb / 4 / 256;   // float4 per thread
    float4 r[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = tid + 256 * u;                  // float4 index in the tile
      const int pos = c0 + i / (kPvDpb / 4), c = 4 * (i % (kPvDpb / 4));
      r[u] = (pos < nmax && c < dl) ? *reinterpret_cast<const float4*>(vbase + (size_t)pos * hd + c) : zero4();
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) reinterpret_cast<float4*>(vt)[tid + 256 * u] = r[u];
    __syncthreads();
    const int np = min(kPvCh, n - c0);
    int j = 0;
    // 16 positions' operands read ahead of their chain steps
    for (; j + 16 <= np; j += 16) {
      float4 pe[4];
      float vv[16];
#pragma unroll
      for (int u = 0; u < 4; ++u) pe[u] = *reinterpret_cast<const float4*>(er + c0 + j + 4 * u);
#pragma unroll
      for (int u = 0; u < 16; ++u) vv[u] = vt[(j + u) * kPvDpb + dd];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float p0 = pe[u].x * vv[4 * u], p1 = pe[u].y * vv[4 * u + 1];
        const float p2 = pe[u].z * vv[4 * u + 2], p3 = pe[u].w * vv[4 * u + 3];
        out = out + p0;
        out = out + p1;
        out = out + p2;
        out = out + p3;
      }
    }
    for (; j < np; ++j) {
      const float pv = er[c0 + j] * vt[j * kPvDpb + dd];
      out = out + pv;
    }
  }
  if (row_live && dd < dl) a.H[(size_t)(t0 + qi) * a.nq * hd + (size_t)h * hd + d0 + dd] = out;
}

// ---------------------------------------------------------------- misc

__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ ids,
                                                    const float* __restrict__ emb, int V, int D,
                                                    float* __restrict__ x) {
  const int t = blockIdx.x;
  int id = ids[t];
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);
  const float* src = emb + (size_t)id * D;
  float* dst = x + (size_t)t * D;
  for (int i = threadIdx.x; i < D; i += 256) dst[i] = src[i];
}

constexpr int kGreedyThreads = 1024;

// The smallest v over the block (all threads get it); red: one int per wave.
__device__ int block_min(int v, int* red) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int o = __shfl_xor(v, off, kWave);
    v = o < v ? o : v;
  }
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  for (int w = 0; w < (int)blockDim.x / kWave; ++w) v = red[w] < v ? red[w] : v;
  return v;
}

// The reference's next token (test_model_trace.c:735-746): softmax_rows of
// the logits, then the first index of the largest probability.  With m the
// largest logit: a NaN or +inf logit, or m = -inf, turns every probability
// into NaN and the scan stays at 0.  Otherwise e_i = expf(v_i - m) <= 1
// with e = 1 at the maximum, the probabilities are e_i * inv with a normal
// inv = 1 / (sum + 1e-9) (sum >= 1), and any e_i <= 1 - 2^-24 gives a
// product that rounds below inv (the exact (1 - 2^-24) inv is at least
// half an ulp of inv under it, and exactly representable when it is only
// that), so the answer is the first i with expf(v_i - m) == 1.
// part (optional): the largest value of every block of `rows` consecutive
// logits (NaN if the block holds one), written by the head's product; only
// the first block whose maximum qualifies is then scanned.
__global__ __launch_bounds__(kGreedyThreads) void greedy_kernel(const float* __restrict__ v, int n,
                                                               const float* __restrict__ part,
                                                               int rows, int32_t* out,
                                                               int32_t* hist, int32_t* hist_pos) {
  __shared__ float fred[kGreedyThreads / kWave];
  __shared__ int ired[kGreedyThreads / kWave];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const float* src = part ? part : v;
  const int ns = part ? (n + rows - 1) / rows : n;
  // up to GR values a thread are loaded at once and kept in registers for
  // both scans (a loop of dependent loads costs a round trip per value)
  constexpr int GR = 12;
  const bool in_regs = ns <= GR * kGreedyThreads;
  float sv[GR];
  float mx = -__builtin_inff();
  if (in_regs) {
#pragma unroll
    for (int u = 0; u < GR; ++u) {
      const int i = tid + kGreedyThreads * u;
      sv[u] = i < ns ? src[i] : -__builtin_inff();
    }
#pragma unroll
    for (int u = 0; u < GR; ++u) mx = nan_max(mx, sv[u]);
  } else {
    for (int i = tid; i < ns; i += kGreedyThreads) mx = nan_max(mx, src[i]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = nan_max(mx, __shfl_xor(mx, off, kWave));
  if (lane == 0) fred[wave] = mx;
  __syncthreads();
  float m = fred[0];
  for (int w = 1; w < kGreedyThreads / kWave; ++w) m = nan_max(m, fred[w]);
  int ans = 0;
  if (m == m && m != __builtin_inff() && m != -__builtin_inff()) {
    int first = INT_MAX;
    if (in_regs) {
#pragma unroll
      for (int u = GR - 1; u >= 0; --u) {
        // (d < -1e-6: e^d < 1 - 9.9e-7, 16 ulps under 1, so expf(d) < 1)
        const int i = tid + kGreedyThreads * u;
        const float d = sv[u] - m;
        if (i < ns && !(d < -1e-6f) && expf_glibc(d) == 1.0f) first = i;
      }
    } else {
      for (int i = tid; i < ns; i += kGreedyThreads)
        if (expf_glibc(src[i] - m) == 1.0f) { first = i; break; }
    }
    first = block_min(first, ired);
    if (part && first != INT_MAX) {
      const int lo = first * rows, hi = min(n, lo + rows);
      first = INT_MAX;
      for (int i = lo + tid; i < hi; i += kGreedyThreads)
        if (expf_glibc(v[i] - m) == 1.0f) { first = i; break; }
      first = block_min(first, ired);
    }
    ans = first == INT_MAX ? 0 : first;
  }
  if (tid == 0) {
    out[0] = ans;
    if (hist) {
      const int p = *hist_pos;
      hist[p] = ans;
      *hist_pos = p + 1;
    }
  }
}

constexpr int kSmThreads = 1024;
constexpr int kSmChunk = 8192;

// softmax_rows (test_model_trace.c:260-272) of one row in place: max as in
// the attention softmax, e_i = expf(v_i - max) in parallel, the sum as one
// chain over LDS-staged chunks, then v_i = e_i * (1 / (sum + 1e-9)).
__global__ __launch_bounds__(kSmThreads) void softmax_vec_kernel(float* v, int n) {
  __shared__ float chunk[kSmChunk];
  __shared__ float red[kSmThreads / kWave];
  __shared__ float inv_s;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  float mx = -__builtin_inff();
  for (int i = tid; i < n; i += kSmThreads) {
    const float s = v[i];
    if (s == s && s > mx) mx = s;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off, kWave);
    mx = o > mx ? o : mx;
  }
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < kSmThreads / kWave; ++w) m = red[w] > m ? red[w] : m;
  const float v0 = v[0];
  if (v0 != v0) m = v0;
  __syncthreads();
  float sum = 0.0f;
  for (int base = 0; base < n; base += kSmChunk) {
    const int len = min(kSmChunk, n - base);
    for (int i = tid; i < len; i += kSmThreads) {
      const float e = expf_glibc(v[base + i] - m);
      chunk[i] = e;
      v[base + i] = e;
    }
    __syncthreads();
    if (tid == 0)
      for (int i = 0; i < len; ++i) sum = sum + chunk[i];
    __syncthreads();
  }
  if (tid == 0) inv_s = 1.0f / (sum + 1e-9f);
  __syncthreads();
  const float inv = inv_s;
  for (int i = tid; i < n; i += kSmThreads) v[i] = v[i] * inv;
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Dynamic LDS above 64 KB needs the kernel's attribute raised; the largest
// size set per kernel is remembered so the runtime is called once per size.
std::mutex g_lds_mu;
std::unordered_map<const void*, size_t> g_lds_set;

template <class F>
moe_status set_lds(F* fn, size_t bytes, const char* what) {
  if (bytes <= 65536) return MOE_OK;
  std::lock_guard<std::mutex> lk(g_lds_mu);
  size_t& cur = g_lds_set[(const void*)fn];
  if (bytes <= cur) return MOE_OK;
  moe_status st = check_hip(hipFuncSetAttribute((const void*)fn,
                                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes),
                            what);
  if (st == MOE_OK) cur = bytes;
  return st;
}

size_t gemv_lds(int RW, int NP, int M, int K, bool norm) {
  const int KC = RW >= 16 ? 4096 / RW : 256;
  return ((size_t)(NP + 1) * M * RW * (KC + 4) + (norm ? (size_t)M * K : 0)) * 4;
}

template <int RW, bool NORM, int PACK, int NP, int MMX = 64 / RW>
moe_status launch_gemv(const DenseArgs& a, hipStream_t s) {
  const size_t lds = gemv_lds(RW, NP, a.M, a.K, NORM);
  moe_status st = set_lds(dense_gemv_kernel<RW, NORM, PACK, NP, MMX>, lds, "gemv LDS attribute");
  if (st) return st;
  hipLaunchKernelGGL((dense_gemv_kernel<RW, NORM, PACK, NP, MMX>), dim3((unsigned)((a.N + RW - 1) / RW)),
                     dim3(64 * (NP + 1)), lds, s, a);
  return check_hip(hipGetLastError(), "dense gemv launch");
}

template <int CT, int CE, int KC>
moe_status launch_tile(const DenseArgs& a, hipStream_t s) {
  constexpr size_t lds = 2 * (size_t)(16 * CT + 16 * CE) * (KC + 4) * 4;
  dim3 grid((unsigned)((a.N + 16 * CE - 1) / (16 * CE)), (unsigned)((a.M + 16 * CT - 1) / (16 * CT)));
  hipLaunchKernelGGL((dense_tile_kernel<CT, CE, KC>), grid, dim3(256), lds, s, a);
  return check_hip(hipGetLastError(), "dense tile launch");
}

}  // namespace

// Producer waves of the few-token GEMV: three for one token (the LDS of four
// product buffers fits), one otherwise; the wide one-token products (the
// vocabulary head) keep three as well: their rows stream from HBM and more
// producers keep more bytes in flight.
constexpr int kNpOne = 3;
constexpr int kNpWide = 3;

bool dense_norm_ok(int M, int K) {
  return M >= 1 && M <= 4 && K % 4 == 0 && K <= 8192 &&
         gemv_lds(16, M == 1 ? kNpOne : 1, M, K, true) <= 150 * 1024;
}

// The last block selects with one wave per token, keys (8 bytes per
// logit, up to 1024) in the product buffers.
bool dense_select_ok(int M, int N) { return M >= 1 && M <= 4 && N <= 1024; }

bool dense_amax_ok(const DenseArgs& a) {
  return a.M == 1 && a.K > 0 && a.K % 4 == 0 && a.lda % 4 == 0 && a.ldw % 4 == 0 && al16(a.A) &&
         al16(a.W) && !a.norm && !a.sel_counter;
}

// 16 rows a block also for the vocabulary head: each chunk then reads 1 KB
// of every row (64-row blocks read 256 B pieces), measured ~0.4% faster per
// decode token even though the greedy choice then reads 4x the block maxima.
int dense_amax_rows(int) { return 16; }

// One token against few rows: the row kernel.
// Row kernel: one token, or up to 4 without the fused rmsnorm and packing.
bool dense_row_ok(const DenseArgs& a, bool vec) {
  const bool rows = a.M == 1 || (a.M <= 4 && !a.norm);
  return rows && a.N <= 1024 && vec && a.K <= kRowMaxK && !a.amax_part;
}

bool dense_rows4_ok(const DenseArgs& a, bool vec) {
  return a.M > 4 && a.M <= 16 && !a.norm && !a.sel_counter && !a.amax_part && a.N <= 1024 && vec &&
         a.K <= kRowsMaxK;
}

// The block-parallel rows kernel instead of the chain kernel for 5-16
// given rows (MOEHIP_ROUTER_ROWS4=1, for comparison).
bool rows4_kernel_chosen() {
  static const bool v = getenv("MOEHIP_ROUTER_ROWS4") != nullptr;
  return v;
}

bool dense_rows4_path(const DenseArgs& a) {
  const bool vec = a.K > 0 && a.K % 4 == 0 && a.lda % 4 == 0 && a.ldw % 4 == 0 && al16(a.A) &&
                   al16(a.W);
  return a.N > 0 && dense_rows4_ok(a, vec);
}

bool dense_row_path(const DenseArgs& a) {
  const bool vec = a.K > 0 && a.K % 4 == 0 && a.lda % 4 == 0 && a.ldw % 4 == 0 && al16(a.A) &&
                   al16(a.W);
  return a.N > 0 && dense_row_ok(a, vec) && (!a.norm || dense_norm_ok(a.M, a.K));
}

template <bool NORM, int PACK>
moe_status launch_row(const DenseArgs& a, hipStream_t s) {
  const size_t lds = (size_t)2 * a.K * 4;
  moe_status st = set_lds(dense_row_kernel<NORM, PACK>, lds, "row kernel LDS attribute");
  if (st) return st;
  hipLaunchKernelGGL((dense_row_kernel<NORM, PACK>), dim3((unsigned)a.N, (unsigned)a.M), dim3(kRowThreads), lds,
                     s, a);
  if ((st = check_hip(hipGetLastError(), "dense row launch"))) return st;
  if (!a.sel_counter || a.sel_defer) return MOE_OK;
  hipLaunchKernelGGL(row_finish_kernel, dim3(1), dim3(kWave * a.M), 0, s, a);
  return check_hip(hipGetLastError(), "row finish launch");
}

moe_status dense_matmul(const DenseArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return MOE_OK;
  if (a.amax_part) {
    if (!dense_amax_ok(a))
      return set_error(MOE_ERR_ARG, "dense matmul: block maxima need one aligned row");
    return launch_gemv<16, false, 0, kNpOne>(a, s);
  }
  if (a.sel_counter && (!dense_select_ok(a.M, a.N) || a.sel_topk < 1 || a.sel_topk > kMaxTopK ||
                        a.ldc != a.N))
    return set_error(MOE_ERR_ARG, "dense matmul: fused selection needs M <= 4, N <= 1024");
  if (a.K <= 0) return set_error(MOE_ERR_ARG, "dense matmul: K = %d", a.K);
  if (a.sel_defer && (!a.sel_counter || !dense_row_path(a)))
    return set_error(MOE_ERR_ARG, "dense matmul: a deferred selection needs the row kernel");
  const bool vec = a.K % 4 == 0 && a.lda % 4 == 0 && a.ldw % 4 == 0 && al16(a.A) && al16(a.W);
  if (a.norm) {
    if (!vec || !dense_norm_ok(a.M, a.K))
      return set_error(MOE_ERR_ARG, "dense matmul: fused rmsnorm needs M <= 4 aligned rows");
    if (a.pack_dtype && (!a.sel_counter || !a.pack_part || !a.pack_tabs))
      return set_error(MOE_ERR_ARG, "dense matmul: packing needs the fused selection");
    if (dense_row_ok(a, vec)) {
      if (a.pack_dtype == 2) return launch_row<true, 2>(a, s);
      if (a.pack_dtype == 3) return launch_row<true, 3>(a, s);
      return launch_row<true, 0>(a, s);
    }
    if (a.M == 1) {
      if (a.pack_dtype == 2) return launch_gemv<16, true, 2, kNpOne>(a, s);
      if (a.pack_dtype == 3) return launch_gemv<16, true, 3, kNpOne>(a, s);
      // 8 rows a block: twice the blocks of the 16-row shape that the
      // packing paths keep (the [Wq;Wk;Wv] product 17.5 -> 16.9-17.2 us);
      // its four buffers (8320 floats) hold the squares of a row of K <= 8320
      if (a.K <= (kNpOne + 1) * 8 * 260) return launch_gemv<8, true, 0, kNpOne, 1>(a, s);
      return launch_gemv<16, true, 0, kNpOne>(a, s);
    }
    if (a.pack_dtype == 2) return launch_gemv<16, true, 2, 1>(a, s);
    if (a.pack_dtype == 3) return launch_gemv<16, true, 3, 1>(a, s);
    return launch_gemv<16, true, 0, 1>(a, s);
  }
  if (!vec) {
    const long long total = (long long)a.M * a.N;
    hipLaunchKernelGGL(dense_generic_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    return check_hip(hipGetLastError(), "dense generic launch");
  }
  if (a.pack_dtype && (!a.pack_part || !a.pack_tabs ||
                       !((a.sel_counter && dense_row_ok(a, vec)) || dense_rows4_ok(a, vec))))
    return set_error(MOE_ERR_ARG, "dense matmul: packing given rows needs the row kernel and the fused "
                                  "selection, or the 5-16 token rows kernel");
  if (dense_row_ok(a, vec)) {
    if (a.pack_dtype == 2) return launch_row<false, 2>(a, s);
    if (a.pack_dtype == 3) return launch_row<false, 3>(a, s);
    return launch_row<false, 0>(a, s);
  }
  if (dense_rows4_ok(a, vec) && !rows4_kernel_chosen()) {
    // 5-16 given rows against few rows (the router): one block per row, one
    // consumer lane per token's sequential chain, three producer waves
    if (a.pack_dtype == 2) return launch_gemv<1, false, 2, 3, 16>(a, s);
    if (a.pack_dtype == 3) return launch_gemv<1, false, 3, 3, 16>(a, s);
    return launch_gemv<1, false, 0, 3, 16>(a, s);
  }
  if (dense_rows4_ok(a, vec)) {
    const size_t lds = (size_t)kRowGroups * a.K * 4;
    const dim3 grid((unsigned)a.N, (unsigned)((a.M + kRowGroups - 1) / kRowGroups));
    moe_status st;
    if (a.pack_dtype == 2) {
      if ((st = set_lds(dense_rows4_kernel<2>, lds, "rows kernel LDS attribute"))) return st;
      hipLaunchKernelGGL(dense_rows4_kernel<2>, grid, dim3(kRowThreads), lds, s, a);
    } else if (a.pack_dtype == 3) {
      if ((st = set_lds(dense_rows4_kernel<3>, lds, "rows kernel LDS attribute"))) return st;
      hipLaunchKernelGGL(dense_rows4_kernel<3>, grid, dim3(kRowThreads), lds, s, a);
    } else {
      if ((st = set_lds(dense_rows4_kernel<0>, lds, "rows kernel LDS attribute"))) return st;
      hipLaunchKernelGGL(dense_rows4_kernel<0>, grid, dim3(kRowThreads), lds, s, a);
    }
    return check_hip(hipGetLastError(), "dense rows launch");
  }
  if (a.sel_counter) {
    if (!vec) return set_error(MOE_ERR_ARG, "dense matmul: fused selection needs aligned rows");
    return a.M == 1 ? launch_gemv<16, false, 0, kNpOne>(a, s) : launch_gemv<16, false, 0, 1>(a, s);
  }
  if (a.M == 1 && a.N >= 65536) {
    return launch_gemv<64, false, 0, kNpWide>(a, s);
  } else if (a.M <= 2 && a.N >= 32768) {
    return launch_gemv<32, false, 0, 1>(a, s);
  } else if (a.M == 1) {
    // 8 rows a block (the Wo product: 128 -> 256 blocks, 18.0 -> 17.0-17.6 us)
    return launch_gemv<8, false, 0, kNpOne, 1>(a, s);
  } else if (a.M <= 4) {
    return launch_gemv<16, false, 0, 1>(a, s);
  } else if (a.M <= 16) {
    return launch_gemv<4, false, 0, 1>(a, s);
  } else if (a.M >= 256 && (long long)((a.N + 63) / 64) * ((a.M + 63) / 64) >= 1024) {
    // 64 x 64 tiles only with >= 1024 blocks; below that 32-token x 64-row
    // tiles keep more waves on each SIMD (prefill at T = 512: Wo 256 and
    // [Wq;Wk;Wv] 640 blocks of 64 x 64; the model's 512-token prefill 49.7
    // -> 43.5 ms with 32 x 32 tiles, 41.5 -> 39.8 ms with 32 x 64: eight
    // chains a thread, each x value read for four rows)
    return launch_tile<4, 4, 32>(a, s);
  } else {
    return launch_tile<2, 4, 64>(a, s);
  }
  return check_hip(hipGetLastError(), "dense gemv launch");
}

moe_status embed_rows(const int32_t* ids, int T, const float* emb, int V, int D, float* x,
                      hipStream_t s) {
  if (T <= 0) return MOE_OK;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)T), dim3(256), 0, s, ids, emb, V, D, x);
  return check_hip(hipGetLastError(), "embed launch");
}

moe_status heads_norm_rope(const HeadArgs& a, hipStream_t s) {
  if (a.T <= 0) return MOE_OK;
  if (a.hd > kMaxHd || (a.hd & 1)) return set_error(MOE_ERR_ARG, "head_dim %d unsupported", a.hd);
  hipLaunchKernelGGL(heads_kernel, dim3((unsigned)a.T, (unsigned)(a.nq + 2 * a.nkv)), dim3(64), 0, s, a);
  return check_hip(hipGetLastError(), "heads launch");
}

moe_status attention_rows(const AttnArgs& a, hipStream_t s) {
  if (a.T <= 0) return MOE_OK;
  if (a.hd % 4 || a.hd > kMaxHd) return set_error(MOE_ERR_ARG, "attention: head_dim %d", a.hd);
  if (a.fuse_heads && a.T != 1) return set_error(MOE_ERR_ARG, "attention: fused heads need T == 1");
  if (a.T > 4 && !a.fuse_heads && a.nkv > 0 && a.nq % a.nkv == 0 &&
      attn_pv_qt_lds(a.pos0, a.T) <= 160 * 1024 && !getenv("MOEHIP_ATTN_ROWWISE")) {
    const unsigned qg = (unsigned)((a.T + kQt - 1) / kQt);
    const size_t lds_s = ((size_t)64 * (a.hd + 4) + (size_t)kSq * a.hd) * 4;
    moe_status st;
    if ((st = set_lds(attn_scores_qt_kernel, lds_s, "scores LDS attribute"))) return st;
    hipLaunchKernelGGL(attn_scores_qt_kernel,
                       dim3((unsigned)((a.pos0 + a.T + 63) / 64), (unsigned)a.nq, (unsigned)((a.T + kSq - 1) / kSq)),
                       dim3(256), lds_s, s, a);
    if ((st = check_hip(hipGetLastError(), "scores launch"))) return st;
    const size_t lds_m = attn_softmax_rows_lds(a.pos0, a.T);
    if ((st = set_lds(attn_softmax_rows_kernel, lds_m, "softmax rows LDS attribute"))) return st;
    hipLaunchKernelGGL(attn_softmax_rows_kernel, dim3((unsigned)((a.nq + kSmRowWaves - 1) / kSmRowWaves), (unsigned)a.T),
                       dim3(kSmRowWaves * kWave), lds_m, s, a);
    if ((st = check_hip(hipGetLastError(), "softmax rows launch"))) return st;
    const size_t lds_p = attn_pv_qt_lds(a.pos0, a.T);
    if ((st = set_lds(attn_pv_qt_kernel, lds_p, "softmax/pv LDS attribute"))) return st;
    hipLaunchKernelGGL(attn_pv_qt_kernel, dim3((unsigned)((a.hd + kPvDpb - 1) / kPvDpb), (unsigned)a.nq, qg),
                       dim3(256), lds_p, s, a);
    return check_hip(hipGetLastError(), "softmax/pv launch");
  }
  const int nmax = a.pos0 + a.T;   // positions of the last row
  const size_t hdp = (size_t)((a.hd + 3) & ~3);
  static const bool no_xcd = getenv("MOEHIP_ATTN_NO_XCD") != nullptr;
  AttnArgs ax = a;
  ax.xcd_map = no_xcd ? 0 : 1;
  const dim3 sgrid((unsigned)((nmax + 63) / 64), (unsigned)a.nq, (unsigned)a.T);
  moe_status st;
  if (a.hd <= kRegHd) {
    const size_t lds_s = 10 * hdp * 4;
    hipLaunchKernelGGL(attn_scores_kernel<true>, sgrid, dim3(64), lds_s, s, ax);
  } else {
    const size_t lds_s = (9 * hdp + 64 * (size_t)(a.hd + 4)) * 4;
    if ((st = set_lds(attn_scores_kernel<false>, lds_s, "scores LDS attribute"))) return st;
    hipLaunchKernelGGL(attn_scores_kernel<false>, sgrid, dim3(64), lds_s, s, ax);
  }
  if ((st = check_hip(hipGetLastError(), "scores launch"))) return st;
  const size_t es_f = (size_t)((a.max_seq + 3) & ~3);
  if (a.T <= 4) {
    const size_t lds_p = (es_f + 16 * (16384 / 16 + 4)) * 4;
    if ((st = set_lds(attn_softmax_pv_kernel<16>, lds_p, "softmax/pv LDS attribute"))) return st;
    hipLaunchKernelGGL(attn_softmax_pv_kernel<16>, dim3((unsigned)((a.hd + 15) / 16), (unsigned)a.nq, (unsigned)a.T),
                       dim3(kPvThreads), lds_p, s, ax);
  } else {
    const size_t lds_p = (es_f + 128 * (16384 / 128 + 4)) * 4;
    if ((st = set_lds(attn_softmax_pv_kernel<128>, lds_p, "softmax/pv LDS attribute"))) return st;
    hipLaunchKernelGGL(attn_softmax_pv_kernel<128>, dim3((unsigned)((a.hd + 127) / 128), (unsigned)a.nq, (unsigned)a.T),
                       dim3(kPvThreads), lds_p, s, ax);
  }
  return check_hip(hipGetLastError(), "softmax/pv launch");
}

moe_status greedy_vec(const float* v, int n, const float* part, int rows, int32_t* out,
                      int32_t* out_hist, int32_t* hist_pos, hipStream_t s) {
  if (n <= 0) return set_error(MOE_ERR_ARG, "greedy: %d logits", n);
  if (part && rows <= 0) return set_error(MOE_ERR_ARG, "greedy: %d rows per partial", rows);
  hipLaunchKernelGGL(greedy_kernel, dim3(1), dim3(kGreedyThreads), 0, s, v, n, part, rows, out,
                     out_hist, hist_pos);
  return check_hip(hipGetLastError(), "greedy launch");
}

moe_status softmax_vec(float* v, int n, hipStream_t s) {
  hipLaunchKernelGGL(softmax_vec_kernel, dim3(1), dim3(kSmThreads), 0, s, v, n);
  return check_hip(hipGetLastError(), "softmax launch");
}

}  // namespace moe
