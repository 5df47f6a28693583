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
#include <math.h>

#include "dense.h"
#include "moe_device.h"

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

__device__ __forceinline__ float dense_epilogue(const DenseArgs& a, int m, int n, float acc) {
  float c = acc;
  if (a.bias) c = c + a.bias[n];
  if (a.resid) c = a.resid[(size_t)m * a.ldr + n] + c;
  return c;
}

// ---------------------------------------------------------------- products

// Few tokens (M <= 64 / RW): one wave per block owns RW output rows; lane
// m * RW + r runs the chain of token m and row n0 + r.  The RW weight rows
// and the M token rows stream through two LDS buffers in chunks of KC
// columns (RW * KC = 4096 floats), the next chunk held in registers while
// the current one is consumed.  Columns past K are zero in both operands:
// 0 * 0 = +0 and adding +0 leaves a chain unchanged (a chain that starts at
// +0 and adds round-to-nearest sums is never -0).  Rows past N read row
// N - 1 and are not stored.  K % 4 == 0, 16-byte aligned rows.
template <int RW>
__global__ __launch_bounds__(64) void dense_gemv_kernel(DenseArgs a) {
  constexpr int KC = 4096 / RW;
  constexpr int V4 = KC / 4;                 // float4 per row chunk (<= 64)
  constexpr int LD = KC + 4;                 // padded LDS row (floats)
  constexpr int RPL = 64 / V4;               // rows one load instruction covers
  constexpr int NW = RW / RPL;               // W float4 per lane per chunk
  constexpr int MM = 64 / RW;                // token rows staged
  constexpr int NX = (MM + RPL - 1) / RPL;   // A float4 per lane per chunk
  __shared__ float wl[2][RW * LD];
  __shared__ float xl[2][MM * LD];
  const int lane = threadIdx.x;
  const int n0 = blockIdx.x * RW;
  const int c4 = lane % V4, r0 = lane / V4;
  const int M = a.M, N = a.N, K = a.K;
  const int nc = (K + KC - 1) / KC;
  const float* wsrc[NW];
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    const int n = min(n0 + r0 + v * RPL, N - 1);
    wsrc[v] = a.W + (size_t)n * a.ldw + 4 * c4;
  }
  const float* xsrc[NX];
#pragma unroll
  for (int v = 0; v < NX; ++v) {
    const int m = min(r0 + v * RPL, M - 1);
    xsrc[v] = a.A + (size_t)m * a.lda + 4 * c4;
  }
  float4 rw[NW], rx[NX];
  auto load = [&](int c) {
    const int k = c * KC + 4 * c4;
    const bool in = k < K;
#pragma unroll
    for (int v = 0; v < NW; ++v)
      rw[v] = in ? *reinterpret_cast<const float4*>(wsrc[v] + (size_t)c * KC) : zero4();
#pragma unroll
    for (int v = 0; v < NX; ++v)
      rx[v] = in ? *reinterpret_cast<const float4*>(xsrc[v] + (size_t)c * KC) : zero4();
  };
  auto store = [&](int b) {
#pragma unroll
    for (int v = 0; v < NW; ++v)
      *reinterpret_cast<float4*>(&wl[b][(r0 + v * RPL) * LD + 4 * c4]) = rw[v];
#pragma unroll
    for (int v = 0; v < NX; ++v)
      if (r0 + v * RPL < MM) *reinterpret_cast<float4*>(&xl[b][(r0 + v * RPL) * LD + 4 * c4]) = rx[v];
  };
  load(0);
  store(0);
  if (nc > 1) load(1);
  const int m = lane / RW, r = lane % RW;
  float acc = 0.0f;
  for (int c = 0; c < nc; ++c) {
    __syncthreads();
    if (c + 1 < nc) {
      store((c + 1) & 1);
      if (c + 2 < nc) load(c + 2);
    }
    acc = chain_dot(acc, &xl[c & 1][m * LD], &wl[c & 1][r * LD], V4);
  }
  const int n = n0 + r;
  if (m < M && n < N) a.C[(size_t)m * a.ldc + n] = dense_epilogue(a, m, n, acc);
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

// Block (t, h) over the heads of row t of [Q | K | V] (each head hd wide, so
// head h starts at h * hd): q/k heads get the per-head RMSNorm of
// test_model_trace.c:381-402 (sequential sum of squares in lane 0,
// inv = 1/sqrtf(msq/hd + eps), v = (v*inv)*w) and RoPE (:326-336: the pair
// (i, i + hd/2) turned by the tabled cos/sin of position pos0 + t, each
// product rounded, then one subtraction / addition); Q stays in place, K
// and V rows are written to the caches.
__global__ __launch_bounds__(64) void heads_kernel(HeadArgs a) {
  __shared__ float v[kMaxHd];
  __shared__ float inv_s;
  const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int hd = a.hd, d2 = hd / 2, pos = a.pos0 + t;
  float* row = a.qkv + (size_t)t * a.ld + (size_t)h * hd;
  for (int d = lane; d < hd; d += 64) v[d] = row[d];
  if (h >= a.nq + a.nkv) {   // V head: into the cache unchanged
    float* dst = a.vc + ((size_t)(h - a.nq - a.nkv) * a.max_seq + pos) * hd;
    for (int d = lane; d < hd; d += 64) dst[d] = v[d];
    return;
  }
  const bool isq = h < a.nq;
  const float* w = isq ? a.q_norm : a.k_norm;
  __syncthreads();
  if (w) {
    if (lane == 0) {
      float msq = 0.0f;
      for (int d = 0; d < hd; ++d) {
        const float z = v[d];
        const float zz = z * z;
        msq = msq + zz;
      }
      const float mean = msq / (float)hd;
      inv_s = 1.0f / sqrtf(mean + a.eps);
    }
    __syncthreads();
    const float inv = inv_s;
    for (int d = lane; d < hd; d += 64) {
      const float s = v[d] * inv;
      v[d] = s * w[d];
    }
    __syncthreads();
  }
  float* out = isq ? row : a.kc + ((size_t)(h - a.nq) * a.max_seq + pos) * hd;
  const float* cs = a.rope_cos + (size_t)pos * d2;
  const float* sn = a.rope_sin + (size_t)pos * d2;
  for (int i = lane; i < d2; i += 64) {
    const float e = v[i], o = v[i + d2], c = cs[i], s = sn[i];
    const float ec = e * c, os = o * s, oc = o * c, es = e * s;
    out[i] = ec - os;
    out[i + d2] = oc + es;
  }
}

// ---------------------------------------------------------------- attention

// Scores of query row t, head h against cache positions tk0 .. tk0 + 63
// (<= pos0 + t): the 64 K rows are staged in LDS, lane i runs the chain
// dot = (((0 + q0 k0) + q1 k1) + ...) over hd and stores dot * scale.
__global__ __launch_bounds__(64) void attn_scores_kernel(AttnArgs a) {
  extern __shared__ float lds[];
  const int hd = a.hd, LD = hd + 4;
  float* q = lds;               // [hd]
  float* kt = lds + hd;         // [64][LD]
  const int t = blockIdx.z, h = blockIdx.y, lane = threadIdx.x;
  const int P = a.pos0 + t;
  const int tk0 = blockIdx.x * 64;
  if (tk0 > P) return;
  const int kvh = h / (a.nq / a.nkv);
  const float* qrow = a.qkv + (size_t)t * a.ld + (size_t)h * hd;
  for (int d = lane; d < hd; d += 64) q[d] = qrow[d];
  const float* kbase = a.kc + ((size_t)kvh * a.max_seq + tk0) * hd;
  const int rows = min(64, P + 1 - tk0);
  const int h4 = hd / 4;
  for (int i = lane; i < rows * h4; i += 64) {
    const int rr = i / h4, c4 = i % h4;
    *reinterpret_cast<float4*>(kt + rr * LD + 4 * c4) =
        *reinterpret_cast<const float4*>(kbase + (size_t)rr * hd + 4 * c4);
  }
  __syncthreads();
  if (lane < rows) {
    const float dot = chain_dot(0.0f, q, kt + lane * LD, h4);
    a.S[((size_t)t * a.nq + h) * a.max_seq + tk0 + lane] = dot * a.scale;
  }
}

constexpr int kPvThreads = 256;
constexpr int kPvChunk = 128;   // positions per staged V tile

// Softmax of the n = pos0 + t + 1 scores of (t, h) and the weighted V sum
// for head dimensions 64g .. 64g + 63 (test_model_trace.c:408-426):
//   m = S[0], then every larger score (a NaN S[0] stays; later NaNs never
//   win); e_i = expf(S_i - m); sum = (((0 + e_0) + e_1) + ...) in lane 0;
//   p_i = e_i * (1 / (sum + 1e-9)); out_d = (((0 + p_0 v_0d) + p_1 v_1d) + ...)
// in wave 0, lane d, with V tiles of kPvChunk positions staged in LDS by the
// whole block a tile ahead.
__global__ __launch_bounds__(kPvThreads) void attn_softmax_pv_kernel(AttnArgs a) {
  extern __shared__ float lds[];
  const int hd = a.hd;
  const int t = blockIdx.z, h = blockIdx.y, g = blockIdx.x;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int n = a.pos0 + t + 1;
  float* es = lds;                                  // [max_seq, rounded up to 4]
  float* vt = lds + ((a.max_seq + 3) & ~3);         // [2][kPvChunk][64]
  __shared__ float red[kPvThreads / kWave];
  __shared__ float inv_s;
  const float* Srow = a.S + ((size_t)t * a.nq + h) * a.max_seq;
  float mx = -__builtin_inff();
  bool any = false;
  for (int i = tid; i < n; i += kPvThreads) {
    const float s = Srow[i];
    es[i] = s;
    if (s == s && (!any || s > mx)) { mx = s; any = true; }
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
  __syncthreads();
  if (tid == 0) {
    const float4* e4 = reinterpret_cast<const float4*>(es);
    float sum = 0.0f;
    int i = 0;
    for (; i + 64 <= n; i += 64) {
      float4 ev[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) ev[j] = e4[i / 4 + j];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        sum = sum + ev[j].x;
        sum = sum + ev[j].y;
        sum = sum + ev[j].z;
        sum = sum + ev[j].w;
      }
    }
    for (; i < n; ++i) sum = sum + es[i];
    inv_s = 1.0f / (sum + 1e-9f);
  }
  __syncthreads();
  const float inv = inv_s;
  for (int i = tid; i < n; i += kPvThreads) es[i] = es[i] * inv;
  // weighted V sum: tiles of kPvChunk positions x 64 dims, double buffered
  const int kvh = h / (a.nq / a.nkv);
  const int d0 = 64 * g;
  const int dl = min(64, hd - d0);
  const float* vbase = a.vc + (size_t)kvh * a.max_seq * hd + d0;
  constexpr int NV = kPvChunk * 16 / kPvThreads;    // float4 per thread per tile
  const int nch = (n + kPvChunk - 1) / kPvChunk;
  float4 rg[NV];
  auto load = [&](int c) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = tid + kPvThreads * v;
      const int p = c * kPvChunk + i / 16, c4 = i % 16;
      rg[v] = (p < n && 4 * c4 < dl) ? *reinterpret_cast<const float4*>(vbase + (size_t)p * hd + 4 * c4)
                                     : zero4();
    }
  };
  auto store = [&](int b) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = tid + kPvThreads * v;
      *reinterpret_cast<float4*>(vt + (b * kPvChunk + i / 16) * 64 + 4 * (i % 16)) = rg[v];
    }
  };
  load(0);
  store(0);
  if (nch > 1) load(1);
  float out = 0.0f;
  for (int c = 0; c < nch; ++c) {
    __syncthreads();
    if (c + 1 < nch) {
      store((c + 1) & 1);
      if (c + 2 < nch) load(c + 2);
    }
    if (wave == 0) {
      const float* tile = vt + (c & 1) * kPvChunk * 64 + lane;
      const int p0 = c * kPvChunk;
      const int np = min(kPvChunk, n - p0);
      int j = 0;
      for (; j + 16 <= np; j += 16) {
        float pv[16], vv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) { pv[u] = es[p0 + j + u]; vv[u] = tile[(j + u) * 64]; }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const float pr = pv[u] * vv[u];
          out = out + pr;
        }
      }
      for (; j < np; ++j) {
        const float pr = es[p0 + j] * tile[j * 64];
        out = out + pr;
      }
    }
  }
  if (wave == 0 && lane < dl)
    a.H[(size_t)t * a.nq * hd + (size_t)h * hd + d0 + lane] = out;
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

// (v, i) beats (w, j): v is not NaN and (larger, or equal with a lower index)
__device__ __forceinline__ bool am_beats(float v, int i, float w, int j) {
  if (i < 0 || v != v) return false;
  if (j < 0) return true;
  return v > w || (v == w && i < j);
}

constexpr int kArgThreads = 1024;

__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float* __restrict__ v, int n,
                                                             int32_t* out, int32_t* hist,
                                                             int32_t* hist_pos) {
  __shared__ float bv_s[kArgThreads / kWave];
  __shared__ int bi_s[kArgThreads / kWave];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  float bv = 0.0f;
  int bi = -1;
  for (int i = tid; i < n; i += kArgThreads) {
    const float x = v[i];
    if (am_beats(x, i, bv, bi)) { bv = x; bi = i; }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (am_beats(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane == 0) { bv_s[wave] = bv; bi_s[wave] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgThreads / kWave; ++w)
      if (am_beats(bv_s[w], bi_s[w], bv, bi)) { bv = bv_s[w]; bi = bi_s[w]; }
    // the scan starts from index 0: a NaN there is never replaced
    const float v0 = v[0];
    const int r = (v0 != v0 || bi < 0) ? 0 : bi;
    out[0] = r;
    if (hist) {
      const int p = *hist_pos;
      hist[p] = r;
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

template <class F>
moe_status set_lds(F* fn, size_t bytes, const char* what) {
  if (bytes <= 65536) return MOE_OK;
  return check_hip(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)bytes), what);
}

template <int CT, int CE, int KC>
moe_status launch_tile(const DenseArgs& a, hipStream_t s) {
  constexpr size_t lds = 2 * (size_t)(16 * CT + 16 * CE) * (KC + 4) * 4;
  dim3 grid((unsigned)((a.N + 16 * CE - 1) / (16 * CE)), (unsigned)((a.M + 16 * CT - 1) / (16 * CT)));
  hipLaunchKernelGGL((dense_tile_kernel<CT, CE, KC>), grid, dim3(256), lds, s, a);
  return check_hip(hipGetLastError(), "dense tile launch");
}

}  // namespace

moe_status dense_matmul(const DenseArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return MOE_OK;
  if (a.K <= 0) return set_error(MOE_ERR_ARG, "dense matmul: K = %d", a.K);
  const bool vec = a.K % 4 == 0 && a.lda % 4 == 0 && a.ldw % 4 == 0 && al16(a.A) && al16(a.W);
  if (!vec) {
    const long long total = (long long)a.M * a.N;
    hipLaunchKernelGGL(dense_generic_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    return check_hip(hipGetLastError(), "dense generic launch");
  }
  if (a.M == 1 && a.N >= 65536) {
    hipLaunchKernelGGL(dense_gemv_kernel<64>, dim3((unsigned)((a.N + 63) / 64)), dim3(64), 0, s, a);
  } else if (a.M <= 2 && a.N >= 32768) {
    hipLaunchKernelGGL(dense_gemv_kernel<32>, dim3((unsigned)((a.N + 31) / 32)), dim3(64), 0, s, a);
  } else if (a.M <= 4) {
    hipLaunchKernelGGL(dense_gemv_kernel<16>, dim3((unsigned)((a.N + 15) / 16)), dim3(64), 0, s, a);
  } else if (a.M >= 256) {
    return launch_tile<4, 4, 32>(a, s);
  } else {
    return launch_tile<2, 2, 64>(a, s);
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
  const int nmax = a.pos0 + a.T;   // positions of the last row
  const size_t lds_s = (size_t)(a.hd + 64 * (a.hd + 4)) * 4;
  moe_status st = set_lds(attn_scores_kernel, lds_s, "scores LDS attribute");
  if (st) return st;
  hipLaunchKernelGGL(attn_scores_kernel, dim3((unsigned)((nmax + 63) / 64), (unsigned)a.nq, (unsigned)a.T),
                     dim3(64), lds_s, s, a);
  if ((st = check_hip(hipGetLastError(), "scores launch"))) return st;
  const size_t lds_p = ((size_t)((a.max_seq + 3) & ~3) + 2 * kPvChunk * 64) * 4;
  if ((st = set_lds(attn_softmax_pv_kernel, lds_p, "softmax/pv LDS attribute"))) return st;
  hipLaunchKernelGGL(attn_softmax_pv_kernel, dim3((unsigned)((a.hd + 63) / 64), (unsigned)a.nq, (unsigned)a.T),
                     dim3(kPvThreads), lds_p, s, a);
  return check_hip(hipGetLastError(), "softmax/pv launch");
}

moe_status argmax_vec(const float* v, int n, int32_t* out, int32_t* out_hist, int32_t* hist_pos,
                      hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgThreads), 0, s, v, n, out, out_hist, hist_pos);
  return check_hip(hipGetLastError(), "argmax launch");
}

moe_status softmax_vec(float* v, int n, hipStream_t s) {
  hipLaunchKernelGGL(softmax_vec_kernel, dim3(1), dim3(kSmThreads), 0, s, v, n);
  return check_hip(hipGetLastError(), "softmax launch");
}

}  // namespace moe
