/*
 * moe_oracle.c - CPU restatement of moe.cc's quantized expert path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built with gcc -O2 and no -march,
 * the flags of the reference Makefile:3, so that fp32 expressions are
 * evaluated exactly as in the reference: every multiply and add rounded on
 * its own (x86-64 baseline has no FMA), IEEE division and sqrt, glibc expf.
 *
 * Integer dot products use uint32_t so that the wrap-around the reference
 * gets from int32 overflow (signed overflow compiled by gcc to plain add/imul)
 * is reproduced with defined behaviour.
 *
 * The same file is also built with -fopenmp (liboracle_omp.so): the loops
 * marked `omp parallel for` hand whole output rows (or whole tokens, or whole
 * heads) to threads, each of which runs the row's arithmetic in the
 * reference's order, so that build's results are bit-identical to the
 * single-thread one (tests/test_oracle_omp.py).  Without -fopenmp the
 * pragmas are ignored.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int32_t orc_f2i_trunc(float v) {
  /* cvttss2si: in-range iff -2^31 <= v < 2^31 (NaN fails both tests). */
  if (v >= -2147483648.0f && v < 2147483648.0f) return (int32_t)v;
  return INT32_MIN;
}

/* kernels.c:51-74.  Loop order m, n, k; the activation is truncated to int
 * (kernels.c:66) and multiplied by the int8 weight in int32 (kernels.c:67);
 * epilogue (kernels.c:71): one int->float conversion, a division by 127.0f,
 * a multiplication by the row scale.  One output row per call of q8_row (a
 * function of its own, so that the threaded build's loop body is the same
 * code as the single-thread one's). */
static float q8_row(const float* a, const int8_t* w, int K, float scale) {
  uint32_t acc = 0;
  for (int k = 0; k < K; ++k) {
    int32_t ai = orc_f2i_trunc(a[k] * 127.0f);
    acc += (uint32_t)ai * (uint32_t)(int32_t)w[k];
  }
  float f = (float)(int32_t)acc;
  f = f / 127.0f;
  return f * scale;
}

void orc_gemv_q8(const float* A, const int8_t* Bq, const float* Bs, float* C,
                 int M, int N, int K) {
  for (int m = 0; m < M; ++m) {
    const float* a = A + (size_t)m * K;
    float* c = C + (size_t)m * N;
#pragma omp parallel for schedule(static) if ((size_t)N * (size_t)K >= 65536)
    for (int n = 0; n < N; ++n) c[n] = q8_row(a, Bq + (size_t)n * K, K, Bs[n]);
  }
}

/* kernels.c:96-128.  Row n starts at byte n*(K/2) (integer division, so an
 * odd K makes rows overlap by one byte, as in the reference).  Byte k/2 holds
 * column k in its low nibble and column k+1 in its high nibble, both stored
 * with a +8 offset (kernels.c:110-112).  For odd K the final high nibble is
 * skipped (kernels.c:116-121).  Epilogue divides by 7.0f (kernels.c:125). */
static float q4_row(const float* a, const uint8_t* w, int K, float scale) {
  uint32_t acc = 0;
  for (int k = 0; k < K; k += 2) {
    uint8_t byte = w[k / 2];
    int32_t lo = (int32_t)(byte & 0x0F) - 8;
    int32_t hi = (int32_t)((byte >> 4) & 0x0F) - 8;
    int32_t a0 = orc_f2i_trunc(a[k] * 7.0f);
    acc += (uint32_t)a0 * (uint32_t)lo;
    if (k + 1 < K) {
      int32_t a1 = orc_f2i_trunc(a[k + 1] * 7.0f);
      acc += (uint32_t)a1 * (uint32_t)hi;
    }
  }
  float f = (float)(int32_t)acc;
  f = f / 7.0f;
  return f * scale;
}

void orc_gemv_q4(const float* A, const uint8_t* Bq, const float* Bs, float* C,
                 int M, int N, int K) {
  for (int m = 0; m < M; ++m) {
    const float* a = A + (size_t)m * K;
    float* c = C + (size_t)m * N;
#pragma omp parallel for schedule(static) if ((size_t)N * (size_t)K >= 65536)
    for (int n = 0; n < N; ++n) c[n] = q4_row(a, Bq + (size_t)n * (size_t)(K / 2), K, Bs[n]);
  }
}

/* test_model_trace.c:213-227: fp32 accumulator, k ascending, one rounding
 * for each product and each sum. */
static float f32_dot(const float* a, const float* b, int K) {
  float acc = 0.0f;
  for (int k = 0; k < K; ++k) {
    float p = a[k] * b[k];
    acc = acc + p;
  }
  return acc;
}

void orc_matmul_f32(const float* A, const float* B, float* C, int M, int N, int K) {
#pragma omp parallel for collapse(2) schedule(static) \
    if ((size_t)M * (size_t)N * (size_t)K >= 65536)
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n)
      C[(size_t)m * N + n] = f32_dot(A + (size_t)m * K, B + (size_t)n * K, K);
}

/* kernels.c:149-181 */
void orc_matmul_adaptive(const float* A, const float* W_fp32, const orc_qweight* W_q,
                         float* C, int M, int N, int K) {
  if (W_q == NULL) {
    orc_matmul_f32(A, W_fp32, C, M, N, K);
  } else if (W_q->dtype == 2) {
    orc_gemv_q8(A, W_q->q, W_q->s, C, M, N, K);
  } else if (W_q->dtype == 3) {
    orc_gemv_q4(A, (const uint8_t*)W_q->q, W_q->s, C, M, N, K);
  } else {
    memset(C, 0, sizeof(float) * (size_t)M * (size_t)N);
  }
}

/* test_model_trace.c:229-236: x / (1 + expf(-x)) */
void orc_silu(float* x, int n) {
  for (int i = 0; i < n; ++i) {
    float v = x[i];
    float den = 1.0f + expf(-v);
    x[i] = v / den;
  }
}

/* test_model_trace.c:241-255: sequential sum of squares, divide by D,
 * inv = 1/sqrtf(msq+eps), y = (x*inv)*w. */
void orc_rmsnorm(const float* x, const float* w, int T, int D, float eps, float* y) {
  for (int t = 0; t < T; ++t) {
    const float* xt = x + (size_t)t * D;
    float* yt = y + (size_t)t * D;
    float msq = 0.0f;
    for (int i = 0; i < D; ++i) {
      float sq = xt[i] * xt[i];
      msq = msq + sq;
    }
    msq = msq / (float)D;
    float inv = 1.0f / sqrtf(msq + eps);
    for (int i = 0; i < D; ++i) {
      float v = xt[i] * inv;
      yt[i] = v * (w ? w[i] : 1.0f);
    }
  }
}

/* test_model_trace.c:275-288: descending insertion list initialised to
 * (-inf, -1); a value enters before the first entry it strictly exceeds, so
 * equal values keep the lower index first and NaN / -inf never enter. */
void orc_topk_desc(const float* x, int E, int k, int* idx, float* val) {
  for (int i = 0; i < k; ++i) { val[i] = -INFINITY; idx[i] = -1; }
  for (int e = 0; e < E; ++e) {
    float v = x[e];
    int at = -1;
    for (int i = 0; i < k; ++i) {
      if (v > val[i]) { at = i; break; }
    }
    if (at < 0) continue;
    for (int j = k - 1; j > at; --j) { val[j] = val[j - 1]; idx[j] = idx[j - 1]; }
    val[at] = v;
    idx[at] = e;
  }
}

/* test_model_trace.c:482-487 */
void orc_softmax_topk(float* val, int k) {
  float mx = val[0];
  for (int i = 1; i < k; ++i) if (val[i] > mx) mx = val[i];
  float sum = 0.0f;
  for (int i = 0; i < k; ++i) {
    val[i] = expf(val[i] - mx);
    sum = sum + val[i];
  }
  float inv = 1.0f / (sum + 1e-9f);
  for (int i = 0; i < k; ++i) val[i] = val[i] * inv;
}

/* test_model_trace.c:478-515 for one token t: top-k and softmax of its
 * logits, then per rank gate -> SiLU -> up -> g*u -> down and the weighted
 * sum in rank order into at[D] (starting from zeros). */
static void moe_token(const float* xt, const float* lg, int D, int E, int top_k, int d_ff,
                      const orc_qweight* Wg, const orc_qweight* Wu, const orc_qweight* Wd,
                      float* at, int* idx_out, float* p_out) {
  float* g = (float*)malloc(sizeof(float) * (size_t)d_ff);
  float* u = (float*)malloc(sizeof(float) * (size_t)d_ff);
  float* y = (float*)malloc(sizeof(float) * (size_t)D);
  int* idx = (int*)malloc(sizeof(int) * (size_t)top_k);
  float* val = (float*)malloc(sizeof(float) * (size_t)top_k);
  /* :480-487 top-k then softmax over the selected logits */
  orc_topk_desc(lg, E, top_k, idx, val);
  orc_softmax_topk(val, top_k);
  if (idx_out) memcpy(idx_out, idx, sizeof(int) * (size_t)top_k);
  if (p_out) memcpy(p_out, val, sizeof(float) * (size_t)top_k);
  for (int j = 0; j < top_k; ++j) {
    int e = idx[j];
    float p = val[j];
    /* Fewer than top_k selectable logits (NaN / -inf) leave idx -1, which
     * the reference dereferences (UB at :496); here such a slot adds
     * nothing. */
    if (e < 0) continue;
    /* :496-503 gate -> SiLU -> up -> g*u -> down */
    orc_matmul_adaptive(xt, NULL, &Wg[e], g, 1, d_ff, D);
    orc_silu(g, d_ff);
    orc_matmul_adaptive(xt, NULL, &Wu[e], u, 1, d_ff, D);
    for (int i = 0; i < d_ff; ++i) g[i] = g[i] * u[i];
    orc_matmul_adaptive(g, NULL, &Wd[e], y, 1, D, d_ff);
    /* :513 weighted sum in rank order */
    for (int i = 0; i < D; ++i) {
      float py = p * y[i];
      at[i] = at[i] + py;
    }
  }
  free(g); free(u); free(y); free(idx); free(val);
}

/* test_model_trace.c:463-517 (quantized-expert branch, 494-503). */
void orc_moe_block(const float* x_norm, const float* x_resid, int T, int D,
                   int E, int top_k, int d_ff,
                   const float* router_w, const float* router_b,
                   const orc_qweight* Wg, const orc_qweight* Wu, const orc_qweight* Wd,
                   float* out, int* idx_out, float* p_out, float* logits_out) {
  float* logits = (float*)malloc(sizeof(float) * (size_t)T * (size_t)E);
  float* acc = (float*)calloc((size_t)T * (size_t)D, sizeof(float));

  /* :465-468 router logits (+ optional bias) */
  orc_matmul_f32(x_norm, router_w, logits, T, E, D);
  if (router_b) {
    for (int t = 0; t < T; ++t)
      for (int e = 0; e < E; ++e) logits[(size_t)t * E + e] += router_b[e];
  }
  if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)T * (size_t)E);

  /* Tokens are independent after the router: with -fopenmp each thread
   * takes whole tokens from 4 tokens on; fewer run one at a time outside
   * any parallel region, so that their GEMVs split by rows instead. */
#define MOE_TOKEN(t)                                                                      \
  moe_token(x_norm + (size_t)(t) * D, logits + (size_t)(t) * E, D, E, top_k, d_ff, Wg, Wu, \
            Wd, acc + (size_t)(t) * D, idx_out ? idx_out + (size_t)(t) * top_k : NULL,      \
            p_out ? p_out + (size_t)(t) * top_k : NULL)
  if (T >= 4) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int t = 0; t < T; ++t) MOE_TOKEN(t);
  } else {
    for (int t = 0; t < T; ++t) MOE_TOKEN(t);
  }
#undef MOE_TOKEN
  /* :517 residual */
  for (size_t i = 0; i < (size_t)T * (size_t)D; ++i)
    out[i] = x_resid ? x_resid[i] + acc[i] : acc[i];

  free(logits); free(acc);
}

/* export.py:23-27.  amax per row, clamped below at 1e-8 (as an fp32 value),
 * divided by 127 in fp32; q = round-half-to-even(w / s). */
void orc_quant_q8_rows(const float* W, int N, int K, int8_t* q, float* s) {
  for (int n = 0; n < N; ++n) {
    const float* w = W + (size_t)n * K;
    float amax = 0.0f;
    for (int k = 0; k < K; ++k) { float a = fabsf(w[k]); if (a > amax) amax = a; }
    if (amax < 1e-8f) amax = 1e-8f;
    float sc = amax / 127.0f;
    s[n] = sc;
    for (int k = 0; k < K; ++k) {
      float r = nearbyintf(w[k] / sc);
      q[(size_t)n * K + k] = (int8_t)(int)r;
    }
  }
}

/* export.py:29-36 */
void orc_quant_q4_rows(const float* W, int N, int K, uint8_t* q, float* s) {
  for (int n = 0; n < N; ++n) {
    const float* w = W + (size_t)n * K;
    float amax = 0.0f;
    for (int k = 0; k < K; ++k) { float a = fabsf(w[k]); if (a > amax) amax = a; }
    if (amax < 1e-8f) amax = 1e-8f;
    float sc = amax / 7.0f;
    s[n] = sc;
    for (int j = 0; j < K / 2; ++j) {
      float r0 = nearbyintf(w[2 * j] / sc);
      float r1 = nearbyintf(w[2 * j + 1] / sc);
      if (r0 < -8.0f) r0 = -8.0f;
      if (r0 > 7.0f) r0 = 7.0f;
      if (r1 < -8.0f) r1 = -8.0f;
      if (r1 > 7.0f) r1 = 7.0f;
      uint32_t lo = (uint32_t)((int)r0 + 8), hi = (uint32_t)((int)r1 + 8);
      q[(size_t)n * (K / 2) + j] = (uint8_t)(lo | (hi << 4));
    }
  }
}

/* ---- seeded synthetic data ---- */
static uint64_t splitmix64(uint64_t* x) {
  uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
typedef struct { uint64_t s[4]; } xo256;
static void xo_seed(xo256* r, uint64_t seed) {
  uint64_t x = seed;
  for (int i = 0; i < 4; ++i) r->s[i] = splitmix64(&x);
}
static uint64_t xo_next(xo256* r) {
  uint64_t* s = r->s;
  uint64_t out = rotl64(s[1] * 5, 7) * 9;
  uint64_t t = s[1] << 17;
  s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl64(s[3], 45);
  return out;
}

void orc_fill_normal(float* out, size_t n, uint64_t seed, float mean, float std) {
  xo256 r;
  xo_seed(&r, seed);
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    /* u1 in (0, 1], u2 in [0, 1) */
    double u1 = (double)((xo_next(&r) >> 11) + 1) * 0x1.0p-53;
    double u2 = (double)(xo_next(&r) >> 11) * 0x1.0p-53;
    double rad = sqrt(-2.0 * log(u1));
    double z0 = rad * cos(two_pi * u2), z1 = rad * sin(two_pi * u2);
    out[i++] = (float)((double)mean + (double)std * z0);
    if (i < n) out[i++] = (float)((double)mean + (double)std * z1);
  }
}

void orc_fill_uniform_u32(uint32_t* out, size_t n, uint64_t seed) {
  xo256 r;
  xo_seed(&r, seed);
  for (size_t i = 0; i < n; ++i) out[i] = (uint32_t)(xo_next(&r) >> 32);
}

void orc_expf_array(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

uint64_t orc_expf_mismatch_u32range(uint32_t lo, uint32_t count, const float* dev,
                                    uint32_t* first_bad) {
  uint64_t bad = 0;
  for (uint32_t i = 0; i < count; ++i) {
    uint32_t bits = lo + i;
    float x, want;
    memcpy(&x, &bits, 4);
    want = expf(x);
    uint32_t wb, gb;
    memcpy(&wb, &want, 4);
    memcpy(&gb, &dev[i], 4);
    /* every NaN input gives a NaN; compare NaN-ness rather than payload */
    if (wb != gb && !(want != want && dev[i] != dev[i])) {
      if (bad == 0 && first_bad) *first_bad = bits;
      ++bad;
    }
  }
  return bad;
}

/* Threads the row-parallel loops use: 1 in the single-thread build. */
int orc_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
