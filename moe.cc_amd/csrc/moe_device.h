// moe_device.h - device-side arithmetic shared by the gfx950 kernels.
//
// Everything here exists to make GPU results bit-identical to moe.cc's CPU
// path (kernels.c, test_model_trace.c) compiled by gcc -O2 for x86-64:
//   * activation truncation with x86 cvttss2si semantics,
//   * exact integer dot products through int8 "limbs" and v_dot4_i32_i8,
//   * an expf that reproduces glibc 2.35's expf bit for bit,
//   * fp32 glue evaluated with separate roundings (the library is compiled
//     with -ffp-contract=off, so a*b+c is never fused).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kWave = 64;

// (int32_t)v as gcc compiles it for x86-64 (cvttss2si): truncation toward
// zero; NaN and values whose truncation leaves int32 give INT32_MIN.  The GPU
// conversion instruction saturates instead, so the out-of-range case is
// handled explicitly.  Used for kernels.c:66 and kernels.c:115-116.
__device__ __forceinline__ int32_t f2i_trunc_x86(float v) {
  // |v| < 2^31 is the in-range test (one compare); -2^31 itself and NaN fall
  // outside it and give INT32_MIN, as the x86 conversion does
  return __builtin_fabsf(v) < 2147483648.0f ? (int32_t)v : INT32_MIN;
}

// Number of signed int8 limbs needed so that sum_l limb_l * 256^l == a:
//   1 limb: [-128, 127]; 2 limbs: [-32896, 32639]; otherwise 4 limbs, which
//   represent every int32 modulo 2^32 (all the dot product needs, since the
//   reference accumulates in wrapping int32).
__device__ __forceinline__ int limbs_needed(int32_t a) {
  const uint32_t u = (uint32_t)a;
  const int n2 = u + 32896u < 65536u ? 2 : 4;   // a in [-32896, 32639]
  return u + 128u < 256u ? 1 : n2;             // a in [-128, 127]
}

// Splits a into 4 signed bytes (least significant first) with
// a == b0 + 256 b1 + 65536 b2 + 2^24 b3 (mod 2^32).  Returned as the raw
// byte values (0..255) ready to be packed into a dword.
__device__ __forceinline__ void split_limbs(int32_t a, uint32_t b[4]) {
  uint32_t r = (uint32_t)a;
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    int32_t lo = (int32_t)(int8_t)(r & 0xFFu);
    b[l] = (uint32_t)lo & 0xFFu;
    r = (uint32_t)((int32_t)(r - (uint32_t)lo) >> 8);
  }
}

__device__ __forceinline__ uint32_t pack4(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Combines per-limb partial sums: sum_l acc[l] << 8l, modulo 2^32.
template <int NL>
__device__ __forceinline__ uint32_t combine_limbs(const int32_t* acc) {
  uint32_t r = (uint32_t)acc[0];
  if (NL > 1) r += (uint32_t)acc[1] << 8;
  if (NL > 2) r += (uint32_t)acc[2] << 16;
  if (NL > 3) r += (uint32_t)acc[3] << 24;
  return r;
}

// Wrapping uint32 sum over the lanes of a group of W consecutive lanes
// (W a power of two <= 64); every lane of the group receives the total.
template <int W>
__device__ __forceinline__ uint32_t group_sum_u32(uint32_t v) {
#pragma unroll
  for (int off = W / 2; off > 0; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, W);
  return v;
}

// Correctly rounded x / d for x = (float) of an int32 and d = 127 or 7:
// q = RN(x * RN(1/d)), one exact remainder r = x - q*d (fma), q + r * RN(1/d)
// rounded once (Markstein's correction step).  Equal to the IEEE quotient for
// every int32 x and both divisors (exhaustive check on the device:
// moe_selfcheck_qdot_dev; on the host the same identity holds for all 2^32
// inputs).  Three operations instead of a full division sequence.
__device__ __forceinline__ float div_int_by_const(float x, float d) {
  const float inv = 1.0f / d;   // folded for the constant divisors
  const float q = x * inv;
  const float r = __builtin_fmaf(-q, d, x);
  return __builtin_fmaf(r, inv, q);
}

// kernels.c:71 / kernels.c:125 epilogue: ((float)dot / div) * scale, each
// operation rounded on its own.
__device__ __forceinline__ float qdot_epilogue(uint32_t dot, float div, float scale) {
  const float f = div_int_by_const((float)(int32_t)dot, div);
  return f * scale;
}

// ---------------------------------------------------------------------------
// expf, bit-identical to glibc 2.35 expf on x86-64 with FMA (the variant the
// host's ifunc selects).  Method: the published ARM Optimized Routines expf
// (also glibc's sysdeps/ieee754/flt-32/e_expf.c): x*32/ln2 = k + r, a 32-entry
// table of 2^(i/32) and a cubic in r, evaluated in double, with the fused
// multiply-adds a compiler contracts in that source under -mfma.  The table
// entries are the nearest doubles to 2^(i/32), minus i << 47.  Equality with
// the host expf on all 2^32 inputs is checked by tests/test_gpu_expf.py.
// ---------------------------------------------------------------------------
__constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

// tab: the 32 table entries (kExp2Tab or a copy, e.g. in LDS, which a
// kernel that evaluates many expf per lane reads with less latency).
// Branch-free: the polynomial path runs for every x (its table index is
// ki % 32, in range for any input) and the published special cases replace
// its result afterwards, one select each -- x above the overflow threshold
// (+inf included) +inf, x below the underflow threshold (-inf included) +0,
// NaN x + x -- so that many evaluations per lane schedule together instead
// of each in its own divergent region.
__device__ __forceinline__ float expf_glibc_t(float x, const uint64_t* tab) {
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = (double)x;
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd = kd - kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  uint64_t t = tab[ki % 32];
  t += ki << 47;
  const double s = __longlong_as_double((long long)t);
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  float e = (float)y;
  e = x > 0x1.62e42ep6f ? __builtin_inff() : e;
  e = x < -0x1.9fe368p6f ? 0.0f : e;
  return x != x ? x + x : e;
}

__device__ __forceinline__ float expf_glibc(float x) { return expf_glibc_t(x, kExp2Tab); }

// Hand-over between the waves of one block through LDS counters instead of
// a block barrier: the producing side stores or adds to a counter after
// its data (release), the consuming side polls it (acquire).  The poll is
// capped (2^22 polls, about a hundred times any kernel's own time) so that a
// kernel always exits; the users arrange that no wait depends on itself.
__device__ __forceinline__ void ring_wait(int* ctr, int target, bool nap) {
  for (int i = 0; i < (1 << 22); ++i) {
    if (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
    if (nap) __builtin_amdgcn_s_sleep(1);
  }
}
__device__ __forceinline__ void ring_post(int* ctr, int v) {
  __hip_atomic_store(ctr, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// acc = ((acc + p0) + p1) + ... over 4*n4 values of an LDS row (16-byte
// aligned): the sequential fp32 sum of the reference, as pure dependent adds
// (operands formed beforehand, by other lanes); 16 float4 are read ahead of
// their 64 adds.  A dependent v_add_f32 chain issues an add every 8 clocks
// on gfx950; with a multiply feeding each add it takes 12-13.
__device__ __forceinline__ float chain_sum(float acc, const float* p, int n4) {
  const float4* p4 = reinterpret_cast<const float4*>(p);
  int k4 = 0;
  for (; k4 + 16 <= n4; k4 += 16) {
    float4 v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = p4[k4 + i];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc = acc + v[i].x;
      acc = acc + v[i].y;
      acc = acc + v[i].z;
      acc = acc + v[i].w;
    }
  }
  for (; k4 < n4; ++k4) {
    const float4 v = p4[k4];
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
  }
  return acc;
}

// ---------------------------------------------------------------------------
// The sequential fp32 sum s = (((0 + p0) + p1) + ... + p_{n-1}), each add
// rounded, computed by a whole block in about n/8 dependent adds.
//
// The n values are split into kSeqSegs segments.  Segment j starts from the
// unknown partial sum s_j; its estimate e_j (the exact sum of p_0 .. p_{k-1}
// in double, rounded to fp32) is within a few ulps of s_j (the rounding
// errors of k adds grow like sqrt(k) ulps), so the segment's chain is run
// from the kSeqCands consecutive fp32 values centred on e_j: NT / kSeqSegs
// threads per segment, kSeqCands / that many independent chains each (which
// fill the add latency instead of lengthening it).  Then one wave walks the
// segments in order: s_0 = +0, and s_{j+1} is the chain output of the
// candidate whose bits equal s_j's.  A chain that starts from the same bits
// adds the same values in the same order, so that output is s_{j+1}
// exactly.  When no candidate matches (a far estimate, or NaN / inf among
// the values) the wave runs the segment's chain itself.  The result is
// bit-identical to the sequential loop in every case; only the latency
// depends on the values.
// ---------------------------------------------------------------------------
constexpr int kSeqSegs = 8;
constexpr int kSeqCands = 64;

struct SeqSumScratch {
  double part[kSeqSegs];
  uint32_t base[kSeqSegs];   // key of each segment's first candidate
  float out[kSeqSegs][kSeqCands];
  float result;
};

// Order-preserving integer image of a float's bits (-0 just below +0).
__device__ __forceinline__ int32_t seq_key(float f) {
  const int32_t b = __float_as_int(f);
  return b >= 0 ? b : b ^ 0x7FFFFFFF;
}
__device__ __forceinline__ float seq_unkey(int32_t k) {
  return __int_as_float(k >= 0 ? k : k ^ 0x7FFFFFFF);
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, 0xF, 0xF, true);
  const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, 0xF, 0xF, true);
  return __hiloint2double(hi, lo);
}

// Sum over groups of W consecutive lanes (W = 4 .. 64, a power of two);
// every lane of a group gets its group's total.
template <int W>
__device__ __forceinline__ double group_sum_f64(double v) {
  v += dpp_f64<0xB1>(v);                 // quad_perm [1,0,3,2]
  v += dpp_f64<0x4E>(v);                 // quad_perm [2,3,0,1]
  if (W >= 8) v += dpp_f64<0x141>(v);    // row_half_mirror
  if (W >= 16) v += dpp_f64<0x140>(v);   // row_mirror
  if (W >= 32) v += __shfl_xor(v, 16, 64);
  if (W >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Every thread of the block (NT threads: 32 to 512, a power of two) must
// call this; p (LDS) holds the n values; returns s to every thread.
// group_seq_sum: the same over a group of NT threads (whole waves; gtid in
// [0, NT) its thread number) when the block runs several groups side by
// side, each on its own values and scratch; every thread of the block calls
// it (block barriers inside).
template <int NT>
__device__ __forceinline__ float group_seq_sum(const float* p, int n, SeqSumScratch& sc, int gtid) {
  constexpr int S = kSeqSegs, C = NT / S, CPT = kSeqCands / C;
  static_assert(C >= 4 && C <= 64 && (C & (C - 1)) == 0 && CPT >= 1 && C * CPT == kSeqCands,
                "threads per segment");
  static_assert(NT % kWave == 0, "whole waves");
  const int tid = gtid, j = tid / C, i = tid % C;
  const int L = ((n + S - 1) / S + 3) & ~3;   // segments start on float4 boundaries
  const int k0 = min(n, j * L), k1 = min(n, k0 + L);
  const float4* p4 = reinterpret_cast<const float4*>(p);   // p is 16-byte aligned
  // 1. segment sums in double (the C threads of a segment are adjacent
  // lanes; any order: this is an estimate)
  double d = 0.0;
  {
    const int f1 = k0 / 4 + (k1 - k0) / 4;   // whole float4 of the segment
#pragma unroll 2
    for (int f = k0 / 4 + i; f < f1; f += C) {
      const float4 v = p4[f];
      d += ((double)v.x + (double)v.y) + ((double)v.z + (double)v.w);
    }
    if (4 * f1 + i < k1) d += (double)p[4 * f1 + i];
  }
  d = group_sum_f64<C>(d);
  if (i == 0) sc.part[j] = d;
  __syncthreads();
  // 2.-3. the start estimate of segment j and this thread's candidates
  float c[CPT];
  if (j > 0) {
    double est = 0.0;
#pragma unroll
    for (int q = 0; q < S - 1; ++q)
      if (q < j) est += sc.part[q];
    // candidate c = i * CPT + u has key base + c (keys wrap as uint32)
    const uint32_t base = (uint32_t)seq_key((float)est) - (uint32_t)(kSeqCands / 2);
    if (i == 0) sc.base[j] = base;
#pragma unroll
    for (int u = 0; u < CPT; ++u) c[u] = seq_unkey((int32_t)(base + (uint32_t)(i * CPT + u)));
  } else {
#pragma unroll
    for (int u = 0; u < CPT; ++u) c[u] = 0.0f;   // segment 0 starts at +0
  }
  // 4. the segment's chains from the candidates (independent, interleaved)
  float acc[CPT];
#pragma unroll
  for (int u = 0; u < CPT; ++u) acc[u] = c[u];
  {
    // 16 float4 read ahead of their 64 x CPT adds; the chains take turns
    // value by value
    int k = k0;
    for (; k + 64 <= k1; k += 64) {
      float4 v[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) v[r] = p4[k / 4 + r];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int u = 0; u < CPT; ++u) acc[u] = acc[u] + v[r].x;
#pragma unroll
        for (int u = 0; u < CPT; ++u) acc[u] = acc[u] + v[r].y;
#pragma unroll
        for (int u = 0; u < CPT; ++u) acc[u] = acc[u] + v[r].z;
#pragma unroll
        for (int u = 0; u < CPT; ++u) acc[u] = acc[u] + v[r].w;
      }
    }
    for (; k < k1; ++k) {
      const float v = p[k];
#pragma unroll
      for (int u = 0; u < CPT; ++u) acc[u] = acc[u] + v;
    }
  }
#pragma unroll
  for (int u = 0; u < CPT; ++u) sc.out[j][i * CPT + u] = acc[u];
  __syncthreads();
  // 5. stitch the segments in order (wave 0, lane l <-> candidate l; all
  // outputs read up front).  Segment 0's chains all start at +0.  A true
  // start t is candidate key(t) - base of its segment when that index is
  // below kSeqCands (key is a bijection, candidates are consecutive keys):
  // one subtraction and a readlane per segment, no search.
  if (tid < 64) {
    const int lane = tid;
    uint32_t bs[S];
    float ob[S];
#pragma unroll
    for (int q = 0; q < S; ++q) {
      bs[q] = sc.base[q];
      ob[q] = sc.out[q][lane];
    }
    float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ob[0]), 0));
#pragma unroll
    for (int q = 1; q < S; ++q) {
      const uint32_t idx = (uint32_t)seq_key(t) - bs[q];
      if (idx < (uint32_t)kSeqCands) {
        t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ob[q]), (int)idx));
      } else {
        const int q0 = min(n, q * L), q1 = min(n, q0 + L);
        int k = q0;
        if (q1 - q0 >= 4) {
          t = chain_sum(t, p + q0, (q1 - q0) / 4);
          k = q0 + (q1 - q0) / 4 * 4;
        }
        for (; k < q1; ++k) t = t + p[k];
      }
    }
    if (lane == 0) sc.result = t;
  }
  __syncthreads();
  return sc.result;
}

template <int NT>
__device__ __forceinline__ float block_seq_sum(const float* p, int n, SeqSumScratch& sc) {
  return group_seq_sum<NT>(p, n, sc, (int)threadIdx.x);
}

// test_model_trace.c:233 then :500: h = (g / (1 + expf(-g))) * u
__device__ __forceinline__ float silu_mul_t(float g, float u, const uint64_t* tab) {
  const float den = 1.0f + expf_glibc_t(-g, tab);
  const float sg = g / den;
  return sg * u;
}
__device__ __forceinline__ float silu_mul(float g, float u) { return silu_mul_t(g, u, kExp2Tab); }

}  // namespace moe
