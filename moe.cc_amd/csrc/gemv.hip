// gemv.hip - rowwise Q8 / Q4 matrix-times-vectors kernels for gfx950.
//
// Semantics: kernels.c:51-74 (Q8) and kernels.c:96-128 (Q4), bit for bit.
//   a_k  = (int32)(A[m,k] * 127.0f)        (Q8; 7.0f for Q4), x86 truncation
//   dot  = sum_k a_k * w[n,k]               wrapping int32, any order (exact)
//   C    = ((float)dot / 127.0f) * s[n]     (7.0f for Q4)
//
// Design (decode is HBM-bound; one weight byte feeds one multiply-add):
//   * The truncated activations of the block's tokens are built once per
//     block in LDS as packed signed-int8 "limbs" (a = sum_l b_l 256^l), so the
//     integer dot runs on v_dot4_i32_i8: 1, 2 or 4 dot4 per weight dword
//     depending on the activation range (chosen per block at run time).
//   * Q4 weights are used as unsigned nibbles u = q + 8 in [0, 15]:
//     sum a*(u-8) = sum a*u - 8*sum a; the even/odd nibbles of a dword are
//     split with two masks and meet activations pre-split into even and odd
//     columns.
//   * A lane owns C consecutive dwords of a row per pass (dwordx4 or dwordx3
//     global loads, coalesced across the LPR lanes that share a row), a wave
//     keeps UR rows of loads in flight, and a row's partial sums are reduced
//     across its lanes with cross-lane shuffles.
//   * Shapes whose row bytes are not one of the tiled sizes, unaligned rows
//     and odd-K Q4 go to a plain one-wave-per-row kernel with the same
//     arithmetic.
#include "moe_device.h"
#include "moe_internal.h"

namespace moe {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;

template <int C>
__device__ __forceinline__ void load_chunk(const uint8_t* p, uint32_t* out) {
  if constexpr (C == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else {
    static_assert(C == 3, "chunk of 3 or 4 dwords");
    const uint3 v = *reinterpret_cast<const uint3*>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z;
  }
}

// Builds the limb tables for tokens m0..m0+MT-1 in LDS and returns the number
// of limbs (1, 2 or 4) the block needs.  KD = weight dwords per row.
//   Q8: act[(m*4 + l)*KD + d] packs limb l of a[4d .. 4d+3]
//   Q4: act[(m*4 + l)*KD + d]        packs limb l of a[8d], a[8d+2], a[8d+4], a[8d+6]
//       act[(m*4 + l)*KD + KD/2 + d] packs limb l of a[8d+1], ..., a[8d+7]
//       (here KD counts both halves: KD = 2 * weight dwords per row)
//   asum[m] = sum_k a_k (wrapping), used by the Q4 offset correction.
template <bool Q4, int MT>
__device__ int build_act_lds(const float* __restrict__ A, int lda, int M, int m0, int K, int KD,
                             uint32_t* act, uint32_t* asum) {
  const float mult = Q4 ? 7.0f : 127.0f;
  const int tid = threadIdx.x;
  int need2 = 0, need4 = 0;
  if (tid < MT) asum[tid] = 0;
  __syncthreads();
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const bool valid = (m0 + m) < M;
    const float* a = A + (size_t)(valid ? (m0 + m) : 0) * lda;
    uint32_t* base = act + (size_t)m * 4 * KD;
    if constexpr (!Q4) {
      for (int d = tid; d < KD; d += kBlock) {
        uint32_t b[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int k = 4 * d + i;
          const int32_t v = (valid && k < K) ? f2i_trunc_x86(a[k] * mult) : 0;
          const int nl = limbs_needed(v);
          need2 |= nl >= 2;
          need4 |= nl >= 4;
          split_limbs(v, b[i]);
        }
#pragma unroll
        for (int l = 0; l < 4; ++l) base[l * KD + d] = pack4(b[0][l], b[1][l], b[2][l], b[3][l]);
      }
    } else {
      const int KH = KD / 2;
      uint32_t part = 0;
      for (int d = tid; d < KH; d += kBlock) {
        uint32_t b[8][4];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int k = 8 * d + i;
          const int32_t v = (valid && k < K) ? f2i_trunc_x86(a[k] * mult) : 0;
          const int nl = limbs_needed(v);
          need2 |= nl >= 2;
          need4 |= nl >= 4;
          part += (uint32_t)v;
          split_limbs(v, b[i]);
        }
#pragma unroll
        for (int l = 0; l < 4; ++l) {
          base[l * KD + d] = pack4(b[0][l], b[2][l], b[4][l], b[6][l]);
          base[l * KD + KH + d] = pack4(b[1][l], b[3][l], b[5][l], b[7][l]);
        }
      }
      atomicAdd(&asum[m], part);
    }
  }
  const int any4 = __syncthreads_or(need4);
  const int any2 = __syncthreads_or(need2);
  return any4 ? 4 : (any2 ? 2 : 1);
}

// Tiled body.  Geometry: LPR lanes share a row; a lane loads P chunks of C
// dwords at dword offsets (p*LPR + r)*C of the row; WR = 64/LPR rows per wave
// at once; UR such row groups per wave; the block covers
// kWaves*UR*WR consecutive rows.
template <bool Q4, int C, int P, int LPR, int UR, int MT, int NL>
__device__ __forceinline__ void qgemv_body(const QJob& job, const QShape& sh, int row0, int m0,
                                           const uint32_t* act, const uint32_t* asum, int KD) {
  constexpr int WR = kWave / LPR;
  constexpr int DW = P * C;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int g = lane / LPR, r = lane % LPR;

  uint32_t w[UR][DW];
  int rows[UR];
#pragma unroll
  for (int u = 0; u < UR; ++u) {
    rows[u] = row0 + (wave * UR + u) * WR + g;
    if (rows[u] < sh.N) {
      const uint8_t* wr = job.W + (size_t)rows[u] * (size_t)sh.rs;
#pragma unroll
      for (int p = 0; p < P; ++p) load_chunk<C>(wr + (size_t)((p * LPR + r) * C) * 4, &w[u][p * C]);
    } else {
#pragma unroll
      for (int i = 0; i < DW; ++i) w[u][i] = 0;
    }
  }

  uint32_t dot[UR][MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const uint32_t* am = act + (size_t)m * 4 * KD;
    if constexpr (!Q4) {
      uint32_t av[NL][DW];
#pragma unroll
      for (int l = 0; l < NL; ++l)
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int c = 0; c < C; ++c) av[l][p * C + c] = am[l * KD + (p * LPR + r) * C + c];
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        int32_t acc[NL];
#pragma unroll
        for (int l = 0; l < NL; ++l) {
          acc[l] = 0;
#pragma unroll
          for (int i = 0; i < DW; ++i) acc[l] = dot4(w[u][i], av[l][i], acc[l]);
        }
        dot[u][m] = combine_limbs<NL>(acc);
      }
    } else {
      const int KH = KD / 2;
      uint32_t ev[NL][DW], ov[NL][DW];
#pragma unroll
      for (int l = 0; l < NL; ++l)
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int c = 0; c < C; ++c) {
            const int d = (p * LPR + r) * C + c;
            ev[l][p * C + c] = am[l * KD + d];
            ov[l][p * C + c] = am[l * KD + KH + d];
          }
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        int32_t acc[NL];
#pragma unroll
        for (int l = 0; l < NL; ++l) acc[l] = 0;
#pragma unroll
        for (int i = 0; i < DW; ++i) {
          const uint32_t lo = w[u][i] & 0x0F0F0F0Fu;
          const uint32_t hi = (w[u][i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
          for (int l = 0; l < NL; ++l) {
            acc[l] = dot4(lo, ev[l][i], acc[l]);
            acc[l] = dot4(hi, ov[l][i], acc[l]);
          }
        }
        dot[u][m] = combine_limbs<NL>(acc);
      }
    }
  }

  const float div = Q4 ? 7.0f : 127.0f;
#pragma unroll
  for (int u = 0; u < UR; ++u) {
    float sc = 0.0f;
    if (r == 0 && rows[u] < sh.N) sc = job.S[rows[u]];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      uint32_t v = group_sum_u32<LPR>(dot[u][m]);
      if (Q4) v -= 8u * asum[m];
      if (r == 0 && rows[u] < sh.N && (m0 + m) < sh.M)
        job.C[(size_t)(m0 + m) * sh.ldc + rows[u]] = qdot_epilogue(v, div, sc);
    }
  }
}

template <bool Q4, int C, int P, int LPR, int UR, int MT>
__global__ __launch_bounds__(kBlock) void qgemv_tiled(QShape sh, const QJob* __restrict__ jobs,
                                                      QJob one, int blocks_per_job) {
  extern __shared__ uint32_t smem[];
  constexpr int WR = kWave / LPR;
  constexpr int RB = kWaves * UR * WR;
  const int job_id = blockIdx.x / blocks_per_job;
  const int row0 = (blockIdx.x % blocks_per_job) * RB;
  const QJob job = jobs ? jobs[job_id] : one;
  const int m0 = blockIdx.y * MT;
  const int KD = (LPR * C * P) * (Q4 ? 2 : 1);  // LDS dwords per (token, limb)
  uint32_t* act = smem;
  uint32_t* asum = smem + (size_t)MT * 4 * KD;
  const int nl = build_act_lds<Q4, MT>(job.A, sh.lda, sh.M, m0, sh.K, KD, act, asum);
  if (nl == 1)
    qgemv_body<Q4, C, P, LPR, UR, MT, 1>(job, sh, row0, m0, act, asum, KD);
  else if (nl == 2)
    qgemv_body<Q4, C, P, LPR, UR, MT, 2>(job, sh, row0, m0, act, asum, KD);
  else
    qgemv_body<Q4, C, P, LPR, UR, MT, 4>(job, sh, row0, m0, act, asum, KD);
}

// Any shape: one wave per output row, activations truncated on the fly,
// plain wrapping int32 multiply-add.  Q4 follows the reference's byte
// addressing exactly (row start n*rs, byte k/2, odd-K guard).
template <bool Q4>
__global__ __launch_bounds__(kBlock) void qgemv_generic(QShape sh, const QJob* __restrict__ jobs,
                                                        QJob one, int blocks_per_job) {
  const int job_id = blockIdx.x / blocks_per_job;
  const int row = (blockIdx.x % blocks_per_job) * kWaves + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const QJob job = jobs ? jobs[job_id] : one;
  if (row >= sh.N) return;
  const uint8_t* wr = job.W + (size_t)row * (size_t)sh.rs;
  const float sc = job.S[row];
  for (int m = blockIdx.y; m < sh.M; m += gridDim.y) {
    const float* a = job.A + (size_t)m * sh.lda;
    uint32_t acc = 0;
    if constexpr (!Q4) {
      for (int k = lane; k < sh.K; k += kWave) {
        const int32_t ai = f2i_trunc_x86(a[k] * 127.0f);
        acc += (uint32_t)ai * (uint32_t)(int32_t)(int8_t)wr[k];
      }
    } else {
      for (int j = lane; 2 * j < sh.K; j += kWave) {
        const uint32_t byte = wr[j];
        const int k = 2 * j;
        const int32_t lo = (int32_t)(byte & 0x0Fu) - 8;
        const int32_t hi = (int32_t)((byte >> 4) & 0x0Fu) - 8;
        acc += (uint32_t)f2i_trunc_x86(a[k] * 7.0f) * (uint32_t)lo;
        if (k + 1 < sh.K) acc += (uint32_t)f2i_trunc_x86(a[k + 1] * 7.0f) * (uint32_t)hi;
      }
    }
    acc = group_sum_u32<kWave>(acc);
    if (lane == 0) job.C[(size_t)m * sh.ldc + row] = qdot_epilogue(acc, Q4 ? 7.0f : 127.0f, sc);
  }
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

// ---- host-side variant selection ----
using KernelFn = void (*)(QShape, const QJob*, QJob, int);

struct Variant {
  KernelFn fn;
  int rows_per_block;
  int mt;
  int kd;          // LDS dwords per (token, limb)
  const char* name;
};

template <bool Q4, int C, int P, int LPR, int UR, int MT>
Variant make_variant(const char* name) {
  constexpr int WR = kWave / LPR;
  return Variant{qgemv_tiled<Q4, C, P, LPR, UR, MT>, kWaves * UR * WR, MT,
                 LPR * C * P * (Q4 ? 2 : 1), name};
}

// Row byte counts with a tiled kernel: lanes-per-row x chunk x passes x 4.
template <bool Q4, int MT>
bool pick_tiled(long long rb, Variant* v) {
  switch (rb) {
    case 384:  *v = make_variant<Q4, 3, 1, 32, 2, MT>("tiled_c3p1l32"); return true;
    case 512:  *v = make_variant<Q4, 4, 1, 32, 2, MT>("tiled_c4p1l32"); return true;
    case 768:  *v = make_variant<Q4, 3, 1, 64, 4, MT>("tiled_c3p1l64"); return true;
    case 1024: *v = make_variant<Q4, 4, 1, 64, 4, MT>("tiled_c4p1l64"); return true;
    case 1536: *v = make_variant<Q4, 3, 2, 64, 4, MT>("tiled_c3p2l64"); return true;
    case 2048: *v = make_variant<Q4, 4, 2, 64, 4, MT>("tiled_c4p2l64"); return true;
    case 4096: *v = make_variant<Q4, 4, 4, 64, 2, MT>("tiled_c4p4l64"); return true;
    default: return false;
  }
}

bool select_tiled(const QShape& sh, const void* w_base, Variant* v) {
  const bool q4 = sh.dtype == 3;
  if (q4 && (sh.K & 1)) return false;
  const long long rb = q4 ? sh.K / 2 : sh.K;
  if (sh.rs != rb) return false;
  if (w_base && ((uintptr_t)w_base % 16) != 0) return false;
  if (sh.rs % 16 != 0) return false;
  const int mt = sh.M == 1 ? 1 : 4;
  if (q4) return mt == 1 ? pick_tiled<true, 1>(rb, v) : pick_tiled<true, 4>(rb, v);
  return mt == 1 ? pick_tiled<false, 1>(rb, v) : pick_tiled<false, 4>(rb, v);
}

}  // namespace

const char* qgemv_variant_name(const QShape& sh, const void* w_base) {
  Variant v;
  if (select_tiled(sh, w_base, &v)) return v.name;
  return "generic";
}

hipError_t launch_qgemv(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                        hipStream_t stream) {
  if (sh.M <= 0 || sh.N <= 0 || sh.K <= 0 || njobs <= 0) return hipSuccess;
  if (sh.dtype != 2 && sh.dtype != 3) return hipErrorInvalidValue;
  Variant v;
  // With a device job array the host cannot see the pointers; callers of the
  // batched entry point guarantee 16-byte aligned rows (checked in capi.cpp).
  if (select_tiled(sh, jobs_dev ? nullptr : one.W, &v)) {
    const int bpj = (sh.N + v.rows_per_block - 1) / v.rows_per_block;
    const size_t lds = ((size_t)v.mt * 4 * v.kd + 4) * sizeof(uint32_t);
    dim3 grid((unsigned)((long long)bpj * njobs), (unsigned)((sh.M + v.mt - 1) / v.mt));
    hipLaunchKernelGGL(v.fn, grid, dim3(kBlock), lds, stream, sh, jobs_dev, one, bpj);
  } else {
    const int bpj = (sh.N + kWaves - 1) / kWaves;
    dim3 grid((unsigned)((long long)bpj * njobs), (unsigned)(sh.M < 64 ? sh.M : 64));
    if (sh.dtype == 3)
      hipLaunchKernelGGL(qgemv_generic<true>, grid, dim3(kBlock), 0, stream, sh, jobs_dev, one, bpj);
    else
      hipLaunchKernelGGL(qgemv_generic<false>, grid, dim3(kBlock), 0, stream, sh, jobs_dev, one, bpj);
  }
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

hipError_t launch_zero(float* C, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((n + kBlock - 1) / kBlock);
  hipLaunchKernelGGL(zero_fill, dim3(blocks), dim3(kBlock), 0, stream, C, n);
  return hipGetLastError();
}

}  // namespace moe
