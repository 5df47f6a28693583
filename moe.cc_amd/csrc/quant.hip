// quant.hip - device-side synthetic weights and the exporter's rowwise
// quantizers (export.py:23-36), for building large expert pools in HBM.
//
//   moe_fill_normal_dev   counter-based N(mean, std^2) fp32 (synthetic data)
//   moe_quantize_rows_dev Q8: s = max(amax, 1e-8) / 127, q = rne(w / s)
//                         Q4: s = max(amax, 1e-8) / 7,  q = clamp(rne(w/s), -8, 7) + 8,
//                             byte j = q[2j] | q[2j+1] << 4
// One wave per row: amax by a wave max-reduction, then the row is written with
// the same IEEE division and round-half-even as torch's fp32 ops.
#include "moe_device.h"
#include "moe_internal.h"
#include "moe_lib.h"

namespace moe {
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(float* __restrict__ out, size_t n, uint64_t seed, float mean,
                                   float stdv) {
  const size_t pairs = (n + 1) / 2;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs;
       i += (size_t)gridDim.x * blockDim.x) {
    const uint64_t a = mix64(seed + 0x9E3779B97F4A7C15ull * (2 * i + 1));
    const uint64_t b = mix64(seed + 0x9E3779B97F4A7C15ull * (2 * i + 2));
    const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(b >> 11) * 0x1.0p-53;
    const double rad = sqrt(-2.0 * log(u1));
    const double ang = 6.283185307179586 * u2;
    out[2 * i] = (float)((double)mean + (double)stdv * rad * cos(ang));
    if (2 * i + 1 < n) out[2 * i + 1] = (float)((double)mean + (double)stdv * rad * sin(ang));
  }
}

template <bool Q4>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ W, long long N,
                                                           int K, uint8_t* __restrict__ q,
                                                           float* __restrict__ s) {
  const long long row = (long long)blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= N) return;
  const float* w = W + (size_t)row * K;
  float amax = 0.0f;
  for (int k = lane; k < K; k += kWave) amax = fmaxf(amax, fabsf(w[k]));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if (amax < 1e-8f) amax = 1e-8f;
  const float sc = amax / (Q4 ? 7.0f : 127.0f);
  if (lane == 0) s[row] = sc;
  if constexpr (!Q4) {
    int8_t* qr = reinterpret_cast<int8_t*>(q) + (size_t)row * K;
    for (int k = lane; k < K; k += kWave) qr[k] = (int8_t)(int)rintf(w[k] / sc);
  } else {
    uint8_t* qr = q + (size_t)row * (K / 2);
    for (int j = lane; j < K / 2; j += kWave) {
      float r0 = rintf(w[2 * j] / sc), r1 = rintf(w[2 * j + 1] / sc);
      r0 = fminf(fmaxf(r0, -8.0f), 7.0f);
      r1 = fminf(fmaxf(r1, -8.0f), 7.0f);
      const uint32_t lo = (uint32_t)((int)r0 + 8), hi = (uint32_t)((int)r1 + 8);
      qr[j] = (uint8_t)(lo | (hi << 4));
    }
  }
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" {

moe_status moe_fill_normal_dev(float* out, size_t n, uint64_t seed, float mean, float stdv) {
  moe_status st = ensure_init();
  if (st) return st;
  if (n == 0) return MOE_OK;
  if (!out) return set_error(MOE_ERR_ARG, "fill_normal: null pointer");
  const size_t pairs = (n + 1) / 2;
  size_t blocks = (pairs + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, stream(), out, n,
                     seed, mean, stdv);
  return check_hip(hipGetLastError(), "fill_normal launch");
}

moe_status moe_quantize_rows_dev(int dtype, const float* W, long long N, int K, void* q, float* s) {
  moe_status st = ensure_init();
  if (st) return st;
  if (dtype != 2 && dtype != 3) return set_error(MOE_ERR_ARG, "quantize: dtype %d", dtype);
  if (N < 0 || K < 0) return set_error(MOE_ERR_ARG, "quantize: negative shape");
  if (dtype == 3 && (K & 1)) return set_error(MOE_ERR_ARG, "quantize: Q4 needs even K");
  if (N == 0) return MOE_OK;
  if (!W || !q || !s) return set_error(MOE_ERR_ARG, "quantize: null pointer");
  const unsigned blocks = (unsigned)((N + 3) / 4);
  if (dtype == 2)
    hipLaunchKernelGGL(quantize_rows_kernel<false>, dim3(blocks), dim3(256), 0, stream(), W, N, K,
                       (uint8_t*)q, s);
  else
    hipLaunchKernelGGL(quantize_rows_kernel<true>, dim3(blocks), dim3(256), 0, stream(), W, N, K,
                       (uint8_t*)q, s);
  return check_hip(hipGetLastError(), "quantize launch");
}

}  // extern "C"
