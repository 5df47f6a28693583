// pointwise.hip - elementwise ops of the MoE path on device pointers:
//   h = silu(g) * u     (test_model_trace.c:229-236 then :500)
//   y = expf(x)         (glibc-exact, moe_device.h)
#include "moe_device.h"
#include "moe_internal.h"
#include "moe_lib.h"

namespace moe {
namespace {

__global__ void silu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                float* __restrict__ h, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    const float gv = g[i];
    const float den = 1.0f + expf_glibc(-gv);
    const float sg = gv / den;
    h[i] = u ? sg * u[i] : sg;
  }
}

__global__ void expf_kernel(const float* __restrict__ x, float* __restrict__ y, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    y[i] = expf_glibc(x[i]);
}

__global__ void expf_bits_kernel(uint32_t start, float* __restrict__ y, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    y[i] = expf_glibc(__uint_as_float(start + (uint32_t)i));
}

// Every int32 dot through the production epilogue division against the
// IEEE quotient (x / d, correctly rounded under this build's flags); counts
// mismatching bit patterns.  One 64-bit atomic per block.
__global__ __launch_bounds__(256) void qdot_check_kernel(float d, unsigned long long* bad) {
  __shared__ unsigned long long sbad;
  if (threadIdx.x == 0) sbad = 0;
  __syncthreads();
  unsigned long long mine = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < (1ull << 32); i += stride) {
    const float x = (float)(int32_t)(uint32_t)i;
    const float fast = div_int_by_const(x, d);
    const float ieee = x / d;
    mine += __float_as_uint(fast) != __float_as_uint(ieee);
  }
  atomicAdd(&sbad, mine);
  __syncthreads();
  if (threadIdx.x == 0 && sbad) atomicAdd(bad, sbad);
}

unsigned grid_for(size_t n) {
  size_t b = (n + 255) / 256;
  return (unsigned)(b < 65536 ? (b ? b : 1) : 65536);
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" {

moe_status moe_silu_mul_dev(const float* g, const float* u, float* h, size_t n) {
  moe_status st = ensure_init();
  if (st) return st;
  if (n == 0) return MOE_OK;
  if (!g || !h) return set_error(MOE_ERR_ARG, "silu_mul: null pointer");
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(n)), dim3(256), 0, stream(), g, u, h, n);
  return check_hip(hipGetLastError(), "silu_mul launch");
}

moe_status moe_expf_dev(const float* x, float* y, size_t n) {
  moe_status st = ensure_init();
  if (st) return st;
  if (n == 0) return MOE_OK;
  if (!x || !y) return set_error(MOE_ERR_ARG, "expf: null pointer");
  hipLaunchKernelGGL(expf_kernel, dim3(grid_for(n)), dim3(256), 0, stream(), x, y, n);
  return check_hip(hipGetLastError(), "expf launch");
}

moe_status moe_expf_bits_dev(uint32_t start_bits, float* y, size_t n) {
  moe_status st = ensure_init();
  if (st) return st;
  if (n == 0) return MOE_OK;
  if (!y) return set_error(MOE_ERR_ARG, "expf_bits: null pointer");
  hipLaunchKernelGGL(expf_bits_kernel, dim3(grid_for(n)), dim3(256), 0, stream(), start_bits, y, n);
  return check_hip(hipGetLastError(), "expf_bits launch");
}

moe_status moe_selfcheck_qdot_dev(int dtype, unsigned long long* mismatches) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!mismatches) return set_error(MOE_ERR_ARG, "selfcheck_qdot: null pointer");
  if (dtype != 2 && dtype != 3) return set_error(MOE_ERR_ARG, "selfcheck_qdot: dtype %d", dtype);
  unsigned long long* dbad = nullptr;
  if ((st = check_hip(hipMalloc(&dbad, sizeof(*dbad)), "selfcheck alloc"))) return st;
  st = check_hip(hipMemsetAsync(dbad, 0, sizeof(*dbad), stream()), "selfcheck clear");
  if (!st) {
    hipLaunchKernelGGL(qdot_check_kernel, dim3(4096), dim3(256), 0, stream(), dtype == 3 ? 7.0f : 127.0f,
                       dbad);
    st = check_hip(hipGetLastError(), "selfcheck launch");
  }
  if (!st) st = check_hip(hipMemcpyAsync(mismatches, dbad, sizeof(*dbad), hipMemcpyDeviceToHost, stream()),
                          "selfcheck copy");
  if (!st) st = check_hip(hipStreamSynchronize(stream()), "selfcheck sync");
  (void)hipFree(dbad);
  return st;
}

}  // extern "C"
