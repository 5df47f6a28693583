// moe_internal.h - host-side interfaces between the C ABI (capi.cpp) and the
// kernel translation units.  Not installed; the public ABI is include/moehip.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace moe {

// One matrix-times-vectors product of the quantized path:
//   C[m, n] = epilogue(sum_k trunc(A[m, k] * mult) * w[n, k])
// W rows are `rs` bytes apart (int8 values for Q8, nibble pairs for Q4).
struct QJob {
  const uint8_t* W;
  const float* S;
  const float* A;
  float* C;
};

struct QShape {
  int dtype;        // 2 = Q8, 3 = Q4 (the reference's TensorBin dtypes)
  int M, N, K;      // tokens, output rows, logical input length
  int lda, ldc;     // row strides (elements) of A and C
  long long rs;     // weight row stride in bytes
};

// Launches C = A * W^T for `njobs` jobs of one shape.  `jobs_dev` is a device
// array of jobs, or nullptr to use `one` (a single job passed by value).
hipError_t launch_qgemv(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                        hipStream_t stream);

// The two halves of a tiled launch, for callers that pack activations once
// and reuse them: act tables for job j, row m at tabs + (j*M + m)*table bytes
// (shared_tabs: every job uses job 0's).  launch_qgemv_tables requires a
// shape with a tiled geometry (qgemv_tiled_ok).
hipError_t launch_act_pack(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                           uint8_t* tabs, hipStream_t stream);
hipError_t launch_qgemv_tables(const QShape& sh, const QJob* jobs_dev, const QJob& one, int njobs,
                               const uint8_t* tabs, int shared_tabs, hipStream_t stream);
bool qgemv_tiled_ok(const QShape& sh, const void* w_base);
size_t act_table_size(int K);

// fp32 path of matmul_adaptive (kernels.c:153-165): sequential k, one
// rounding per multiply and per add.  W row-major [N][ldw].
hipError_t launch_f32gemv(const float* A, const float* W, float* C, int M, int N, int K,
                          int lda, int ldw, int ldc, hipStream_t stream);

// Read-only stream of bytes / 16 16-byte words at src (16-byte aligned), the
// XOR of all its 32-bit words folded into *sink (the caller zeroes it).
hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream);

// The reads of a batch-1 tiled launch (launch_qgemv_tables' geometry for
// these jobs: weights and scales, no arithmetic), every word XORed into one
// of sink[0..3] (the caller zeroes them).  M must be 1; shapes as launch_qgemv_tables.
// blocks_per_cu: 0 = the GEMV's own cap, else 1..8 blocks a CU (LDS-capped).
hipError_t launch_rows_read(const QShape& sh, const QJob* jobs_dev, int njobs, int blocks_per_cu,
                            uint32_t* sink, hipStream_t stream);

// Zero-fill used for unsupported dtypes (kernels.c:172-179).
hipError_t launch_zero(float* C, size_t n, hipStream_t stream);

// Which kernel variant launch_qgemv picks for a shape (for tests/profiles).
const char* qgemv_variant_name(const QShape& sh, const void* w_base);

}  // namespace moe
