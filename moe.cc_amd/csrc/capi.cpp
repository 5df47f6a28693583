// capi.cpp - the C ABI of libmoehip.so (declared in include/moehip.h).
//
// Library state: one device, one stream (default priority), a cache of
// weights uploaded by the drop-in matmul_adaptive, a thread-local last-error
// message.  Every entry point is thread-compatible; the cache is guarded by a
// mutex.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/moehip.h"
#include "dense.h"
#include "moe_internal.h"
#include "moe_lib.h"

namespace moe {

namespace {
thread_local std::string g_err;
std::mutex g_mu;
bool g_ready = false;
int g_device = -1;
hipStream_t g_stream = nullptr;

struct CacheKey {
  const void* host;
  size_t bytes;
  bool operator==(const CacheKey& o) const { return host == o.host && bytes == o.bytes; }
};
struct CacheKeyHash {
  size_t operator()(const CacheKey& k) const {
    return std::hash<const void*>()(k.host) ^ (std::hash<size_t>()(k.bytes) * 1315423911u);
  }
};
struct CacheEntry {
  void* dev;
  uint64_t digest;
};
std::unordered_map<CacheKey, CacheEntry, CacheKeyHash> g_cache;
// 0: re-hash the host bytes on every call and re-upload when they changed
//    (safe when callers free and reuse host memory); 1: trust the address.
int g_trust_addresses = 0;

// staging buffers of the drop-in (grown on demand)
void* g_stage_a = nullptr;
size_t g_stage_a_bytes = 0;
void* g_stage_c = nullptr;
size_t g_stage_c_bytes = 0;
}  // namespace

moe_status set_error(moe_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return st;
}

namespace {
std::atomic<int> g_live{0};
}  // namespace

void live_objects(int delta) { g_live.fetch_add(delta); }

moe_status check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return MOE_OK;
  return set_error(MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

moe_status ensure_init() {
  if (g_ready) return MOE_OK;
  return moe_init(0);
}

hipStream_t stream() { return g_stream; }

namespace {

moe_status grow(void** buf, size_t* cap, size_t need) {
  if (need <= *cap) return MOE_OK;
  if (*buf) (void)hipFree(*buf);
  *buf = nullptr;
  *cap = 0;
  moe_status st = check_hip(hipMalloc(buf, need), "hipMalloc(staging)");
  if (st == MOE_OK) *cap = need;
  return st;
}

// 64-bit digest of a host buffer: four interleaved multiply-xorshift lanes
// over 8-byte words, tail bytes folded in one at a time.
uint64_t digest(const void* p, size_t n) {
  const unsigned char* b = (const unsigned char*)p;
  uint64_t h[4] = {0x9E3779B97F4A7C15ull, 0xC2B2AE3D27D4EB4Full, 0x165667B19E3779F9ull,
                   0x27D4EB2F165667C5ull};
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    for (int l = 0; l < 4; ++l) {
      uint64_t w;
      std::memcpy(&w, b + i + 8 * l, 8);
      h[l] = (h[l] ^ w) * 0xFF51AFD7ED558CCDull;
      h[l] ^= h[l] >> 29;
    }
  }
  uint64_t r = h[0] ^ (h[1] * 31) ^ (h[2] * 131) ^ (h[3] * 1313) ^ (uint64_t)n;
  for (; i < n; ++i) r = (r ^ b[i]) * 0x100000001B3ull;
  r ^= r >> 33;
  return r * 0xC4CEB9FE1A85EC53ull;
}

// Device copy of a host weight, uploaded once per (address, size) and
// re-uploaded when its bytes change (unless addresses are trusted).
moe_status cached_upload(const void* host, size_t bytes, const void** dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  CacheKey key{host, bytes};
  const uint64_t dg = g_trust_addresses ? 0 : digest(host, bytes);
  auto it = g_cache.find(key);
  if (it != g_cache.end() && (g_trust_addresses || it->second.digest == dg)) {
    *dev = it->second.dev;
    return MOE_OK;
  }
  void* d = nullptr;
  moe_status st = MOE_OK;
  if (it != g_cache.end()) {
    d = it->second.dev;  // same size: refill in place
  } else {
    st = check_hip(hipMalloc(&d, bytes ? bytes : 1), "hipMalloc(weight)");
    if (st) return st;
  }
  st = check_hip(hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, g_stream), "upload weight");
  if (st == MOE_OK) st = check_hip(hipStreamSynchronize(g_stream), "upload weight sync");
  if (st) {
    if (it != g_cache.end()) g_cache.erase(it);
    (void)hipFree(d);
    return st;
  }
  g_cache[key] = CacheEntry{d, dg};
  *dev = d;
  return MOE_OK;
}

[[noreturn]] void die(const char* where) {
  std::fprintf(stderr, "libmoehip: %s failed: %s\n", where, g_err.c_str());
  std::fflush(stderr);
  std::abort();
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" {

moe_status moe_init(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ready) {
    if (device == g_device) return MOE_OK;
    return set_error(MOE_ERR_UNSUPPORTED, "moe_init: already initialised on device %d", g_device);
  }
  int n = 0;
  moe_status st = check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (st) return st;
  if (device < 0 || device >= n)
    return set_error(MOE_ERR_ARG, "moe_init: device %d not present (%d visible)", device, n);
  st = check_hip(hipSetDevice(device), "hipSetDevice");
  if (st) return st;
  st = check_hip(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), "hipStreamCreate");
  if (st) return st;
  // callers that cannot call moe_weight_cache_mode (an unmodified reference
  // build linked against this library) opt in to address trust here
  if (const char* v = std::getenv("MOEHIP_WEIGHT_CACHE_TRUST"))
    if (*v) g_trust_addresses = std::atoi(v) != 0;
  g_device = device;
  g_ready = true;
  return MOE_OK;
}

const char* moe_last_error(void) { return g_err.c_str(); }
const char* moe_version(void) { return "moehip 0.1 (gfx950)"; }

void* moe_get_stream(void) {
  if (ensure_init()) return nullptr;
  return (void*)g_stream;
}

moe_status moe_synchronize(void) {
  moe_status st = ensure_init();
  if (st) return st;
  return check_hip(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
}

moe_status moe_weight_cache_clear(void) {
  moe_status st = ensure_init();
  if (st) return st;
  st = check_hip(hipStreamSynchronize(g_stream), "hipStreamSynchronize");
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& kv : g_cache) (void)hipFree(kv.second.dev);
  g_cache.clear();
  return st;
}

moe_status moe_weight_cache_mode(int trust_addresses) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_trust_addresses = trust_addresses ? 1 : 0;
  return MOE_OK;
}

moe_status moe_malloc(void** dptr, size_t bytes) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!dptr) return set_error(MOE_ERR_ARG, "moe_malloc: null out pointer");
  return check_hip(hipMalloc(dptr, bytes ? bytes : 1), "hipMalloc");
}

moe_status moe_free(void* dptr) {
  moe_status st = ensure_init();
  if (st) return st;
  return check_hip(hipFree(dptr), "hipFree");
}

static moe_status copy_sync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind,
                            const char* what) {
  moe_status st = ensure_init();
  if (st) return st;
  st = check_hip(hipMemcpyAsync(dst, src, bytes, kind, g_stream), what);
  if (st) return st;
  return check_hip(hipStreamSynchronize(g_stream), what);
}

moe_status moe_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyHostToDevice, "memcpy h2d");
}
moe_status moe_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyDeviceToHost, "memcpy d2h");
}
moe_status moe_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  return copy_sync(dst, src, bytes, hipMemcpyDeviceToDevice, "memcpy d2d");
}
moe_status moe_memset(void* dptr, int value, size_t bytes) {
  moe_status st = ensure_init();
  if (st) return st;
  return check_hip(hipMemsetAsync(dptr, value, bytes, g_stream), "hipMemsetAsync");
}

moe_status moe_event_create(void** ev) {
  moe_status st = ensure_init();
  if (st) return st;
  return check_hip(hipEventCreate((hipEvent_t*)ev), "hipEventCreate");
}
moe_status moe_event_record(void* ev) {
  return check_hip(hipEventRecord((hipEvent_t)ev, g_stream), "hipEventRecord");
}
moe_status moe_event_elapsed_ms(void* start, void* stop, float* ms) {
  moe_status st = check_hip(hipEventSynchronize((hipEvent_t)stop), "hipEventSynchronize");
  if (st) return st;
  return check_hip(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop),
                   "hipEventElapsedTime");
}
moe_status moe_event_destroy(void* ev) {
  return check_hip(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
}

static moe_status qgemv_dev(int dtype, const float* A, const void* Wq, const float* s, float* C,
                            int M, int N, int K) {
  moe_status st = ensure_init();
  if (st) return st;
  if (M < 0 || N < 0) return set_error(MOE_ERR_ARG, "matmul: negative M or N");
  if (K < 0) K = 0;  // the reference's loops run zero times: dot = 0
  if (M == 0 || N == 0) return MOE_OK;
  if (!A || !Wq || !s || !C) return set_error(MOE_ERR_ARG, "matmul: null pointer");
  QShape sh;
  sh.dtype = dtype;
  sh.M = M;
  sh.N = N;
  sh.K = K;
  sh.lda = K;
  sh.ldc = N;
  sh.rs = dtype == 3 ? K / 2 : K;
  QJob one{(const uint8_t*)Wq, s, A, C};
  return check_hip(launch_qgemv(sh, nullptr, one, 1, g_stream), "qgemv launch");
}

moe_status moe_matmul_q8_dev(const float* A, const int8_t* Wq, const float* s, float* C, int M,
                             int N, int K) {
  return qgemv_dev(2, A, Wq, s, C, M, N, K);
}

moe_status moe_matmul_q4_dev(const float* A, const uint8_t* Wq, const float* s, float* C, int M,
                             int N, int K) {
  return qgemv_dev(3, A, Wq, s, C, M, N, K);
}

moe_status moe_matmul_f32_dev(const float* A, const float* W, float* C, int M, int N, int K) {
  moe_status st = ensure_init();
  if (st) return st;
  if (M < 0 || N < 0) return set_error(MOE_ERR_ARG, "matmul_f32: negative M or N");
  if (K < 0) K = 0;
  if (M == 0 || N == 0) return MOE_OK;
  if (!A || !W || !C) return set_error(MOE_ERR_ARG, "matmul_f32: null pointer");
  if (K == 0) return check_hip(launch_f32gemv(A, W, C, M, N, K, K, K, N, g_stream), "f32gemv launch");
  DenseArgs a{A, K, W, K, nullptr, nullptr, 0, C, N, M, N, K};
  return dense_matmul(a, g_stream);
}

moe_status moe_greedy_dev(const float* logits, int n, int32_t* next) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!logits || !next) return set_error(MOE_ERR_ARG, "greedy: null pointer");
  return greedy_vec(logits, n, nullptr, 0, next, nullptr, nullptr, g_stream);
}

namespace {
float* g_head_part = nullptr;   // block maxima of moe_head_greedy_dev (grown, never freed)
size_t g_head_part_n = 0;
}  // namespace

moe_status moe_head_greedy_dev(const float* x, const float* W, int N, int K, float* logits,
                               int32_t* next) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!x || !W || !logits || !next) return set_error(MOE_ERR_ARG, "head_greedy: null pointer");
  if (N <= 0 || K <= 0) return set_error(MOE_ERR_ARG, "head_greedy: N = %d, K = %d", N, K);
  DenseArgs a{x, K, W, K, nullptr, nullptr, 0, logits, N, 1, N, K};
  if (!dense_amax_ok(a)) {
    if ((st = dense_matmul(a, g_stream))) return st;
    return greedy_vec(logits, N, nullptr, 0, next, nullptr, nullptr, g_stream);
  }
  const size_t need = (size_t)N / 16 + 1;
  if (need > g_head_part_n) {
    if (g_head_part) {
      if ((st = check_hip(hipStreamSynchronize(g_stream), "head_greedy sync"))) return st;
      (void)hipFree(g_head_part);
      g_head_part = nullptr;
      g_head_part_n = 0;
    }
    if ((st = check_hip(hipMalloc(&g_head_part, need * 4), "head_greedy scratch"))) return st;
    g_head_part_n = need;
  }
  a.amax_part = g_head_part;
  if ((st = dense_matmul(a, g_stream))) return st;
  return greedy_vec(logits, N, g_head_part, dense_amax_rows(N), next, nullptr, nullptr, g_stream);
}

moe_status moe_matmul_adaptive_dev(const float* A, const float* W_fp32, const QuantizedWeight* W_q,
                                   float* C, int M, int N, int K) {
  if (!W_q) return moe_matmul_f32_dev(A, W_fp32, C, M, N, K);
  if (W_q->dtype == 2) return qgemv_dev(2, A, W_q->q, W_q->s, C, M, N, K);
  if (W_q->dtype == 3) return qgemv_dev(3, A, W_q->q, W_q->s, C, M, N, K);
  moe_status st = ensure_init();
  if (st) return st;
  if (M <= 0 || N <= 0) return MOE_OK;
  return check_hip(launch_zero(C, (size_t)M * (size_t)N, g_stream), "zero fill");
}

moe_status moe_matmul_q_batched_dev(int dtype, const moe_qjob* jobs_dev, int njobs, int M, int N,
                                    int K) {
  moe_status st = ensure_init();
  if (st) return st;
  if (dtype != 2 && dtype != 3) return set_error(MOE_ERR_ARG, "batched: dtype %d", dtype);
  if (M < 0 || N < 0 || K < 0 || njobs < 0) return set_error(MOE_ERR_ARG, "batched: bad shape");
  if (dtype == 3 && (K & 1)) return set_error(MOE_ERR_ARG, "batched: Q4 needs even K");
  const long long rb = dtype == 3 ? K / 2 : K;
  if (rb % 16 != 0) return set_error(MOE_ERR_ARG, "batched: row bytes must be a multiple of 16");
  if (njobs == 0 || M == 0 || N == 0) return MOE_OK;
  QShape sh;
  sh.dtype = dtype;
  sh.M = M;
  sh.N = N;
  sh.K = K;
  sh.lda = K;
  sh.ldc = N;
  sh.rs = rb;
  static_assert(sizeof(moe_qjob) == sizeof(QJob), "job layout");
  QJob none{nullptr, nullptr, nullptr, nullptr};
  return check_hip(launch_qgemv(sh, (const QJob*)jobs_dev, none, njobs, g_stream),
                   "batched qgemv launch");
}

size_t moe_act_table_bytes(int K) { return K < 0 ? 0 : act_table_size(K); }

static moe_status prepacked_shape(int dtype, int M, int N, int K, const char* who, QShape* sh) {
  if (dtype != 2 && dtype != 3) return set_error(MOE_ERR_ARG, "%s: dtype %d", who, dtype);
  if (M < 0 || N < 0 || K <= 0) return set_error(MOE_ERR_ARG, "%s: bad shape", who);
  if (dtype == 3 && (K & 1)) return set_error(MOE_ERR_ARG, "%s: Q4 needs even K", who);
  sh->dtype = dtype;
  sh->M = M;
  sh->N = N;
  sh->K = K;
  sh->lda = K;
  sh->ldc = N;
  sh->rs = dtype == 3 ? K / 2 : K;
  if (!qgemv_tiled_ok(*sh, nullptr))
    return set_error(MOE_ERR_ARG, "%s: no tiled geometry for %lld-byte rows", who, sh->rs);
  return MOE_OK;
}

moe_status moe_stream_read_dev(const void* src, size_t bytes, uint32_t* sink) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!src || !sink) return set_error(MOE_ERR_ARG, "stream_read: null pointer");
  if (((uintptr_t)src % 16) != 0 || bytes % 16 != 0 || ((uintptr_t)sink % 4) != 0)
    return set_error(MOE_ERR_ARG, "stream_read: src and bytes must be multiples of 16");
  return check_hip(launch_stream_read(src, bytes, sink, g_stream), "stream_read launch");
}

moe_status moe_act_pack_dev(int dtype, const float* A, int M, int K, void* tabs) {
  moe_status st = ensure_init();
  if (st) return st;
  QShape sh;
  st = prepacked_shape(dtype, M, 1, K, "act_pack", &sh);
  if (st) return st;
  if (((uintptr_t)tabs % 16) != 0) return set_error(MOE_ERR_ARG, "act_pack: tabs not 16-byte aligned");
  if (M == 0) return MOE_OK;
  QJob one{nullptr, nullptr, A, nullptr};
  return check_hip(launch_act_pack(sh, nullptr, one, 1, (uint8_t*)tabs, g_stream), "act_pack launch");
}

moe_status moe_matmul_q_prepacked_dev(int dtype, const moe_qjob* jobs_dev, int njobs, int M, int N,
                                      int K, const void* tabs) {
  moe_status st = ensure_init();
  if (st) return st;
  QShape sh;
  st = prepacked_shape(dtype, M, N, K, "prepacked", &sh);
  if (st) return st;
  if (njobs < 0) return set_error(MOE_ERR_ARG, "prepacked: njobs %d", njobs);
  if (((uintptr_t)tabs % 16) != 0) return set_error(MOE_ERR_ARG, "prepacked: tabs not 16-byte aligned");
  if (njobs == 0 || M == 0 || N == 0) return MOE_OK;
  QJob none{nullptr, nullptr, nullptr, nullptr};
  return check_hip(launch_qgemv_tables(sh, (const QJob*)jobs_dev, none, njobs, (const uint8_t*)tabs,
                                       1, g_stream),
                   "prepacked qgemv launch");
}

moe_status moe_rows_read_dev(int dtype, const moe_qjob* jobs_dev, int njobs, int N, int K,
                             int blocks_per_cu, uint32_t* sink) {
  moe_status st = ensure_init();
  if (st) return st;
  QShape sh;
  st = prepacked_shape(dtype, 1, N, K, "rows_read", &sh);
  if (st) return st;
  if (njobs < 0) return set_error(MOE_ERR_ARG, "rows_read: njobs %d", njobs);
  if (!sink) return set_error(MOE_ERR_ARG, "rows_read: null sink");
  if (blocks_per_cu < 0 || blocks_per_cu > 8)
    return set_error(MOE_ERR_ARG, "rows_read: blocks_per_cu %d (0..8)", blocks_per_cu);
  if (njobs == 0 || N == 0) return MOE_OK;
  return check_hip(launch_rows_read(sh, (const QJob*)jobs_dev, njobs, blocks_per_cu, sink, g_stream),
                   "rows_read launch");
}

const char* moe_gemv_variant(int dtype, int M, int N, int K) {
  QShape sh;
  sh.dtype = dtype;
  sh.M = M;
  sh.N = N;
  sh.K = K;
  sh.lda = K;
  sh.ldc = N;
  sh.rs = dtype == 3 ? K / 2 : K;
  return qgemv_variant_name(sh, nullptr);
}

void matmul_adaptive(const float* A, const float* W_fp32, const void* W_q_ptr, float* C, int M,
                     int N, int K) {
  if (ensure_init()) die("matmul_adaptive init");
  if (M <= 0 || N <= 0) return;
  if (K < 0) K = 0;
  const QuantizedWeight* wq = (const QuantizedWeight*)W_q_ptr;
  const size_t a_bytes = (size_t)M * (size_t)K * sizeof(float);
  const size_t c_bytes = (size_t)M * (size_t)N * sizeof(float);
  if (grow(&g_stage_c, &g_stage_c_bytes, c_bytes)) die("matmul_adaptive staging");
  float* dC = (float*)g_stage_c;
  moe_status st = MOE_OK;
  if (wq && wq->dtype != 2 && wq->dtype != 3) {
    st = check_hip(launch_zero(dC, (size_t)M * (size_t)N, g_stream), "zero fill");
  } else {
    if (grow(&g_stage_a, &g_stage_a_bytes, a_bytes)) die("matmul_adaptive staging");
    float* dA = (float*)g_stage_a;
    if (a_bytes)
      st = check_hip(hipMemcpyAsync(dA, A, a_bytes, hipMemcpyHostToDevice, g_stream), "upload A");
    if (st) die("matmul_adaptive");
    if (!wq) {
      const void* dW = nullptr;
      st = cached_upload(W_fp32, (size_t)N * (size_t)K * sizeof(float), &dW);
      if (!st) st = moe_matmul_f32_dev(dA, (const float*)dW, dC, M, N, K);
    } else {
      // Q4 rows are K/2 bytes apart but a row reads ceil(K/2) bytes
      // (kernels.c:103,108), so an odd K reads one byte past N*(K/2).
      const size_t q_bytes = wq->dtype == 2 ? (size_t)N * (size_t)K
                                            : (size_t)N * (size_t)(K / 2) + (size_t)(K & 1);
      const void* dq = nullptr;
      const void* ds = nullptr;
      st = cached_upload(wq->q, q_bytes, &dq);
      if (!st) st = cached_upload(wq->s, (size_t)N * sizeof(float), &ds);
      if (!st) st = qgemv_dev(wq->dtype, dA, dq, (const float*)ds, dC, M, N, K);
    }
  }
  if (st) die("matmul_adaptive");
  st = check_hip(hipMemcpyAsync(C, dC, c_bytes, hipMemcpyDeviceToHost, g_stream), "download C");
  if (!st) st = check_hip(hipStreamSynchronize(g_stream), "matmul_adaptive sync");
  if (st) die("matmul_adaptive");
}

moe_status moe_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ready) return MOE_OK;
  const int live = g_live.load();
  if (live)
    return set_error(MOE_ERR_ARG, "moe_shutdown: %d layer(s) or model(s) still alive; destroy them first",
                     live);
  moe_status st = check_hip(hipStreamSynchronize(g_stream), "moe_shutdown: sync");
  for (auto& kv : g_cache) (void)hipFree(kv.second.dev);
  g_cache.clear();
  for (void** b : {&g_stage_a, &g_stage_c, reinterpret_cast<void**>(&g_head_part)})
    if (*b) (void)hipFree(*b);
  g_stage_a = g_stage_c = nullptr;
  g_head_part = nullptr;
  g_stage_a_bytes = g_stage_c_bytes = g_head_part_n = 0;
  release_gemv_workspace();
  release_layer_scratch();
  const moe_status sd = check_hip(hipStreamDestroy(g_stream), "moe_shutdown: hipStreamDestroy");
  g_stream = nullptr;
  g_ready = false;
  g_device = -1;
  return st ? st : sd;
}

}  // extern "C"
