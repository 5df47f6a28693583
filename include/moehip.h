/*
 * moehip.h - C ABI of libmoehip.so, the gfx950 implementation of moe.cc's
 * quantized expert path.
 *
 * Two layers:
 *   1. The drop-in: matmul_adaptive() with the exact signature of the
 *      reference (kernels.h:16-17) and the QuantizedWeight layout of
 *      model.h:26-31.  A program built against the reference's kernels.o
 *      links against this library unchanged; it takes host pointers and is
 *      synchronous, like the reference.
 *   2. A device-resident API (moe_*) on plain device pointers: GEMVs, the
 *      MoE block of one layer (test_model_trace.c:460-517) and the
 *      weight upload from the reference's QwenLayerWeights (model.h:34-58).
 *
 * All moe_* functions return 0 on success and a nonzero moe_status on
 * failure, with a message in moe_last_error().  Device work is queued on the
 * library's stream (moe_get_stream) and is asynchronous unless stated.
 * No torch types appear anywhere in this interface.
 */
#ifndef MOEHIP_H
#define MOEHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference-compatible types (layouts identical to model.h) ---- */
#ifndef QUANTIZED_WEIGHT_DEFINED
/* model.h:26-31.  dtype 2 = Q8 (int8 [rows x cols]); 3 = Q4 (uint8
 * [rows x cols/2], low nibble = even column, value = q + 8). */
typedef struct {
  const int8_t* q;
  const float* s;
  int rows, cols;
  int dtype;
} QuantizedWeight;
#define QUANTIZED_WEIGHT_DEFINED
#endif

#ifndef MOEHIP_NO_MODEL_TYPES
/* model.h:9-23 */
typedef struct {
  int d_model;
  int n_layers;
  int head_dim;
  int n_q;
  int n_kv;
  int d_ff;
  int n_experts;
  int top_k;
  int vocab_size;
  int causal;
  float rope_theta;
  float rms_eps;
} QwenConfig;

/* model.h:34-58 */
typedef struct {
  const float* Wq; const float* bq;
  const float* Wk; const float* bk;
  const float* Wv; const float* bv;
  const float* Wo; const float* bo;
  const float* q_norm;
  const float* k_norm;
  const float* rms1_w;
  const float* rms2_w;
  const float* router_w;
  const float* router_b;
  const float** Wg; const float** bg;
  const float** Wu; const float** bu;
  const float** Wd; const float** bd;
  QuantizedWeight* Wg_q;
  QuantizedWeight* Wu_q;
  QuantizedWeight* Wd_q;
  int experts_quantized;
} QwenLayerWeights;

/* model.h:60-69; lm_head NULL = tied to tok_emb */
typedef struct {
  const float* tok_emb;
  const float* final_norm_w;
  const float* lm_head;
  QwenLayerWeights* layers;
} QwenWeights;
#endif

/* ==== 1. drop-in ==================================================== */

/* Replaces kernels.c:149-181 (declared at kernels.h:16-17).
 *   W_q_ptr == NULL : C = A * W_fp32^T, fp32, k ascending (kernels.c:153-165)
 *   dtype 2 / 3     : rowwise Q8 / Q4 (kernels.c:51-74 / 96-128)
 *   other dtype     : C is zero-filled (kernels.c:172-179)
 * A [M x K], W [N x K] (Q4: N x K/2 bytes, rows K/2 bytes apart), C [M x N],
 * all host memory.  Results are bit-identical to the reference.  Weights are
 * uploaded on first use and cached by (host address, size); by default each
 * call re-hashes the host bytes and re-uploads them if they changed, so freed
 * and reused host memory is safe.  moe_weight_cache_mode(1), or the
 * environment variable MOEHIP_WEIGHT_CACHE_TRUST=1 read at initialisation,
 * skips the hash for callers whose weights never change (the reference's
 * loader).  Errors
 * from the GPU runtime abort the process with a message: there is no CPU
 * fallback. */
void matmul_adaptive(const float* A, const float* W_fp32, const void* W_q_ptr,
                     float* C, int M, int N, int K);

/* ==== 2. device-resident API ======================================== */

typedef int moe_status;
enum {
  MOE_OK = 0,
  MOE_ERR_HIP = 1,        /* a HIP runtime call failed */
  MOE_ERR_ARG = 2,        /* invalid argument (shape, pointer, dtype) */
  MOE_ERR_NOMEM = 3,
  MOE_ERR_UNSUPPORTED = 4
};

/* Initialises the library on `device` (creates its stream).  Called lazily
 * with device 0 by every entry point if not called first. */
moe_status moe_init(int device);
/* Ends the library's use of the GPU (the context destroy of this API): waits
 * for queued work, frees every device buffer the library owns (the weight
 * cache of matmul_adaptive, its staging buffers, the shared forward scratch)
 * and destroys the stream.  Layers and models belong to the caller and must
 * be destroyed first: while any is alive it returns MOE_ERR_ARG and frees
 * nothing.  A later call of any entry point initialises the library again
 * (moe_init, or device 0 lazily).  The no-allocation entry point's
 * file-scope array is not freed (it lives as long as the process).  No
 * reference counterpart: the reference runs on the host and frees its
 * buffers at exit (test_model_trace.c:763-769). */
moe_status moe_shutdown(void);
const char* moe_last_error(void);
const char* moe_version(void);
/* hipStream_t the library queues work on */
void* moe_get_stream(void);
moe_status moe_synchronize(void);
/* drops every cached upload made by matmul_adaptive */
moe_status moe_weight_cache_clear(void);
/* 0 (default): verify cached weights by content on every call;
 * 1: trust that a host address keeps its bytes (no hashing) */
moe_status moe_weight_cache_mode(int trust_addresses);

moe_status moe_malloc(void** dptr, size_t bytes);
moe_status moe_free(void* dptr);
/* synchronous copies (hipMemcpy on the library stream, then wait) */
moe_status moe_memcpy_h2d(void* dst, const void* src, size_t bytes);
moe_status moe_memcpy_d2h(void* dst, const void* src, size_t bytes);
moe_status moe_memcpy_d2d(void* dst, const void* src, size_t bytes);
moe_status moe_memset(void* dptr, int value, size_t bytes);

/* Events on the library stream, for timing (milliseconds). */
moe_status moe_event_create(void** ev);
moe_status moe_event_record(void* ev);
moe_status moe_event_elapsed_ms(void* start, void* stop, float* ms);
moe_status moe_event_destroy(void* ev);

/* kernels.c:51-74 on device pointers: C[M x N] = Q8(A[M x K], Wq[N x K], s[N]) */
moe_status moe_matmul_q8_dev(const float* A, const int8_t* Wq, const float* s, float* C,
                             int M, int N, int K);
/* kernels.c:96-128 on device pointers; Wq rows are K/2 bytes apart */
moe_status moe_matmul_q4_dev(const float* A, const uint8_t* Wq, const float* s, float* C,
                             int M, int N, int K);
/* kernels.c:153-165 on device pointers: fp32, k ascending, unfused */
moe_status moe_matmul_f32_dev(const float* A, const float* W, float* C, int M, int N, int K);
/* kernels.c:149-181 with W_q->q / W_q->s (and W_fp32) device pointers;
 * W_q itself is a host struct */
moe_status moe_matmul_adaptive_dev(const float* A, const float* W_fp32,
                                   const QuantizedWeight* W_q, float* C, int M, int N, int K);

/* Many independent products of one shape in one launch (the expert-GEMV
 * building block).  jobs_dev: device array of njobs moe_qjob; every W must be
 * 16-byte aligned with rows packed (K bytes for Q8, K/2 for Q4). */
typedef struct {
  const void* W;
  const float* S;
  const float* A;
  float* C;
} moe_qjob;
moe_status moe_matmul_q_batched_dev(int dtype, const moe_qjob* jobs_dev, int njobs,
                                    int M, int N, int K);

/* The two halves of moe_matmul_q_batched_dev, for callers that reuse one set
 * of activations across many products (gate and up of every expert read the
 * same x).  moe_act_pack_dev is the activation quantization of
 * kernels.c:56-60 (Q8) / kernels.c:107-110 (Q4) for M rows of A [M x K],
 * written as M packed tables of moe_act_table_bytes(K) bytes each into tabs
 * (16-byte aligned).  moe_matmul_q_prepacked_dev then runs the products of
 * kernels.c:62-72 / :112-126 from those tables; every job's A must be the
 * array the tables were packed from (rows whose quantized activations need
 * four bytes fall back to reading it).  Shapes whose row bytes (K or K/2)
 * are not one of the tiled widths 192..4096 return MOE_ERR_ARG. */
size_t moe_act_table_bytes(int K);
moe_status moe_act_pack_dev(int dtype, const float* A, int M, int K, void* tabs);
/* Measurement helper, no counterpart in the reference: reads `bytes` (a
 * multiple of 16) at src (16-byte aligned) once with 16-byte nontemporal
 * loads on the library stream and XORs every 32-bit word into *sink (device
 * memory, zeroed by the caller).  Its rate over a pool that no cache holds is
 * the plain read stream reported beside the GEMV roofline (on MI355X the HBM
 * read rate depends on the data and the access order: a constant buffer
 * streams faster than quantized weights, which the GEMV itself reads faster
 * than this stream). */
moe_status moe_stream_read_dev(const void* src, size_t bytes, uint32_t* sink);
moe_status moe_matmul_q_prepacked_dev(int dtype, const moe_qjob* jobs_dev, int njobs,
                                      int M, int N, int K, const void* tabs);
/* Measurement helper, no counterpart in the reference: the reads of
 * moe_matmul_q_prepacked_dev at M = 1 for the same jobs -- the same blocks,
 * rows per block, lanes per row and loads in flight, every weight row and
 * scale read once -- with no arithmetic.  blocks_per_cu 0 keeps the GEMV's
 * own cap on resident blocks a CU; 1..8 caps them at that many instead
 * (reads without arithmetic between them may stream best at another
 * occupancy).  Each 32-bit word is
 * XORed into one of sink[0..3] (16 bytes of device memory, zeroed by the
 * caller; the XOR of the four is the XOR of every word read; A, C and the
 * tables are not touched).  Its rate is the read ceiling of the GEMV's own
 * access order on the same matrices. */
moe_status moe_rows_read_dev(int dtype, const moe_qjob* jobs_dev, int njobs, int N, int K,
                             int blocks_per_cu, uint32_t* sink);

/* test_model_trace.c:229-236 and :500 on device arrays of n floats:
 * h = (g / (1 + expf(-g))) * u  (u may be NULL: h = silu(g)).  expf is
 * bit-identical to the host glibc expf, so h matches the reference exactly. */
moe_status moe_silu_mul_dev(const float* g, const float* u, float* h, size_t n);
/* y = expf(x), bit-identical to glibc expf (test_model_trace.c:233, :485). */
moe_status moe_expf_dev(const float* x, float* y, size_t n);
/* Verification hook: y[i] = expf(bits_as_float(start_bits + i)), so that all
 * 2^32 inputs can be checked against the host libm without uploading them. */
moe_status moe_expf_bits_dev(uint32_t start_bits, float* y, size_t n);
/* Verification hook: the epilogue division of every int32 dot by 127.0f
 * (dtype 2) or 7.0f (dtype 3) as the kernels compute it (kernels.c:71,
 * :125), compared with the IEEE quotient on all 2^32 inputs; writes the
 * number of mismatching results (0 expected) to *mismatches (host). */
moe_status moe_selfcheck_qdot_dev(int dtype, unsigned long long* mismatches);

/* Synthetic data: out[i] ~ N(mean, std^2), counter-based (seed, i) -> value. */
moe_status moe_fill_normal_dev(float* out, size_t n, uint64_t seed, float mean, float stdv);
/* export.py:23-36 rowwise quantization on device.  W fp32 [N x K];
 * dtype 2: q int8 [N x K], s = max(amax,1e-8)/127, q = round-half-even(w/s);
 * dtype 3: q uint8 [N x K/2], s = max(amax,1e-8)/7, q = clamp(rne(w/s),-8,7)+8,
 *          low nibble = even column.  Bit-identical to the exporter's fp32 ops. */
moe_status moe_quantize_rows_dev(int dtype, const float* W, long long N, int K, void* q, float* s);

/* ---- the MoE block of one layer (test_model_trace.c:460-517) ---- */
typedef struct moe_layer moe_layer;

/* Uploads one layer from the reference's structures (model.h:9-58, bound by
 * load_all_weights model.h:220-305): router_w/router_b, rms2_w and the E
 * quantized gate/up/down experts.  Host pointers; copied. */
moe_status moe_layer_create(const QwenConfig* cfg, const QwenLayerWeights* lw, moe_layer** out);
/* Same from contiguous arrays: router_w [E x D], router_b [E] or NULL,
 * rms2_w [D] or NULL, gq/uq [E x d_ff x rb_g] bytes (rb_g = D for Q8, D/2
 * for Q4), gs/us [E x d_ff], dq [E x D x rb_d] (rb_d = d_ff or d_ff/2),
 * ds [E x D].  src_on_device: the arrays are device pointers (copied). */
moe_status moe_layer_create_raw(int dtype, int D, int d_ff, int E, int top_k,
                                const float* router_w, const float* router_b, const float* rms2_w,
                                const void* gq, const float* gs, const void* uq, const float* us,
                                const void* dq, const float* ds, int src_on_device,
                                moe_layer** out);
moe_status moe_layer_destroy(moe_layer* layer);
/* Forwards of at least min_tokens tokens run expert-major (every routed
 * expert's rows read once for all its tokens, int8 MFMA tiles); fewer
 * tokens run the per-(token, rank) decode kernels.  0 = library default
 * (env MOEHIP_GROUPED_MIN_T, else 32).  Both give identical results.
 * Expert-major needs D and d_ff multiples of 128 (Q8) or 256 (Q4). */
moe_status moe_layer_set_grouped_min_tokens(moe_layer* layer, int min_tokens);
/* test_model_trace.c:463-517 on device arrays:
 *   out[t] = x_resid[t] + sum_j p[t,j] * down_e(silu(gate_e x) * up_e x),
 *   e = idx[t,j], the top_k experts of logits = x_norm Wr^T (+ b), p their
 *   softmax; x_resid may be NULL (no residual).  x_norm, x_resid, out:
 *   [T x D]; idx_out / p_out ([T x top_k], int32 / fp32) may be NULL.
 *   Bit-identical to the reference on the same inputs. */
moe_status moe_layer_forward(moe_layer* layer, const float* x_norm, const float* x_resid, int T,
                             float* out, int32_t* idx_out, float* p_out);
/* moe_layer_forward that allocates nothing.  It has no counterpart in the
 * reference; it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * bit-identical results; always the per-(token, rank) kernels.
 * Its scratch (logits, selection, packed tables, h) lives in a 4 MiB
 * file-scope device array each GPU holds until the process ends; T is at
 * most 32 tokens and the scratch need at most 4 MiB (about 72 KiB per token
 * at d_model 2048, d_ff 768, 128 experts, top-8), else MOE_ERR_ARG with a
 * message.  The first call on a device looks up the array's address.  All
 * no-allocation calls on one GPU share the array: calls that overlap on one
 * GPU race (the library's own stream serialises its calls). */
moe_status moe_layer_forward_noalloc(moe_layer* layer, const float* x_norm, const float* x_resid,
                                     int T, float* out, int32_t* idx_out, float* p_out);
/* test_model_trace.c:460-517 including norm2: out = x + MoE(rmsnorm(x, rms2_w)) */
moe_status moe_block_forward(moe_layer* layer, const float* x, int T, float* out, float eps);
/* test_model_trace.c:241-255 on device arrays: y = (x / sqrt(mean(x^2)+eps)) * w
 * (w may be NULL), sequential sum of squares as in the reference */
moe_status moe_rmsnorm_dev(const float* x, const float* w, float* y, int T, int D, float eps);
/* Device pointers of the last forward's router logits [T x E], SwiGLU
 * outputs h [T*top_k x d_ff] and expert outputs y [T*top_k x D] (for tests). */
moe_status moe_layer_debug_buffers(moe_layer* layer, const float** logits, const float** h,
                                   const float** y);

/* ---- the whole model (test_model_trace.c:526-579) with a KV cache ---- */
typedef struct moe_model moe_model;

/* Uploads a model from the reference's structures (model.h:9-69, filled by
 * load_all_weights model.h:107-323); host pointers, copied.  Experts must be
 * quantized (Q8 or Q4).  max_seq: KV-cache length (1..16384).  Only causal
 * attention (model.h:161 sets causal = 1). */
moe_status moe_model_create(const QwenConfig* cfg, const QwenWeights* w, int max_seq,
                            moe_model** out);
/* Reads a QW3W file (all_q8.bin / all_q4.bin; io.c:193-285) and infers the
 * config from its tensor shapes as load_all_weights does (model.h:110-163),
 * then moe_model_create.  Replaces bin_load + load_all_weights + the
 * reference's per-call host loops. */
moe_status moe_model_load_file(const char* path, int max_seq, moe_model** out);
/* The host half of moe_model_load_file, with no GPU call: reads a QW3W
 * file's index (io.c:193-285), infers the config as load_all_weights does
 * (model.h:110-163) and checks that every tensor the model binds has the
 * dtype, rank and size that config implies.  cfg (and *expert_dtype, 2 or 3,
 * if not NULL) receive the result.  MOE_ERR_ARG names the first bad tensor. */
moe_status moe_model_inspect_file(const char* path, QwenConfig* cfg, int* expert_dtype);
/* A synthetic model generated on the device: every weight ~ N(0, std^2)
 * (counter-based, seeded), norm weights 1, experts quantized with the
 * exporter's rule (export.py:23-36), no biases; lm_head untied if
 * untied_head.  For benchmarks at the real shape without a checkpoint. */
moe_status moe_model_create_synthetic(const QwenConfig* cfg, int expert_dtype, int untied_head,
                                      uint64_t seed, float stdv, int max_seq, moe_model** out);
moe_status moe_model_destroy(moe_model* m);
moe_status moe_model_config(const moe_model* m, QwenConfig* cfg);
/* Empties the KV cache (next forward starts at position 0). */
moe_status moe_model_reset(moe_model* m);
/* Number of positions in the KV cache. */
int moe_model_position(const moe_model* m);
/* T new tokens at the current position (ids on the device if ids_on_device,
 * else host ids checked against [0, vocab)); K/V appended to the cache.
 * The last row's logits go to logits_dev [vocab] and the next token the
 * reference would pick (first index of the largest softmax_rows probability,
 * test_model_trace.c:735-746) to next_dev [1] (device int32); either may be
 * NULL.  Bit-identical to the reference's last-row logits for the whole
 * sequence so far. */
moe_status moe_model_forward(moe_model* m, const int32_t* ids, int T, int ids_on_device,
                             float* logits_dev, int32_t* next_dev);
/* model_forward_f32 (test_model_trace.c:526-579) semantics: resets the
 * cache, runs ids[0..T) (host), writes the last row's logits to out_last
 * (host, [vocab]), softmaxed (softmax_rows, :260-272) if apply_softmax.
 * Synchronous. */
moe_status moe_model_forward_full(moe_model* m, const int32_t* ids, int T, int apply_softmax,
                                  float* out_last);
/* Greedy decoding on the device: resets the cache, runs the prompt (host
 * ids), then n_new - 1 single-token steps, each fed the previous step's
 * choice from device memory (no host round trip).  out_ids (host, n_new):
 * the choice after the prompt and after every step.  ms_prompt / ms_decode
 * (host, may be NULL): HIP-event time of the prompt and of the n_new - 1
 * decode steps.  Synchronous. */
moe_status moe_model_generate(moe_model* m, const int32_t* prompt, int n_prompt, int n_new,
                              int32_t* out_ids, float* ms_prompt, float* ms_decode);

/* The reference's next-token choice (test_model_trace.c:735-746): softmax_rows
 * of the n logits, then the first index of the largest probability.  Equal
 * probabilities keep the lower index, also for logits that differ but round
 * to the same probability; a NaN or +inf logit, or all -inf, gives 0.
 * Device pointers; next: one int32. */
moe_status moe_greedy_dev(const float* logits, int n, int32_t* next);
/* The head and the choice in one pass, as the decode loop runs them
 * (test_model_trace.c:571, :735-746): logits [N] = W [N x K] . x [K] with the
 * sequential fp32 chains of moe_matmul_f32_dev, then next = moe_greedy_dev's
 * answer, the product's blocks handing their maxima to the choice.  Device
 * pointers; logits may not be NULL. */
moe_status moe_head_greedy_dev(const float* x, const float* W, int N, int K, float* logits,
                               int32_t* next);

/* Name of the kernel variant the GEMV entry points use for a shape. */
const char* moe_gemv_variant(int dtype, int M, int N, int K);

#ifdef __cplusplus
}
#endif
#endif /* MOEHIP_H */
