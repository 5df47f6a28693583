/*
 * moe_caller.c - a plain C program that uses libmoehip.so the way the
 * reference's test_model_trace.c uses kernels.o and model.h: QuantizedWeight
 * arrays per expert (model.h:26-31, bound as model.h:228-305 binds them),
 * matmul_adaptive calls with host pointers (test_model_trace.c:496-503), and
 * the device-resident MoE block built from QwenConfig / QwenLayerWeights
 * (model.h:9-58).  Compiled with gcc against include/moehip.h only, so it
 * proves the C ABI (not a Python binding) links and computes.
 *
 * Test infrastructure: tests/test_gpu_c_caller.py writes the input file,
 * runs this program and compares its output file with the oracle.
 *
 *   moe_caller <in.bin> <out.bin>
 * in.bin:  int32 {dtype, D, d_ff, E, top_k, T}, then router_w f32 [E][D],
 *          gq [E][d_ff][rb_g], gs f32 [E][d_ff], uq, us (same shapes),
 *          dq [E][D][rb_d], ds f32 [E][D], x f32 [T][D]
 *          (rb_g = D, rb_d = d_ff for Q8; halves for Q4)
 * out.bin: f32 gate [d_ff]  = matmul_adaptive(x[0], expert 0 gate)
 *          f32 down [D]     = matmul_adaptive(x[0][0..d_ff), expert 1 down)
 *          f32 router [E]   = matmul_adaptive(x[0], router_w) (fp32 branch)
 *          f32 zero [4]     = matmul_adaptive with dtype 9 (zero fill)
 *          f32 out [T][D], int32 idx [T][top_k], f32 p [T][top_k]
 *                           = moe_layer_forward(x, residual x)
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "moehip.h"

static void* read_n(FILE* f, size_t bytes) {
  void* p = malloc(bytes ? bytes : 1);
  if (!p || fread(p, 1, bytes, f) != bytes) {
    fprintf(stderr, "moe_caller: short input\n");
    exit(2);
  }
  return p;
}

static void must(moe_status st, const char* what) {
  if (st != MOE_OK) {
    fprintf(stderr, "moe_caller: %s failed: %s\n", what, moe_last_error());
    exit(3);
  }
}

int main(int argc, char** argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: moe_caller <in.bin> <out.bin>\n");
    return 1;
  }
  FILE* f = fopen(argv[1], "rb");
  if (!f) return 1;
  int hdr[6];
  if (fread(hdr, sizeof(int), 6, f) != 6) return 2;
  const int dtype = hdr[0], D = hdr[1], dff = hdr[2], E = hdr[3], topk = hdr[4], T = hdr[5];
  const size_t rbg = dtype == 2 ? (size_t)D : (size_t)D / 2;
  const size_t rbd = dtype == 2 ? (size_t)dff : (size_t)dff / 2;
  float* router_w = (float*)read_n(f, sizeof(float) * (size_t)E * D);
  unsigned char* gq = (unsigned char*)read_n(f, (size_t)E * dff * rbg);
  float* gs = (float*)read_n(f, sizeof(float) * (size_t)E * dff);
  unsigned char* uq = (unsigned char*)read_n(f, (size_t)E * dff * rbg);
  float* us = (float*)read_n(f, sizeof(float) * (size_t)E * dff);
  unsigned char* dq = (unsigned char*)read_n(f, (size_t)E * D * rbd);
  float* ds = (float*)read_n(f, sizeof(float) * (size_t)E * D);
  float* x = (float*)read_n(f, sizeof(float) * (size_t)T * D);
  fclose(f);

  /* one QuantizedWeight per expert and projection, as model.h binds them */
  QuantizedWeight* Wg = (QuantizedWeight*)calloc((size_t)E, sizeof(QuantizedWeight));
  QuantizedWeight* Wu = (QuantizedWeight*)calloc((size_t)E, sizeof(QuantizedWeight));
  QuantizedWeight* Wd = (QuantizedWeight*)calloc((size_t)E, sizeof(QuantizedWeight));
  for (int e = 0; e < E; ++e) {
    Wg[e].q = (const int8_t*)(gq + (size_t)e * dff * rbg);
    Wg[e].s = gs + (size_t)e * dff;
    Wg[e].rows = dff; Wg[e].cols = D; Wg[e].dtype = dtype;
    Wu[e].q = (const int8_t*)(uq + (size_t)e * dff * rbg);
    Wu[e].s = us + (size_t)e * dff;
    Wu[e].rows = dff; Wu[e].cols = D; Wu[e].dtype = dtype;
    Wd[e].q = (const int8_t*)(dq + (size_t)e * D * rbd);
    Wd[e].s = ds + (size_t)e * D;
    Wd[e].rows = D; Wd[e].cols = dff; Wd[e].dtype = dtype;
  }

  /* the drop-in, called exactly as test_model_trace.c:496-503 calls it */
  float* y_gate = (float*)malloc(sizeof(float) * (size_t)dff);
  float* y_down = (float*)malloc(sizeof(float) * (size_t)D);
  float* y_router = (float*)malloc(sizeof(float) * (size_t)E);
  float y_zero[4] = {1.0f, 2.0f, 3.0f, 4.0f};
  matmul_adaptive(x, NULL, &Wg[0], y_gate, 1, dff, D);
  matmul_adaptive(x, NULL, &Wd[1 % E], y_down, 1, D, dff);
  matmul_adaptive(x, router_w, NULL, y_router, 1, E, D);
  QuantizedWeight odd = Wg[0];
  odd.dtype = 9;
  matmul_adaptive(x, NULL, &odd, y_zero, 1, 4, D);

  /* the device-resident MoE block from the reference's structures */
  QwenConfig cfg;
  memset(&cfg, 0, sizeof(cfg));
  cfg.d_model = D; cfg.n_layers = 1; cfg.d_ff = dff; cfg.n_experts = E; cfg.top_k = topk;
  cfg.causal = 1; cfg.rope_theta = 10000000.f; cfg.rms_eps = 1e-6f;
  QwenLayerWeights lw;
  memset(&lw, 0, sizeof(lw));
  lw.router_w = router_w;
  lw.Wg_q = Wg; lw.Wu_q = Wu; lw.Wd_q = Wd;
  lw.experts_quantized = 1;
  moe_layer* layer = NULL;
  must(moe_layer_create(&cfg, &lw, &layer), "moe_layer_create");
  void *dx = NULL, *dout = NULL, *didx = NULL, *dp = NULL;
  const size_t xb = sizeof(float) * (size_t)T * D, kb = 4 * (size_t)T * topk;
  must(moe_malloc(&dx, xb), "moe_malloc");
  must(moe_malloc(&dout, xb), "moe_malloc");
  must(moe_malloc(&didx, kb), "moe_malloc");
  must(moe_malloc(&dp, kb), "moe_malloc");
  must(moe_memcpy_h2d(dx, x, xb), "upload x");
  must(moe_layer_forward(layer, (const float*)dx, (const float*)dx, T, (float*)dout,
                         (int32_t*)didx, (float*)dp), "moe_layer_forward");
  must(moe_synchronize(), "moe_synchronize");
  float* out = (float*)malloc(xb);
  int32_t* idx = (int32_t*)malloc(kb);
  float* p = (float*)malloc(kb);
  must(moe_memcpy_d2h(out, dout, xb), "download out");
  must(moe_memcpy_d2h(idx, didx, kb), "download idx");
  must(moe_memcpy_d2h(p, dp, kb), "download p");
  must(moe_layer_destroy(layer), "moe_layer_destroy");
  moe_free(dx); moe_free(dout); moe_free(didx); moe_free(dp);

  FILE* o = fopen(argv[2], "wb");
  if (!o) return 1;
  fwrite(y_gate, sizeof(float), (size_t)dff, o);
  fwrite(y_down, sizeof(float), (size_t)D, o);
  fwrite(y_router, sizeof(float), (size_t)E, o);
  fwrite(y_zero, sizeof(float), 4, o);
  fwrite(out, 1, xb, o);
  fwrite(idx, 1, kb, o);
  fwrite(p, 1, kb, o);
  fclose(o);
  printf("moe_caller ok\n");
  return 0;
}
