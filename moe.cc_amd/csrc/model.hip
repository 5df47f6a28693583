// model.hip - a whole Qwen3-MoE model resident on one MI355X: the forward of
// test_model_trace.c:526-579 (embedding, 48 x [rmsnorm, attention, residual,
// MoE block], final norm, head) with a KV cache, greedy decoding on the
// device, and the weights' upload from the reference's structures
// (model.h:9-69) or from a QW3W file (io.c:193-285, model.h:107-323).
//
// Device layout of one layer: [Wq; Wk; Wv] as one row-major [(nq + 2 nkv) hd
// x D] fp32 matrix (one product launch for the three projections; each
// output is still its own chain), Wo [D x nq hd], the norms, and the MoE
// block (moe_layer: router, rms2, experts).  KV caches [L][nkv][max_seq][hd]
// fp32; RoPE cos/sin tables [max_seq][hd/2], computed once at creation with
// the C library's powf / cosf / sinf, the calls the reference makes for
// every position (test_model_trace.c:310-336); they are constants of
// (theta, head_dim, position).
#include <fcntl.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <initializer_list>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "dense.h"
#include "moe_lib.h"

using namespace moe;

namespace {

struct DevLayer {
  float* wqkv = nullptr;   // [nqkv][D]
  float* bqkv = nullptr;   // [nqkv] or null
  float* wo = nullptr;     // [D][Dq]
  float* bo = nullptr;
  float* q_norm = nullptr;
  float* k_norm = nullptr;
  float* rms1 = nullptr;
  moe_layer* moe = nullptr;
};

struct Buf {
  void* p = nullptr;
  size_t bytes = 0;
};

}  // namespace

struct moe_model {
  moe_model() { moe::live_objects(1); }
  ~moe_model() { moe::live_objects(-1); }
  QwenConfig cfg{};
  int max_seq = 0, pos = 0, nqkv = 0, Dq = 0, Dkv = 0;
  float scale = 0.0f;
  float* tok_emb = nullptr;
  float* final_norm = nullptr;
  float* lm_head = nullptr;   // == tok_emb when tied
  std::vector<DevLayer> layers;
  float* kc = nullptr;
  float* vc = nullptr;
  float* rope_cos = nullptr;
  float* rope_sin = nullptr;
  // per-forward scratch, grown on demand
  Buf x, xa, xn, qkv, H, S, ids;
  float* xf = nullptr;
  float* logits = nullptr;
  float* head_part = nullptr;   // block maxima of the head's product
  int32_t* next = nullptr;      // greedy choice of the last forward
  int32_t* hist_pos = nullptr;  // generation counter
  Buf hist;
  std::mutex mu;
};

namespace {

template <class T>
moe_status dalloc(T** p, size_t count, const char* what) {
  *p = nullptr;
  if (!count) return MOE_OK;
  return check_hip(hipMalloc((void**)p, count * sizeof(T)), what);
}

template <class T>
void dfree(T*& p) {
  if (p) (void)hipFree((void*)p);
  p = nullptr;
}

moe_status grow(Buf& b, size_t need) {
  if (need <= b.bytes) return MOE_OK;
  moe_status st = check_hip(hipStreamSynchronize(stream()), "model scratch sync");
  if (st) return st;
  if (b.p) (void)hipFree(b.p);
  b.p = nullptr;
  b.bytes = 0;
  if ((st = check_hip(hipMalloc(&b.p, need), "model scratch"))) return st;
  b.bytes = need;
  return MOE_OK;
}

moe_status h2d(void* dst, const void* src, size_t bytes) {
  if (!bytes) return MOE_OK;
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()), "model upload");
}

moe_status d2d(void* dst, const void* src, size_t bytes) {
  if (!bytes) return MOE_OK;
  return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream()), "model copy");
}

void free_model(moe_model* m) {
  (void)hipStreamSynchronize(stream());
  for (DevLayer& l : m->layers) {
    dfree(l.wqkv); dfree(l.bqkv); dfree(l.wo); dfree(l.bo);
    dfree(l.q_norm); dfree(l.k_norm); dfree(l.rms1);
    if (l.moe) moe_layer_destroy(l.moe);
    l.moe = nullptr;
  }
  if (m->lm_head != m->tok_emb) dfree(m->lm_head);
  m->lm_head = nullptr;
  dfree(m->tok_emb); dfree(m->final_norm); dfree(m->kc); dfree(m->vc);
  dfree(m->rope_cos); dfree(m->rope_sin); dfree(m->xf); dfree(m->logits);
  dfree(m->head_part); dfree(m->next); dfree(m->hist_pos);
  for (Buf* b : {&m->x, &m->xa, &m->xn, &m->qkv, &m->H, &m->S, &m->ids, &m->hist})
    if (b->p) (void)hipFree(b->p);
  delete m;
}

moe_status check_cfg(const QwenConfig* c, int max_seq) {
  if (c->d_model <= 0 || c->n_layers <= 0 || c->head_dim <= 0 || c->n_q <= 0 || c->n_kv <= 0 ||
      c->d_ff <= 0 || c->n_experts <= 0 || c->top_k <= 0 || c->vocab_size <= 0)
    return set_error(MOE_ERR_ARG, "model: bad config");
  if (c->n_q % c->n_kv) return set_error(MOE_ERR_ARG, "model: n_q %% n_kv != 0");
  if (c->head_dim % 4 || c->head_dim > 512)
    return set_error(MOE_ERR_UNSUPPORTED, "model: head_dim %d (need a multiple of 4, <= 512)",
                     c->head_dim);
  if (!c->causal) return set_error(MOE_ERR_UNSUPPORTED, "model: only causal attention");
  if (max_seq <= 0 || max_seq > 16384)
    return set_error(MOE_ERR_ARG, "model: max_seq %d outside 1..16384", max_seq);
  return MOE_OK;
}

// Common part of the creators: sizes, caches, RoPE tables, fixed scratch.
moe_status init_model(moe_model* m, const QwenConfig* cfg, int max_seq) {
  m->cfg = *cfg;
  m->max_seq = max_seq;
  m->Dq = cfg->n_q * cfg->head_dim;
  m->Dkv = cfg->n_kv * cfg->head_dim;
  m->nqkv = m->Dq + 2 * m->Dkv;
  m->scale = 1.0f / sqrtf((float)cfg->head_dim);   // test_model_trace.c:357
  m->layers.resize(cfg->n_layers);
  const size_t cache = (size_t)cfg->n_layers * cfg->n_kv * max_seq * cfg->head_dim;
  const int d2 = cfg->head_dim / 2;
  moe_status st;
  if ((st = dalloc(&m->kc, cache, "kv cache")) || (st = dalloc(&m->vc, cache, "kv cache")) ||
      (st = dalloc(&m->rope_cos, (size_t)max_seq * d2, "rope")) ||
      (st = dalloc(&m->rope_sin, (size_t)max_seq * d2, "rope")) ||
      (st = dalloc(&m->xf, (size_t)cfg->d_model, "model")) ||
      (st = dalloc(&m->logits, (size_t)cfg->vocab_size, "logits")) ||
      (st = dalloc(&m->head_part, (size_t)cfg->vocab_size / 16 + 1, "logits")) ||
      (st = dalloc(&m->next, 1, "model")) || (st = dalloc(&m->hist_pos, 1, "model")))
    return st;
  // test_model_trace.c:310-336: inv_i = powf(theta, (-2 i) / hd), angle =
  // pos * inv_i, cosf / sinf of it (host C library, as in the reference)
  std::vector<float> c((size_t)max_seq * d2), s((size_t)max_seq * d2);
  for (int p = 0; p < max_seq; ++p) {
    const float pf = (float)p;
    for (int i = 0; i < d2; ++i) {
      const float exponent = -2.0f * (float)i / (float)cfg->head_dim;
      const float inv = powf(cfg->rope_theta, exponent);
      const float ang = pf * inv;
      c[(size_t)p * d2 + i] = cosf(ang);
      s[(size_t)p * d2 + i] = sinf(ang);
    }
  }
  if ((st = h2d(m->rope_cos, c.data(), c.size() * 4)) || (st = h2d(m->rope_sin, s.data(), s.size() * 4)))
    return st;
  return check_hip(hipStreamSynchronize(stream()), "model init sync");
}

moe_status ensure_scratch(moe_model* m, int T) {
  const QwenConfig& c = m->cfg;
  moe_status st;
  const size_t td = (size_t)T * c.d_model * 4;
  if ((st = grow(m->x, td)) || (st = grow(m->xa, td)) || (st = grow(m->xn, td)) ||
      (st = grow(m->qkv, (size_t)T * m->nqkv * 4)) || (st = grow(m->H, (size_t)T * m->Dq * 4)) ||
      (st = grow(m->S, (size_t)T * c.n_q * m->max_seq * 4)) || (st = grow(m->ids, (size_t)T * 4)))
    return st;
  return MOE_OK;
}

// T new tokens (device ids) at positions pos..pos+T-1.
moe_status forward_dev(moe_model* m, const int32_t* ids_d, int T, float* logits_out,
                       int32_t* next_out, bool record) {
  const QwenConfig& c = m->cfg;
  hipStream_t s = stream();
  const int D = c.d_model, hd = c.head_dim;
  const float eps = c.rms_eps;
  float* x = (float*)m->x.p;
  float* xa = (float*)m->xa.p;
  float* xn = (float*)m->xn.p;
  float* qkv = (float*)m->qkv.p;
  moe_status st;
  if ((st = embed_rows(ids_d, T, m->tok_emb, c.vocab_size, D, x, s))) return st;
  const size_t per_layer = (size_t)c.n_kv * m->max_seq * hd;
  for (int l = 0; l < c.n_layers; ++l) {
    DevLayer& L = m->layers[l];
    float* kc = m->kc + l * per_layer;
    float* vc = m->vc + l * per_layer;
    // :449 norm1, :363-369 Q, K, V (+ biases); the norm fused into the
    // product for few tokens
    DenseArgs qa{xn, D, L.wqkv, D, L.bqkv, nullptr, 0, qkv, m->nqkv, T, m->nqkv, D};
    if (dense_norm_ok(T, D)) {
      qa.A = x;
      qa.norm = 1; qa.norm_w = L.rms1; qa.eps = eps;
    } else if ((st = moe_rmsnorm_dev(x, L.rms1, xn, T, D, eps))) {
      return st;
    }
    if ((st = dense_matmul(qa, s))) return st;
    // :371-398 q/k norm, :400 RoPE, K/V into the cache
    // (one token: done inside the score launch)
    AttnArgs aa{qkv, m->nqkv, kc, vc, (float*)m->S.p, (float*)m->H.p, T, m->pos, c.n_q, c.n_kv,
                hd, m->max_seq, m->scale};
    if (T == 1) {
      aa.fuse_heads = 1;
      aa.q_norm = L.q_norm; aa.k_norm = L.k_norm; aa.eps = eps;
      aa.rope_cos = m->rope_cos; aa.rope_sin = m->rope_sin;
      static const bool no_pf = getenv("MOEHIP_NO_WO_PREFETCH") != nullptr;
      if (!no_pf) {
        aa.pf_w = L.wo; aa.pf_ld = m->Dq; aa.pf_n = D;
      }
    } else {
      HeadArgs ha{qkv, m->nqkv, T, m->pos, c.n_q, c.n_kv, hd, m->max_seq, L.q_norm, L.k_norm,
                  eps, m->rope_cos, m->rope_sin, kc, vc};
      if ((st = heads_norm_rope(ha, s))) return st;
    }
    // :402-426 causal attention
    if ((st = attention_rows(aa, s))) return st;
    // :427-428 output projection (+ bias), :460 residual
    DenseArgs oa{(float*)m->H.p, m->Dq, L.wo, m->Dq, L.bo, x, D, xa, D, T, D, m->Dq};
    if ((st = dense_matmul(oa, s))) return st;
    // :461-517 norm2, router, experts, weighted sum, residual
    if ((st = moe_block_forward(L.moe, xa, T, x, eps))) return st;
  }
  // :567-571 final norm of the last row, head
  if ((st = moe_rmsnorm_dev(x + (size_t)(T - 1) * D, m->final_norm, m->xf, 1, D, eps))) return st;
  float* lg = logits_out ? logits_out : m->logits;
  DenseArgs ha{m->xf, D, m->lm_head, D, nullptr, nullptr, 0, lg, c.vocab_size, 1, c.vocab_size, D};
  // the head's blocks leave their maxima for the next-token choice (:735-746)
  const bool part = dense_amax_ok(ha);
  if (part) ha.amax_part = m->head_part;
  if ((st = dense_matmul(ha, s))) return st;
  if ((st = greedy_vec(lg, c.vocab_size, part ? m->head_part : nullptr,
                       part ? dense_amax_rows(c.vocab_size) : 0, next_out ? next_out : m->next,
                       record ? (int32_t*)m->hist.p : nullptr, m->hist_pos, s)))
    return st;
  m->pos += T;
  return MOE_OK;
}

moe_status forward_checked(moe_model* m, const int32_t* ids, int T, int ids_on_device,
                           float* logits_out, int32_t* next_out) {
  if (T <= 0) return set_error(MOE_ERR_ARG, "model forward: T = %d", T);
  if (m->pos + T > m->max_seq)
    return set_error(MOE_ERR_ARG, "model forward: position %d + %d tokens exceeds max_seq %d",
                     m->pos, T, m->max_seq);
  moe_status st = ensure_scratch(m, T);
  if (st) return st;
  const int32_t* ids_d = ids;
  if (!ids_on_device) {
    for (int t = 0; t < T; ++t)
      if (ids[t] < 0 || ids[t] >= m->cfg.vocab_size)
        return set_error(MOE_ERR_ARG, "model forward: token id %d outside [0, %d)", ids[t],
                         m->cfg.vocab_size);
    if ((st = h2d(m->ids.p, ids, (size_t)T * 4))) return st;
    ids_d = (const int32_t*)m->ids.p;
  }
  return forward_dev(m, ids_d, T, logits_out, next_out, false);
}

// ---- QW3W file (io.c:193-285) ----

struct Entry {
  int dtype;
  std::vector<int> shape;
  const void* data;
  size_t bytes;
};

struct BinIndex {
  void* map = nullptr;
  size_t size = 0;
  std::unordered_map<std::string, Entry> idx;
  ~BinIndex() {
    if (map) munmap(map, size);
  }
  const Entry* find(const std::string& k) const {
    auto it = idx.find(k);
    return it == idx.end() ? nullptr : &it->second;
  }
};

moe_status bin_open(const char* path, BinIndex* b) {
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return set_error(MOE_ERR_ARG, "load: cannot open %s", path);
  struct stat sb;
  if (fstat(fd, &sb) != 0 || sb.st_size < 10) {
    close(fd);
    return set_error(MOE_ERR_ARG, "load: %s is not a QW3W file", path);
  }
  b->size = (size_t)sb.st_size;
  b->map = mmap(nullptr, b->size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (b->map == MAP_FAILED) {
    b->map = nullptr;
    return set_error(MOE_ERR_ARG, "load: mmap %s failed", path);
  }
  const uint8_t* p = (const uint8_t*)b->map;
  static const uint8_t magic[6] = {'Q', 'W', '3', 'W', 0, 1};
  if (memcmp(p, magic, 6) != 0) return set_error(MOE_ERR_ARG, "load: bad magic in %s", path);
  // the header count may undercount quantized files (merge_dir.py:37): read to the end
  size_t off = 10;
  auto u32 = [&](size_t o) { uint32_t v; memcpy(&v, p + o, 4); return v; };
  while (off + 4 <= b->size) {
    const uint32_t nl = u32(off);
    off += 4;
    if (off + nl + 8 > b->size) return set_error(MOE_ERR_ARG, "load: truncated entry in %s", path);
    std::string name((const char*)p + off, nl);
    off += nl;
    Entry e;
    e.dtype = (int)u32(off);
    const uint32_t nd = u32(off + 4);
    off += 8;
    if (e.dtype < 0 || e.dtype > 3 || nd > 8 || off + 4 * (size_t)nd > b->size)
      return set_error(MOE_ERR_ARG, "load: bad entry %s in %s", name.c_str(), path);
    // every dimension positive and within int; the element count may not
    // exceed what is left of the file (checked before each multiply, so the
    // product cannot wrap)
    size_t elems = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      const uint32_t dim = u32(off);
      off += 4;
      if (dim == 0 || dim > 0x7fffffffu)
        return set_error(MOE_ERR_ARG, "load: %s has dimension %u", name.c_str(), dim);
      if (elems > (b->size - off) / dim)
        return set_error(MOE_ERR_ARG, "load: truncated %s", name.c_str());
      elems *= dim;
      e.shape.push_back((int)dim);
    }
    const size_t bpe = e.dtype == 0 ? 4 : (e.dtype == 1 ? 2 : 1);
    if (elems > (b->size - off) / bpe) return set_error(MOE_ERR_ARG, "load: truncated %s", name.c_str());
    e.bytes = elems * bpe;
    e.data = p + off;
    off += e.bytes;
    b->idx[name] = std::move(e);
  }
  return MOE_OK;
}

// An f32 tensor as an aligned host copy (file offsets are unaligned).
const float* f32_of(const Entry* e, std::vector<std::vector<float>>& keep) {
  if (!e || e->dtype != 0) return nullptr;
  keep.emplace_back(e->bytes / 4);
  memcpy(keep.back().data(), e->data, e->bytes);
  return keep.back().data();
}

// True if e has dtype `dt` and exactly the dimensions `dims`.
bool has_shape(const Entry* e, int dt, std::initializer_list<long long> dims) {
  if (!e || e->dtype != dt || e->shape.size() != dims.size()) return false;
  size_t i = 0;
  for (long long d : dims)
    if (e->shape[i++] != d) return false;
  return true;
}

// The names load_all_weights binds (model.h:107-323) and the first of the
// alternative names it accepts that the file holds.
const char* kProj[3] = {"gate", "up", "down"};

const Entry* find_layer(const BinIndex& b, char* k, size_t kn, int L, const char* fmt,
                        const char* alt = nullptr) {
  snprintf(k, kn, fmt, L);
  const Entry* e = b.find(k);
  if (!e && alt) {
    snprintf(k, kn, alt, L);
    e = b.find(k);
  }
  return e;
}

// Infers the config from the tensor shapes as load_all_weights does
// (model.h:110-163; top_k 8, theta 1e7, eps 1e-6 fixed) and checks, before
// anything is copied or uploaded, that every tensor the model binds exists
// with the rank, dtype and size that config implies: embedding and head
// [V][D], final and layer norms [D], q/k/v/o [nq*hd | nkv*hd][D] and
// [D][nq*hd], biases, q/k norms [hd], router [E][D] (+ [E]), and for every
// layer and expert the gate/up [d_ff][D] and down [D][d_ff] weights (Q4:
// half the columns in bytes) with their [rows] scales.  The reference reads
// such a file without checks; a mismatch there is an out-of-bounds read,
// here it is MOE_ERR_ARG.
moe_status validate_file(const BinIndex& b, const char* path, QwenConfig* out, int* dtype_out) {
  char k[256];
  const Entry* wq0 = b.find("model.layers.0.self_attn.q_proj.weight");
  const Entry* wk0 = b.find("model.layers.0.self_attn.k_proj.weight");
  const Entry* emb = b.find("model.embed_tokens.weight");
  const Entry* fnorm = b.find("model.norm.weight");
  if (!fnorm) fnorm = b.find("model.final_layernorm.weight");
  if (!wq0 || !wk0 || !emb || !fnorm || wq0->shape.size() != 2 || wk0->shape.size() != 2 ||
      emb->shape.size() != 2)
    return set_error(MOE_ERR_ARG, "load: %s lacks the layer-0 attention / embedding / norm", path);
  QwenConfig cfg{};
  cfg.d_model = wq0->shape[1];
  const Entry* qn0 = b.find("model.layers.0.self_attn.q_norm.weight");
  if (qn0 && qn0->shape.size() != 1)
    return set_error(MOE_ERR_ARG, "load: q_norm of layer 0 is not a vector");
  cfg.head_dim = qn0 ? qn0->shape[0] : wq0->shape[0] / 32;
  if (cfg.head_dim <= 0 || wq0->shape[0] % cfg.head_dim || wk0->shape[0] % cfg.head_dim)
    return set_error(MOE_ERR_ARG, "load: q/k rows %d/%d are not multiples of head_dim %d",
                     wq0->shape[0], wk0->shape[0], cfg.head_dim);
  cfg.n_q = wq0->shape[0] / cfg.head_dim;
  cfg.n_kv = wk0->shape[0] / cfg.head_dim;
  cfg.vocab_size = emb->shape[0];
  for (cfg.n_layers = 0;; ++cfg.n_layers) {
    snprintf(k, sizeof k, "model.layers.%d.self_attn.q_proj.weight", cfg.n_layers);
    if (!b.find(k)) break;
  }
  int dtype = 0;
  for (cfg.n_experts = 0;; ++cfg.n_experts) {
    snprintf(k, sizeof k, "model.layers.0.mlp.experts.%d.down_proj.weight", cfg.n_experts);
    const std::string base = k;
    const Entry* e = b.find(base.c_str());
    int dt = 0;
    if (!e && (e = b.find((base + ".q8").c_str()))) dt = 2;
    if (!e && (e = b.find((base + ".q4").c_str()))) dt = 3;
    if (!e) break;
    if (e->shape.size() != 2)
      return set_error(MOE_ERR_ARG, "load: %s is not a matrix", base.c_str());
    const int dff = e->shape[1] * (dt == 3 ? 2 : 1);
    if (cfg.n_experts > 0 && (dt != dtype || dff != cfg.d_ff))
      return set_error(MOE_ERR_ARG, "load: expert %d of layer 0 differs from expert 0", cfg.n_experts);
    cfg.d_ff = dff;
    dtype = dt;
  }
  if (cfg.n_experts == 0 || cfg.d_ff <= 0) return set_error(MOE_ERR_ARG, "load: no experts in %s", path);
  if (dtype == 0) return set_error(MOE_ERR_UNSUPPORTED, "load: fp32 experts are not supported");
  cfg.top_k = 8;
  cfg.causal = 1;
  cfg.rope_theta = 10000000.f;
  cfg.rms_eps = 1e-6f;
  const long long D = cfg.d_model, V = cfg.vocab_size, hd = cfg.head_dim, E = cfg.n_experts;
  const long long Dq = (long long)cfg.n_q * hd, Dkv = (long long)cfg.n_kv * hd, dff = cfg.d_ff;
  if (dtype == 3 && (D % 2 || dff % 2))
    return set_error(MOE_ERR_ARG, "load: Q4 experts need even d_model and d_ff");
  if (!has_shape(emb, 0, {V, D}) || !has_shape(fnorm, 0, {D}))
    return set_error(MOE_ERR_ARG, "load: embedding or final norm is not f32 [%lld x %lld] / [%lld]",
                     V, D, D);
  const Entry* head = b.find("lm_head.weight");
  if (head && !has_shape(head, 0, {V, D}))
    return set_error(MOE_ERR_ARG, "load: lm_head is not f32 [%lld x %lld]", V, D);
  struct Req { const char* fmt; const char* alt; long long r, c; bool need; };
  const Req reqs[] = {
      {"model.layers.%d.self_attn.q_proj.weight", nullptr, Dq, D, true},
      {"model.layers.%d.self_attn.k_proj.weight", nullptr, Dkv, D, true},
      {"model.layers.%d.self_attn.v_proj.weight", nullptr, Dkv, D, true},
      {"model.layers.%d.self_attn.o_proj.weight", nullptr, D, Dq, true},
      {"model.layers.%d.self_attn.q_proj.bias", nullptr, Dq, 0, false},
      {"model.layers.%d.self_attn.k_proj.bias", nullptr, Dkv, 0, false},
      {"model.layers.%d.self_attn.v_proj.bias", nullptr, Dkv, 0, false},
      {"model.layers.%d.self_attn.o_proj.bias", nullptr, D, 0, false},
      {"model.layers.%d.self_attn.q_norm.weight", nullptr, hd, 0, false},
      {"model.layers.%d.self_attn.k_norm.weight", nullptr, hd, 0, false},
      {"model.layers.%d.input_layernorm.weight", "model.layers.%d.rms_1.weight", D, 0, true},
      {"model.layers.%d.post_attention_layernorm.weight", "model.layers.%d.rms_2.weight", D, 0, true},
      {"model.layers.%d.mlp.gate.weight", "model.layers.%d.mlp.router.gate.weight", E, D, true},
      {"model.layers.%d.mlp.gate.bias", nullptr, E, 0, false},
  };
  const char* qsuf = dtype == 2 ? ".q8" : ".q4";
  const long long cg = dtype == 2 ? D : D / 2, cd = dtype == 2 ? dff : dff / 2;
  for (int L = 0; L < cfg.n_layers; ++L) {
    for (const Req& r : reqs) {
      const Entry* e = find_layer(b, k, sizeof k, L, r.fmt, r.alt);
      if (!e) {
        if (r.need) return set_error(MOE_ERR_ARG, "load: layer %d is incomplete in %s (%s)", L, path, k);
        continue;
      }
      const bool ok = r.c ? has_shape(e, 0, {r.r, r.c}) : has_shape(e, 0, {r.r});
      if (!ok) return set_error(MOE_ERR_ARG, "load: %s has the wrong dtype or shape", k);
    }
    for (int e = 0; e < E; ++e)
      for (int j = 0; j < 3; ++j) {
        snprintf(k, sizeof k, "model.layers.%d.mlp.experts.%d.%s_proj.weight", L, e, kProj[j]);
        const std::string base = k;
        const Entry* q = b.find((base + qsuf).c_str());
        const Entry* sc = b.find((base + ".scale").c_str());
        const long long rows = j < 2 ? dff : D, cols = j < 2 ? cg : cd;
        if (!has_shape(q, dtype, {rows, cols}) || !has_shape(sc, 0, {rows}))
          return set_error(MOE_ERR_ARG, "load: %s%s / .scale missing or not [%lld x %lld] / [%lld]",
                           base.c_str(), qsuf, rows, cols, rows);
      }
  }
  *out = cfg;
  *dtype_out = dtype;
  return MOE_OK;
}

}  // namespace

extern "C" {

moe_status moe_model_create(const QwenConfig* cfg, const QwenWeights* w, int max_seq,
                            moe_model** out) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!cfg || !w || !out) return set_error(MOE_ERR_ARG, "model_create: null argument");
  *out = nullptr;
  if ((st = check_cfg(cfg, max_seq))) return st;
  if (!w->tok_emb || !w->final_norm_w || !w->layers)
    return set_error(MOE_ERR_ARG, "model_create: missing tensors");
  moe_model* m = new (std::nothrow) moe_model();
  if (!m) return set_error(MOE_ERR_NOMEM, "model_create: host allocation");
  if ((st = init_model(m, cfg, max_seq))) { free_model(m); return st; }
  const int D = cfg->d_model, V = cfg->vocab_size, hd = cfg->head_dim;
  if ((st = dalloc(&m->tok_emb, (size_t)V * D, "embedding")) ||
      (st = h2d(m->tok_emb, w->tok_emb, (size_t)V * D * 4)) ||
      (st = dalloc(&m->final_norm, (size_t)D, "norm")) ||
      (st = h2d(m->final_norm, w->final_norm_w, (size_t)D * 4))) {
    free_model(m);
    return st;
  }
  if (w->lm_head) {
    if ((st = dalloc(&m->lm_head, (size_t)V * D, "lm_head")) ||
        (st = h2d(m->lm_head, w->lm_head, (size_t)V * D * 4))) {
      free_model(m);
      return st;
    }
  } else {
    m->lm_head = m->tok_emb;   // tied (test_model_trace.c:570)
  }
  const size_t nq = (size_t)m->Dq, nkv = (size_t)m->Dkv;
  for (int l = 0; l < cfg->n_layers; ++l) {
    const QwenLayerWeights& lw = w->layers[l];
    DevLayer& L = m->layers[l];
    if (!lw.Wq || !lw.Wk || !lw.Wv || !lw.Wo) {
      free_model(m);
      return set_error(MOE_ERR_ARG, "model_create: layer %d lacks attention weights", l);
    }
    if ((st = dalloc(&L.wqkv, (size_t)m->nqkv * D, "wqkv")) ||
        (st = h2d(L.wqkv, lw.Wq, nq * D * 4)) || (st = h2d(L.wqkv + nq * D, lw.Wk, nkv * D * 4)) ||
        (st = h2d(L.wqkv + (nq + nkv) * D, lw.Wv, nkv * D * 4)) ||
        (st = dalloc(&L.wo, (size_t)D * nq, "wo")) || (st = h2d(L.wo, lw.Wo, (size_t)D * nq * 4))) {
      free_model(m);
      return st;
    }
    if (lw.bq || lw.bk || lw.bv) {
      // a missing bias is +0: adding +0 leaves a chain result unchanged
      std::vector<float> b((size_t)m->nqkv, 0.0f);
      if (lw.bq) memcpy(b.data(), lw.bq, nq * 4);
      if (lw.bk) memcpy(b.data() + nq, lw.bk, nkv * 4);
      if (lw.bv) memcpy(b.data() + nq + nkv, lw.bv, nkv * 4);
      if ((st = dalloc(&L.bqkv, b.size(), "bias")) || (st = h2d(L.bqkv, b.data(), b.size() * 4)) ||
          (st = check_hip(hipStreamSynchronize(stream()), "bias sync"))) {
        free_model(m);
        return st;
      }
    }
    struct { const float* src; float** dst; size_t n; } small[] = {
        {lw.bo, &L.bo, (size_t)D}, {lw.q_norm, &L.q_norm, (size_t)hd},
        {lw.k_norm, &L.k_norm, (size_t)hd}, {lw.rms1_w, &L.rms1, (size_t)D}};
    for (auto& t : small) {
      if (!t.src) continue;
      if ((st = dalloc(t.dst, t.n, "layer vector")) || (st = h2d(*t.dst, t.src, t.n * 4))) {
        free_model(m);
        return st;
      }
    }
    if ((st = moe_layer_create(cfg, &lw, &L.moe))) {
      free_model(m);
      return st;
    }
  }
  if ((st = check_hip(hipStreamSynchronize(stream()), "model upload sync"))) {
    free_model(m);
    return st;
  }
  *out = m;
  return MOE_OK;
}

moe_status moe_model_create_synthetic(const QwenConfig* cfg, int expert_dtype, int untied_head,
                                      uint64_t seed, float stdv, int max_seq, moe_model** out) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!cfg || !out) return set_error(MOE_ERR_ARG, "model_create_synthetic: null argument");
  *out = nullptr;
  if ((st = check_cfg(cfg, max_seq))) return st;
  if (expert_dtype != 2 && expert_dtype != 3)
    return set_error(MOE_ERR_ARG, "model_create_synthetic: expert dtype %d", expert_dtype);
  moe_model* m = new (std::nothrow) moe_model();
  if (!m) return set_error(MOE_ERR_NOMEM, "model_create_synthetic: host allocation");
  if ((st = init_model(m, cfg, max_seq))) { free_model(m); return st; }
  const int D = cfg->d_model, V = cfg->vocab_size, hd = cfg->head_dim, E = cfg->n_experts;
  const int dff = cfg->d_ff;
  uint64_t sd = seed * 1000003ull;
  auto normal = [&](float* p, size_t n, float mean, float sdv) {
    return moe_fill_normal_dev(p, n, ++sd, mean, sdv);
  };
  auto fail = [&](moe_status s2) { free_model(m); return s2; };
  if ((st = dalloc(&m->tok_emb, (size_t)V * D, "embedding")) ||
      (st = normal(m->tok_emb, (size_t)V * D, 0.0f, stdv)) ||
      (st = dalloc(&m->final_norm, (size_t)D, "norm")) || (st = normal(m->final_norm, D, 1.0f, 0.0f)))
    return fail(st);
  if (untied_head) {
    if ((st = dalloc(&m->lm_head, (size_t)V * D, "lm_head")) ||
        (st = normal(m->lm_head, (size_t)V * D, 0.0f, stdv)))
      return fail(st);
  } else {
    m->lm_head = m->tok_emb;
  }
  const long long rbg = expert_dtype == 2 ? D : D / 2, rbd = expert_dtype == 2 ? dff : dff / 2;
  float* tmp = nullptr;
  uint8_t *gq = nullptr, *uq = nullptr, *dq = nullptr;
  float *gs = nullptr, *us = nullptr, *ds = nullptr, *rw = nullptr, *ones = nullptr;
  auto free_tmp = [&]() {
    dfree(tmp); dfree(gq); dfree(uq); dfree(dq); dfree(gs); dfree(us); dfree(ds); dfree(rw);
    dfree(ones);
  };
  if ((st = dalloc(&tmp, (size_t)E * dff * D, "synthetic tmp")) ||
      (st = dalloc(&gq, (size_t)E * dff * rbg, "tmp")) || (st = dalloc(&uq, (size_t)E * dff * rbg, "tmp")) ||
      (st = dalloc(&dq, (size_t)E * D * rbd, "tmp")) || (st = dalloc(&gs, (size_t)E * dff, "tmp")) ||
      (st = dalloc(&us, (size_t)E * dff, "tmp")) || (st = dalloc(&ds, (size_t)E * D, "tmp")) ||
      (st = dalloc(&rw, (size_t)E * D, "tmp")) || (st = dalloc(&ones, (size_t)D, "tmp")) ||
      (st = normal(ones, D, 1.0f, 0.0f))) {
    free_tmp();
    return fail(st);
  }
  for (int l = 0; l < cfg->n_layers && !st; ++l) {
    DevLayer& L = m->layers[l];
    if ((st = dalloc(&L.wqkv, (size_t)m->nqkv * D, "wqkv")) ||
        (st = normal(L.wqkv, (size_t)m->nqkv * D, 0.0f, stdv)) ||
        (st = dalloc(&L.wo, (size_t)D * m->Dq, "wo")) ||
        (st = normal(L.wo, (size_t)D * m->Dq, 0.0f, stdv)) ||
        (st = dalloc(&L.q_norm, (size_t)hd, "qn")) || (st = d2d(L.q_norm, ones, (size_t)hd * 4)) ||
        (st = dalloc(&L.k_norm, (size_t)hd, "kn")) || (st = d2d(L.k_norm, ones, (size_t)hd * 4)) ||
        (st = dalloc(&L.rms1, (size_t)D, "rms1")) || (st = d2d(L.rms1, ones, (size_t)D * 4)) ||
        (st = normal(rw, (size_t)E * D, 0.0f, stdv)) ||
        (st = normal(tmp, (size_t)E * dff * D, 0.0f, stdv)) ||
        (st = moe_quantize_rows_dev(expert_dtype, tmp, (long long)E * dff, D, gq, gs)) ||
        (st = normal(tmp, (size_t)E * dff * D, 0.0f, stdv)) ||
        (st = moe_quantize_rows_dev(expert_dtype, tmp, (long long)E * dff, D, uq, us)) ||
        (st = normal(tmp, (size_t)E * D * dff, 0.0f, stdv)) ||
        (st = moe_quantize_rows_dev(expert_dtype, tmp, (long long)E * D, dff, dq, ds)) ||
        (st = moe_layer_create_raw(expert_dtype, D, dff, E, cfg->top_k, rw, nullptr, ones, gq, gs,
                                   uq, us, dq, ds, 1, &L.moe)))
      break;
  }
  free_tmp();
  if (st) return fail(st);
  if ((st = check_hip(hipStreamSynchronize(stream()), "synthetic model sync"))) return fail(st);
  *out = m;
  return MOE_OK;
}

moe_status moe_model_inspect_file(const char* path, QwenConfig* cfg, int* expert_dtype) {
  if (!path || !cfg) return set_error(MOE_ERR_ARG, "model_inspect_file: null argument");
  BinIndex b;
  moe_status st = bin_open(path, &b);
  if (st) return st;
  int dtype = 0;
  if ((st = validate_file(b, path, cfg, &dtype))) return st;
  if (expert_dtype) *expert_dtype = dtype;
  return MOE_OK;
}

moe_status moe_model_load_file(const char* path, int max_seq, moe_model** out) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!path || !out) return set_error(MOE_ERR_ARG, "model_load_file: null argument");
  *out = nullptr;
  BinIndex b;
  if ((st = bin_open(path, &b))) return st;
  QwenConfig cfg{};
  int dtype = 0;
  // every shape is checked before anything is copied or uploaded
  if ((st = validate_file(b, path, &cfg, &dtype))) return st;
  std::vector<std::vector<float>> keep;
  char k[256];
  QwenWeights w{};
  const Entry* fnorm = b.find("model.norm.weight");
  if (!fnorm) fnorm = b.find("model.final_layernorm.weight");
  w.tok_emb = f32_of(b.find("model.embed_tokens.weight"), keep);
  w.final_norm_w = f32_of(fnorm, keep);
  w.lm_head = f32_of(b.find("lm_head.weight"), keep);
  std::vector<QwenLayerWeights> lws((size_t)cfg.n_layers);
  std::vector<std::vector<QuantizedWeight>> qws((size_t)cfg.n_layers * 3);
  std::vector<std::vector<uint8_t>> qkeep;
  auto layer_f32 = [&](int L, const char* fmt, const char* alt = nullptr) {
    return f32_of(find_layer(b, k, sizeof k, L, fmt, alt), keep);
  };
  for (int L = 0; L < cfg.n_layers; ++L) {
    QwenLayerWeights& lw = lws[L];
    lw.Wq = layer_f32(L, "model.layers.%d.self_attn.q_proj.weight");
    lw.Wk = layer_f32(L, "model.layers.%d.self_attn.k_proj.weight");
    lw.Wv = layer_f32(L, "model.layers.%d.self_attn.v_proj.weight");
    lw.Wo = layer_f32(L, "model.layers.%d.self_attn.o_proj.weight");
    lw.bq = layer_f32(L, "model.layers.%d.self_attn.q_proj.bias");
    lw.bk = layer_f32(L, "model.layers.%d.self_attn.k_proj.bias");
    lw.bv = layer_f32(L, "model.layers.%d.self_attn.v_proj.bias");
    lw.bo = layer_f32(L, "model.layers.%d.self_attn.o_proj.bias");
    lw.q_norm = layer_f32(L, "model.layers.%d.self_attn.q_norm.weight");
    lw.k_norm = layer_f32(L, "model.layers.%d.self_attn.k_norm.weight");
    lw.rms1_w = layer_f32(L, "model.layers.%d.input_layernorm.weight", "model.layers.%d.rms_1.weight");
    lw.rms2_w = layer_f32(L, "model.layers.%d.post_attention_layernorm.weight",
                          "model.layers.%d.rms_2.weight");
    lw.router_w = layer_f32(L, "model.layers.%d.mlp.gate.weight", "model.layers.%d.mlp.router.gate.weight");
    lw.router_b = layer_f32(L, "model.layers.%d.mlp.gate.bias");
    for (int j = 0; j < 3; ++j) {
      std::vector<QuantizedWeight>& v = qws[(size_t)L * 3 + j];
      v.resize((size_t)cfg.n_experts);
      for (int e = 0; e < cfg.n_experts; ++e) {
        snprintf(k, sizeof k, "model.layers.%d.mlp.experts.%d.%s_proj.weight", L, e, kProj[j]);
        const std::string base = k;
        const Entry* q = b.find((base + (dtype == 2 ? ".q8" : ".q4")).c_str());
        const Entry* sc = b.find((base + ".scale").c_str());
        qkeep.emplace_back((const uint8_t*)q->data, (const uint8_t*)q->data + q->bytes);
        v[e].q = (const int8_t*)qkeep.back().data();
        v[e].s = f32_of(sc, keep);
        v[e].rows = q->shape[0];
        v[e].cols = q->shape[1] * (dtype == 3 ? 2 : 1);
        v[e].dtype = dtype;
      }
    }
    lw.Wg_q = qws[(size_t)L * 3].data();
    lw.Wu_q = qws[(size_t)L * 3 + 1].data();
    lw.Wd_q = qws[(size_t)L * 3 + 2].data();
    lw.experts_quantized = 1;
  }
  w.layers = lws.data();
  return moe_model_create(&cfg, &w, max_seq, out);
}

moe_status moe_model_destroy(moe_model* m) {
  if (!m) return MOE_OK;
  free_model(m);
  return MOE_OK;
}

moe_status moe_model_config(const moe_model* m, QwenConfig* cfg) {
  if (!m || !cfg) return set_error(MOE_ERR_ARG, "model_config: null argument");
  *cfg = m->cfg;
  return MOE_OK;
}

moe_status moe_model_reset(moe_model* m) {
  if (!m) return set_error(MOE_ERR_ARG, "model_reset: null model");
  std::lock_guard<std::mutex> lk(m->mu);
  m->pos = 0;
  return MOE_OK;
}

int moe_model_position(const moe_model* m) { return m ? m->pos : -1; }

moe_status moe_model_forward(moe_model* m, const int32_t* ids, int T, int ids_on_device,
                             float* logits_dev, int32_t* next_dev) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!m || !ids) return set_error(MOE_ERR_ARG, "model_forward: null argument");
  std::lock_guard<std::mutex> lk(m->mu);
  return forward_checked(m, ids, T, ids_on_device, logits_dev, next_dev);
}

moe_status moe_model_forward_full(moe_model* m, const int32_t* ids, int T, int apply_softmax,
                                  float* out_last) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!m || !ids || !out_last) return set_error(MOE_ERR_ARG, "model_forward_full: null argument");
  std::lock_guard<std::mutex> lk(m->mu);
  m->pos = 0;
  if ((st = forward_checked(m, ids, T, 0, nullptr, nullptr))) return st;
  if (apply_softmax && (st = softmax_vec(m->logits, m->cfg.vocab_size, stream()))) return st;
  if ((st = check_hip(hipMemcpyAsync(out_last, m->logits, (size_t)m->cfg.vocab_size * 4,
                                     hipMemcpyDeviceToHost, stream()), "logits download")))
    return st;
  return check_hip(hipStreamSynchronize(stream()), "model_forward_full sync");
}

moe_status moe_model_generate(moe_model* m, const int32_t* prompt, int n_prompt, int n_new,
                              int32_t* out_ids, float* ms_prompt, float* ms_decode) {
  moe_status st = ensure_init();
  if (st) return st;
  if (!m || !prompt || !out_ids || n_prompt <= 0 || n_new <= 0)
    return set_error(MOE_ERR_ARG, "model_generate: bad argument");
  std::lock_guard<std::mutex> lk(m->mu);
  if (n_prompt + n_new - 1 > m->max_seq)
    return set_error(MOE_ERR_ARG, "model_generate: %d + %d tokens exceed max_seq %d", n_prompt,
                     n_new, m->max_seq);
  m->pos = 0;
  if ((st = grow(m->hist, (size_t)n_new * 4)) ||
      (st = check_hip(hipMemsetAsync(m->hist_pos, 0, 4, stream()), "generate counter")))
    return st;
  hipEvent_t e0, e1, e2;
  if ((st = check_hip(hipEventCreate(&e0), "event")) || (st = check_hip(hipEventCreate(&e1), "event")) ||
      (st = check_hip(hipEventCreate(&e2), "event")))
    return st;
  auto run = [&]() -> moe_status {
    moe_status s2;
    if ((s2 = ensure_scratch(m, n_prompt))) return s2;
    for (int t = 0; t < n_prompt; ++t)
      if (prompt[t] < 0 || prompt[t] >= m->cfg.vocab_size)
        return set_error(MOE_ERR_ARG, "model_generate: token id %d out of range", prompt[t]);
    if ((s2 = h2d(m->ids.p, prompt, (size_t)n_prompt * 4))) return s2;
    if ((s2 = check_hip(hipEventRecord(e0, stream()), "event"))) return s2;
    // prompt, then each chosen token fed back from device memory
    if ((s2 = forward_dev(m, (const int32_t*)m->ids.p, n_prompt, nullptr, nullptr, true))) return s2;
    if ((s2 = check_hip(hipEventRecord(e1, stream()), "event"))) return s2;
    for (int i = 1; i < n_new; ++i)
      if ((s2 = forward_dev(m, m->next, 1, nullptr, nullptr, true))) return s2;
    if ((s2 = check_hip(hipEventRecord(e2, stream()), "event"))) return s2;
    if ((s2 = check_hip(hipMemcpyAsync(out_ids, m->hist.p, (size_t)n_new * 4, hipMemcpyDeviceToHost,
                                       stream()), "generate download")))
      return s2;
    if ((s2 = check_hip(hipStreamSynchronize(stream()), "generate sync"))) return s2;
    float a = 0.0f, b2 = 0.0f;
    if ((s2 = check_hip(hipEventElapsedTime(&a, e0, e1), "event")) ||
        (s2 = check_hip(hipEventElapsedTime(&b2, e1, e2), "event")))
      return s2;
    if (ms_prompt) *ms_prompt = a;
    if (ms_decode) *ms_decode = b2;
    return MOE_OK;
  };
  st = run();
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipEventDestroy(e2);
  return st;
}

}  // extern "C"
