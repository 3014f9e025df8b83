/* Test infrastructure only (the oracle).  Restates src/model.rs (Config,
 * Weight, Layer, linear, KvCache, layer_forward[_cached], embed, Model::load,
 * forward_cached, forward_last, last_row_logits) and the temperature-0 path
 * of src/generate.rs::generate. */
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include "oracle.h"
#include "oracle_gguf.h"
#include "oracle_internal.h"

void orc_attention_scores_cached(const float* q, size_t n_new, const float* k_cache, size_t total,
                                 size_t start_pos, size_t nh, size_t nkv, size_t hd, float* probs);
void orc_attention_apply_cached(const float* probs, size_t n_new, size_t total, const float* v_cache,
                                size_t nh, size_t nkv, size_t hd, float* out);

static int g_threads = 0;
void orc_set_threads(int n) {
  g_threads = n;
  if (n > 0) omp_set_num_threads(n);
}
int orc_get_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

/* model.rs:66-74 Weight */
typedef struct {
  int is_f32;
  const float* f32; /* [out, in] */
  float* owned;
  const uint8_t* raw;
  size_t raw_len;
  uint32_t type;
  size_t out, in;
} weight_t;

typedef struct { /* model.rs:130-143 Layer */
  const float *attn_norm, *bq, *bk, *bv, *ffn_norm;
  weight_t wq, wk, wv, wo, w_gate, w_up, w_down;
} layer_t;

struct orc_model {
  gguf_file g;
  orc_config c;
  weight_t embedding, lm_head;
  layer_t* layers;
  const float* output_norm;
  float** owned; /* f32 copies of norm/bias tensors */
  size_t n_owned;
};

struct orc_cache { /* model.rs:321-327 */
  float* k; /* [L][max_ctx * kv_dim] */
  float* v;
  size_t len, max_ctx, kv_dim, n_layers;
};

/* model.rs:99-106 Weight::matmul */
static int weight_matmul(const weight_t* w, const float* x, size_t seq, float* out) {
  if (w->is_f32) {
    orc_matmul_f32(x, seq, w->f32, w->out, w->in, out);
    return 0;
  }
  return orc_matmul_quant(x, seq, w->raw, w->raw_len, w->out, w->in, w->type, out);
}

/* model.rs:169-186 linear: matmul, then the bias added per row. */
static int linear(const float* x, size_t seq, const weight_t* w, const float* bias, float* out) {
  if (weight_matmul(w, x, seq, out)) return -1;
  if (bias)
    for (size_t s = 0; s < seq; ++s)
      for (size_t o = 0; o < w->out; ++o) out[s * w->out + o] += bias[o];
  return 0;
}

/* model.rs:444-478 layer_forward_cached.  k_cache/v_cache point at this
 * layer's [max_ctx * kv_dim] buffers. */
static int layer_forward_cached(const float* x, size_t n_new, const layer_t* L, const orc_config* c,
                                float* k_cache, float* v_cache, size_t max_ctx, size_t start_pos, float* out) {
  size_t H = c->hidden, nh = c->n_heads, nkv = c->n_kv_heads, hd = c->head_dim, F = c->ffn;
  size_t qd = nh * hd, kd = nkv * hd, total = start_pos + n_new;
  if (start_pos + n_new > max_ctx) {
    orc_set_error("kv cache overflow: %zu + %zu > max_ctx %zu", start_pos, n_new, max_ctx);
    return -1;
  }
  float* xn = malloc(n_new * H * 4);
  float* q = malloc(n_new * qd * 4);
  float* k = malloc(n_new * kd * 4);
  float* v = malloc(n_new * kd * 4);
  float* probs = malloc(nh * n_new * total * 4);
  float* ctx = malloc(n_new * qd * 4);
  float* attn = malloc(n_new * H * 4);
  float* h1 = malloc(n_new * H * 4);
  float* gate = malloc(n_new * F * 4);
  float* up = malloc(n_new * F * 4);
  float* act = malloc(n_new * F * 4);
  float* ffn = malloc(n_new * H * 4);
  int rc = -1;
  orc_rmsnorm(x, n_new, H, L->attn_norm, c->rms_eps, xn);
  if (linear(xn, n_new, &L->wq, L->bq, q) || linear(xn, n_new, &L->wk, L->bk, k) ||
      linear(xn, n_new, &L->wv, L->bv, v))
    goto done;
  orc_rope(q, n_new, nh, hd, c->rope_theta, start_pos);
  orc_rope(k, n_new, nkv, hd, c->rope_theta, start_pos);
  memcpy(k_cache + start_pos * kd, k, n_new * kd * 4); /* KvCache::append, :346-356 */
  memcpy(v_cache + start_pos * kd, v, n_new * kd * 4);
  orc_attention_scores_cached(q, n_new, k_cache, total, start_pos, nh, nkv, hd, probs);
  orc_attention_apply_cached(probs, n_new, total, v_cache, nh, nkv, hd, ctx);
  if (linear(ctx, n_new, &L->wo, NULL, attn)) goto done;
  orc_add(x, attn, n_new * H, h1);
  orc_rmsnorm(h1, n_new, H, L->ffn_norm, c->rms_eps, xn);
  if (linear(xn, n_new, &L->w_gate, NULL, gate) || linear(xn, n_new, &L->w_up, NULL, up)) goto done;
  orc_swiglu(gate, up, n_new * F, act);
  if (linear(act, n_new, &L->w_down, NULL, ffn)) goto done;
  orc_add(h1, ffn, n_new * H, out);
  rc = 0;
done:
  free(xn); free(q); free(k); free(v); free(probs); free(ctx); free(attn); free(h1);
  free(gate); free(up); free(act); free(ffn);
  return rc;
}

/* model.rs:294-315 layer_forward (uncached): positions 0..seq, full causal
 * attention over the block's own K/V.  Same dots in the same order as the
 * cached path, which is why cached == uncached holds bit for bit. */
static int layer_forward(const float* x, size_t seq, const layer_t* L, const orc_config* c, float* out) {
  size_t kd = c->n_kv_heads * c->head_dim;
  float* kc = calloc(seq * kd, 4);
  float* vc = calloc(seq * kd, 4);
  int rc = layer_forward_cached(x, seq, L, c, kc, vc, seq, 0, out);
  free(kc);
  free(vc);
  return rc;
}

static weight_t f32_weight(const float* w, size_t out, size_t in) {
  weight_t r;
  memset(&r, 0, sizeof r);
  r.is_f32 = 1;
  r.f32 = w;
  r.out = out;
  r.in = in;
  return r;
}

static layer_t layer_from_f32(const orc_f32_layer* l, const orc_config* c) {
  size_t H = c->hidden, F = c->ffn, qd = c->n_heads * c->head_dim, kd = c->n_kv_heads * c->head_dim;
  layer_t L;
  L.attn_norm = l->attn_norm; L.bq = l->bq; L.bk = l->bk; L.bv = l->bv; L.ffn_norm = l->ffn_norm;
  L.wq = f32_weight(l->wq, qd, H);
  L.wk = f32_weight(l->wk, kd, H);
  L.wv = f32_weight(l->wv, kd, H);
  L.wo = f32_weight(l->wo, H, qd);
  L.w_gate = f32_weight(l->w_gate, F, H);
  L.w_up = f32_weight(l->w_up, F, H);
  L.w_down = f32_weight(l->w_down, H, F);
  return L;
}

void orc_layer_forward_f32(const float* x, size_t seq, const orc_f32_layer* l, const orc_config* c, float* out) {
  layer_t L = layer_from_f32(l, c);
  layer_forward(x, seq, &L, c, out);
}

void orc_layer_forward_cached_f32(const float* x, size_t n_new, const orc_f32_layer* l, const orc_config* c,
                                  float* k_cache, float* v_cache, size_t max_ctx, size_t start_pos, float* out) {
  layer_t L = layer_from_f32(l, c);
  layer_forward_cached(x, n_new, &L, c, k_cache, v_cache, max_ctx, start_pos, out);
}

/* ---- loading ------------------------------------------------------------ */

static float* own(orc_model* m, size_t n) {
  float* p = malloc(n * 4 + 4);
  m->owned = realloc(m->owned, (m->n_owned + 1) * sizeof(float*));
  m->owned[m->n_owned++] = p;
  return p;
}

static size_t n_elems(const gguf_tensor* t) {
  size_t n = 1;
  for (uint32_t d = 0; d < t->n_dims; ++d) n *= (size_t)t->dims[d];
  return n;
}

/* tensor.rs:55-60 Tensor::from_gguf, with the shape check its users make */
static const float* load_f32(orc_model* m, const char* name, size_t expect) {
  const gguf_tensor* t = gguf_find_tensor(&m->g, name);
  if (!t) { orc_set_error("no tensor named '%s'", name); return NULL; }
  const uint8_t* p;
  size_t bytes, n = n_elems(t);
  if (gguf_tensor_data(&m->g, t, &p, &bytes)) return NULL;
  if (n != expect) { orc_set_error("tensor '%s' has %zu elements, expected %zu", name, n, expect); return NULL; }
  float* o = own(m, n);
  if (orc_dequantize(t->type, p, bytes, n, o)) return NULL;
  return o;
}

/* model.rs:112-126 load_weight */
static int load_weight(orc_model* m, const char* name, weight_t* w) {
  memset(w, 0, sizeof *w);
  const gguf_tensor* t = gguf_find_tensor(&m->g, name);
  if (!t) { orc_set_error("no tensor named '%s'", name); return -1; }
  const uint8_t* p;
  size_t bytes;
  if (gguf_tensor_data(&m->g, t, &p, &bytes)) return -1;
  int fused = t->type == ORC_Q8_0 || t->type == ORC_Q5_0 || t->type == ORC_Q4_K || t->type == ORC_Q6_K;
  if (!fused) {
    size_t n = n_elems(t);
    float* o = own(m, n);
    if (orc_dequantize(t->type, p, bytes, n, o)) return -1;
    w->is_f32 = 1;
    w->f32 = o;
    w->in = (size_t)t->dims[0];
    w->out = t->n_dims > 1 ? (size_t)t->dims[1] : 1;
    return 0;
  }
  if (t->n_dims != 2) { orc_set_error("weight '%s' is not 2-D", name); return -1; }
  w->raw = p;
  w->raw_len = bytes;
  w->type = t->type;
  w->out = (size_t)t->dims[1];
  w->in = (size_t)t->dims[0];
  return 0;
}

static int check_dims(const weight_t* w, size_t out, size_t in, const char* what) {
  if (w->out != out || w->in != in) {
    orc_set_error("%s is [%zu, %zu], expected [%zu, %zu]", what, w->out, w->in, out, in);
    return -1;
  }
  return 0;
}

/* model.rs:41-60 Config::from_gguf */
static int config_from_gguf(const gguf_file* g, orc_config* c) {
  const gguf_kv* arch = gguf_find(g, "general.architecture");
  if (!arch || arch->type != 8) { orc_set_error("metadata key 'general.architecture' missing or not a string"); return -1; }
  if (arch->str_len != 5 || memcmp(arch->str, "qwen2", 5)) { orc_set_error("architecture not supported"); return -1; }
  if (gguf_u32(g, "qwen2.attention.head_count", &c->n_heads) ||
      gguf_u32(g, "qwen2.embedding_length", &c->hidden))
    return -1;
  if (c->n_heads == 0 || c->hidden % c->n_heads) {
    orc_set_error("hidden %u not divisible by %u heads", c->hidden, c->n_heads);
    return -1;
  }
  if (gguf_u32(g, "qwen2.block_count", &c->n_layers) ||
      gguf_u32(g, "qwen2.attention.head_count_kv", &c->n_kv_heads) ||
      gguf_u32(g, "qwen2.feed_forward_length", &c->ffn) ||
      gguf_f32(g, "qwen2.rope.freq_base", &c->rope_theta) ||
      gguf_f32(g, "qwen2.attention.layer_norm_rms_epsilon", &c->rms_eps))
    return -1;
  c->head_dim = c->hidden / c->n_heads;
  const gguf_kv* toks = gguf_find(g, "tokenizer.ggml.tokens");
  if (!toks || toks->type != 9) { orc_set_error("metadata key 'tokenizer.ggml.tokens' missing or not an array"); return -1; }
  c->vocab = (uint32_t)toks->arr_len;
  if (gguf_u32(g, "qwen2.context_length", &c->context_length)) return -1;
  if (c->n_kv_heads == 0 || c->n_heads % c->n_kv_heads) {
    orc_set_error("%u q heads not divisible by %u kv heads", c->n_heads, c->n_kv_heads);
    return -1;
  }
  return 0;
}

void orc_model_free(orc_model* m) {
  if (!m) return;
  for (size_t i = 0; i < m->n_owned; ++i) free(m->owned[i]);
  free(m->owned);
  free(m->layers);
  gguf_close(&m->g);
  free(m);
}

/* model.rs:520-552 Model::load */
orc_model* orc_model_load(const char* path) {
  orc_model* m = calloc(1, sizeof *m);
  if (gguf_open(path, &m->g) || config_from_gguf(&m->g, &m->c)) { orc_model_free(m); return NULL; }
  orc_config* c = &m->c;
  size_t H = c->hidden, qd = c->n_heads * c->head_dim, kd = c->n_kv_heads * c->head_dim;
  if (load_weight(m, "token_embd.weight", &m->embedding) ||
      check_dims(&m->embedding, c->vocab, H, "token_embd")) { orc_model_free(m); return NULL; }
  m->layers = calloc(c->n_layers ? c->n_layers : 1, sizeof(layer_t));
  char nm[128];
  for (uint32_t i = 0; i < c->n_layers; ++i) { /* Layer::load, :146-163 */
    layer_t* L = &m->layers[i];
#define F32T(field, suffix, n) \
    snprintf(nm, sizeof nm, "blk.%u." suffix, i); if (!(L->field = load_f32(m, nm, n))) goto fail;
#define WT(field, suffix, o, in_) \
    snprintf(nm, sizeof nm, "blk.%u." suffix, i); if (load_weight(m, nm, &L->field) || check_dims(&L->field, o, in_, nm)) goto fail;
    F32T(attn_norm, "attn_norm.weight", H)
    WT(wq, "attn_q.weight", qd, H)
    F32T(bq, "attn_q.bias", qd)
    WT(wk, "attn_k.weight", kd, H)
    F32T(bk, "attn_k.bias", kd)
    WT(wv, "attn_v.weight", kd, H)
    F32T(bv, "attn_v.bias", kd)
    WT(wo, "attn_output.weight", H, qd)
    F32T(ffn_norm, "ffn_norm.weight", H)
    WT(w_gate, "ffn_gate.weight", c->ffn, H)
    WT(w_up, "ffn_up.weight", c->ffn, H)
    WT(w_down, "ffn_down.weight", H, c->ffn)
#undef F32T
#undef WT
  }
  if (!(m->output_norm = load_f32(m, "output_norm.weight", H))) goto fail;
  /* tied embeddings when output.weight is absent, :541-545 */
  if (load_weight(m, gguf_find_tensor(&m->g, "output.weight") ? "output.weight" : "token_embd.weight",
                  &m->lm_head) ||
      check_dims(&m->lm_head, c->vocab, H, "lm_head"))
    goto fail;
  return m;
fail:
  orc_model_free(m);
  return NULL;
}

int orc_model_get_config(const orc_model* m, orc_config* out) {
  *out = m->c;
  return 0;
}

int64_t orc_model_meta_u32(const orc_model* m, const char* key) {
  uint32_t v;
  return gguf_u32(&m->g, key, &v) ? -1 : (int64_t)v;
}

int orc_model_tensor(const orc_model* m, const char* name, uint32_t* type, uint64_t dims[4], uint32_t* n_dims,
                     const uint8_t** data, size_t* bytes) {
  const gguf_tensor* t = gguf_find_tensor(&m->g, name);
  if (!t) { orc_set_error("no tensor named '%s'", name); return -1; }
  *type = t->type;
  *n_dims = t->n_dims;
  for (int d = 0; d < 4; ++d) dims[d] = d < (int)t->n_dims ? t->dims[d] : 1;
  return gguf_tensor_data(&m->g, t, data, bytes);
}

static size_t wbytes(const weight_t* w) { return w->is_f32 ? w->out * w->in * 4 : w->raw_len; }
size_t orc_model_param_bytes(const orc_model* m) { /* model.rs:555-563 */
  const orc_config* c = &m->c;
  size_t total = 0, qd = c->n_heads * c->head_dim, kd = c->n_kv_heads * c->head_dim;
  for (uint32_t i = 0; i < c->n_layers; ++i) {
    const layer_t* L = &m->layers[i];
    total += wbytes(&L->wq) + wbytes(&L->wk) + wbytes(&L->wv) + wbytes(&L->wo) + wbytes(&L->w_gate) +
             wbytes(&L->w_up) + wbytes(&L->w_down) + (c->hidden + qd + kd + kd + c->hidden) * 4;
  }
  return total + wbytes(&m->embedding) + c->hidden * 4 + wbytes(&m->lm_head);
}

/* ---- KV cache and forward ----------------------------------------------- */

orc_cache* orc_cache_new(const orc_model* m, size_t max_ctx) {
  orc_cache* c = calloc(1, sizeof *c);
  c->kv_dim = (size_t)m->c.n_kv_heads * m->c.head_dim;
  c->n_layers = m->c.n_layers;
  c->max_ctx = max_ctx;
  c->k = calloc(c->n_layers * max_ctx * c->kv_dim + 1, 4);
  c->v = calloc(c->n_layers * max_ctx * c->kv_dim + 1, 4);
  if (!c->k || !c->v) { orc_cache_free(c); orc_set_error("kv cache allocation failed"); return NULL; }
  return c;
}
void orc_cache_free(orc_cache* c) {
  if (!c) return;
  free(c->k);
  free(c->v);
  free(c);
}
size_t orc_cache_len(const orc_cache* c) { return c->len; }
int orc_cache_read(const orc_cache* c, size_t layer, int which_v, size_t n, float* out) {
  if (layer >= c->n_layers || n > c->max_ctx) { orc_set_error("cache read out of range"); return -1; }
  const float* src = (which_v ? c->v : c->k) + layer * c->max_ctx * c->kv_dim;
  memcpy(out, src, n * c->kv_dim * 4);
  return 0;
}

/* model.rs:482-506 embed */
static int embed(const orc_model* m, const uint32_t* tokens, size_t n, float* out) {
  const weight_t* e = &m->embedding;
  size_t H = m->c.hidden;
  for (size_t s = 0; s < n; ++s) {
    size_t t = tokens[s];
    if (t >= e->out) { orc_set_error("token id %zu out of range (vocab %zu)", t, e->out); return -1; }
    if (e->is_f32) {
      memcpy(out + s * H, e->f32 + t * H, H * 4);
    } else {
      size_t be, bb;
      orc_block_layout(e->type, &be, &bb);
      size_t row_bytes = H / be * bb;
      if (orc_dequantize(e->type, e->raw + t * row_bytes, row_bytes, H, out + s * H)) return -1;
    }
  }
  return 0;
}

/* model.rs:594-600 last_row_logits: rmsnorm, last row, lm_head */
static int last_row_logits(const orc_model* m, const float* x, size_t n, float* logits) {
  size_t H = m->c.hidden;
  float* xn = malloc(H * 4);
  orc_rmsnorm(x + (n - 1) * H, 1, H, m->output_norm, m->c.rms_eps, xn);
  int rc = linear(xn, 1, &m->lm_head, NULL, logits);
  free(xn);
  return rc;
}

static int run_layers(const orc_model* m, orc_cache* c, const uint32_t* tokens, size_t n, float* x) {
  size_t H = m->c.hidden;
  if (c->len + n > c->max_ctx) {
    orc_set_error("context overflow: %zu + %zu > max_ctx %zu", c->len, n, c->max_ctx);
    return -1;
  }
  if (embed(m, tokens, n, x)) return -1;
  float* y = malloc(n * H * 4);
  for (uint32_t i = 0; i < m->c.n_layers; ++i) {
    float* kc = c->k + (size_t)i * c->max_ctx * c->kv_dim;
    float* vc = c->v + (size_t)i * c->max_ctx * c->kv_dim;
    if (layer_forward_cached(x, n, &m->layers[i], &m->c, kc, vc, c->max_ctx, c->len, y)) { free(y); return -1; }
    memcpy(x, y, n * H * 4);
  }
  free(y);
  c->len += n;
  return 0;
}

/* model.rs:579-592 forward_cached */
int orc_forward_cached(const orc_model* m, orc_cache* c, const uint32_t* tokens, size_t n, float* logits) {
  if (n == 0) { orc_set_error("forward_cached: empty token list"); return -1; }
  float* x = malloc(n * m->c.hidden * 4);
  int rc = run_layers(m, c, tokens, n, x);
  if (!rc) rc = last_row_logits(m, x, n, logits);
  free(x);
  return rc;
}

int orc_forward_cached_hidden(const orc_model* m, orc_cache* c, const uint32_t* tokens, size_t n, float* hidden_last) {
  if (n == 0) { orc_set_error("forward_cached: empty token list"); return -1; }
  float* x = malloc(n * m->c.hidden * 4);
  int rc = run_layers(m, c, tokens, n, x);
  if (!rc) memcpy(hidden_last, x + (n - 1) * m->c.hidden, m->c.hidden * 4);
  free(x);
  return rc;
}

/* model.rs:569-575 forward_last */
int orc_forward_last(const orc_model* m, const uint32_t* tokens, size_t n, float* logits) {
  size_t H = m->c.hidden;
  if (n == 0) { orc_set_error("forward_last: empty token list"); return -1; }
  float* x = malloc(n * H * 4);
  float* y = malloc(n * H * 4);
  int rc = embed(m, tokens, n, x);
  for (uint32_t i = 0; !rc && i < m->c.n_layers; ++i) {
    rc = layer_forward(x, n, &m->layers[i], &m->c, y);
    memcpy(x, y, n * H * 4);
  }
  if (!rc) rc = last_row_logits(m, x, n, logits);
  free(x);
  free(y);
  return rc;
}

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + ts.tv_nsec * 1e-9;
}

/* generate.rs:83-157 at temperature 0 (sampler.rs:91-94 short-circuits to
 * argmax; repeat penalty 1.0 is a no-op, :39-42). */
long orc_generate_greedy(const orc_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                         size_t max_ctx, const uint32_t* stop_ids, size_t n_stop, uint32_t* out_ids,
                         double* prefill_s, double* decode_s, size_t* decode_steps, float* last_logits) {
  if (n_prompt + max_new > max_ctx) {
    orc_set_error("prompt (%zu) + max tokens (%zu) exceeds context cap %zu", n_prompt, max_new, max_ctx);
    return -1;
  }
  orc_cache* c = orc_cache_new(m, max_ctx);
  if (!c) return -1;
  size_t V = m->c.vocab;
  float* logits = malloc(V * 4);
  double t0 = now_s();
  if (orc_forward_cached(m, c, prompt, n_prompt, logits)) { free(logits); orc_cache_free(c); return -1; }
  *prefill_s = now_s() - t0;
  double dec = 0.0;
  size_t steps = 0;
  long n_gen = 0;
  for (size_t step = 0; step < max_new; ++step) {
    uint32_t next = orc_argmax(logits, V);
    int stop = 0;
    for (size_t i = 0; i < n_stop; ++i) stop |= stop_ids[i] == next;
    if (stop) break;
    out_ids[n_gen++] = next;
    if (step + 1 == max_new) break;
    double t1 = now_s();
    if (orc_forward_cached(m, c, &next, 1, logits)) { free(logits); orc_cache_free(c); return -1; }
    dec += now_s() - t1;
    ++steps;
  }
  *decode_s = dec;
  *decode_steps = steps;
  if (last_logits) memcpy(last_logits, logits, V * 4);
  free(logits);
  orc_cache_free(c);
  return n_gen;
}
