// Host side of model loading and the greedy token loop (C ABI in
// include/furnace_host.h).  Config::from_gguf and Model::load restate furnace
// src/model.rs:41-60 and :520-552; frn_generate_greedy restates
// src/generate.rs:83-157 at temperature 0 over frn_prefill / frn_decode.
#include <stdio.h>
#include <string.h>
#include <time.h>

#include <string>
#include <vector>

#include "../../../include/furnace_host.h"
#include "../common.hpp"
#include "gguf.hpp"

struct frn_gguf {
  frn_host::File f;
};

extern "C" frn_status frn_gguf_open(const char* path, frn_gguf** out) {
  if (!path || !out) return frn_fail(FRN_EINVAL, "frn_gguf_open: null argument");
  *out = nullptr;
  frn_gguf* g = new frn_gguf();
  frn_status st = frn_host::open(path, &g->f);
  if (st) {
    delete g;
    return st;
  }
  *out = g;
  return FRN_OK;
}

extern "C" void frn_gguf_close(frn_gguf* g) { delete g; }

extern "C" frn_status frn_gguf_meta_u32(const frn_gguf* g, const char* key, uint32_t* out) {
  if (!g || !key || !out) return frn_fail(FRN_EINVAL, "frn_gguf_meta_u32: null argument");
  return frn_host::meta_u32(g->f, key, out);
}

extern "C" frn_status frn_gguf_tensor(const frn_gguf* g, const char* name, uint32_t* type, uint64_t dims[4],
                                      uint32_t* n_dims, const void** data, size_t* bytes) {
  if (!g || !name) return frn_fail(FRN_EINVAL, "frn_gguf_tensor: null argument");
  const frn_host::TensorInfo* t;
  const uint8_t* p;
  size_t b;
  frn_status st = frn_host::tensor(g->f, name, &t, &p, &b);
  if (st) return st;
  if (type) *type = t->type;
  if (n_dims) *n_dims = (uint32_t)t->dims.size();
  if (dims)
    for (int d = 0; d < 4; ++d) dims[d] = d < (int)t->dims.size() ? t->dims[d] : 1;
  if (data) *data = p;
  if (bytes) *bytes = b;
  return FRN_OK;
}

extern "C" frn_status frn_gguf_config(const frn_gguf* g, frn_config* c, uint32_t* context_length) {
  if (!g || !c) return frn_fail(FRN_EINVAL, "frn_gguf_config: null argument");
  const frn_host::File& f = g->f;
  auto arch = f.meta.find("general.architecture");
  if (arch == f.meta.end() || arch->second.tag != 8)
    return frn_fail(FRN_EINVAL, "metadata key 'general.architecture' missing or not a string");
  if (arch->second.s != "qwen2") return frn_fail(FRN_EINVAL, "architecture '%s' not supported", arch->second.s.c_str());
  frn_status st;
  uint32_t ctx_len = 0;
  if ((st = frn_host::meta_u32(f, "qwen2.attention.head_count", &c->n_heads)) ||
      (st = frn_host::meta_u32(f, "qwen2.embedding_length", &c->hidden)))
    return st;
  if (c->n_heads == 0 || c->hidden % c->n_heads)
    return frn_fail(FRN_ESHAPE, "hidden %u not divisible by %u heads", c->hidden, c->n_heads);
  if ((st = frn_host::meta_u32(f, "qwen2.block_count", &c->n_layers)) ||
      (st = frn_host::meta_u32(f, "qwen2.attention.head_count_kv", &c->n_kv_heads)) ||
      (st = frn_host::meta_u32(f, "qwen2.feed_forward_length", &c->ffn)) ||
      (st = frn_host::meta_f32(f, "qwen2.rope.freq_base", &c->rope_theta)) ||
      (st = frn_host::meta_f32(f, "qwen2.attention.layer_norm_rms_epsilon", &c->rms_eps)))
    return st;
  c->head_dim = c->hidden / c->n_heads;
  auto toks = f.meta.find("tokenizer.ggml.tokens");
  if (toks == f.meta.end() || toks->second.tag != 9)
    return frn_fail(FRN_EINVAL, "metadata key 'tokenizer.ggml.tokens' missing or not an array");
  c->vocab = (uint32_t)toks->second.arr_len;
  if ((st = frn_host::meta_u32(f, "qwen2.context_length", &ctx_len))) return st;
  if (context_length) *context_length = ctx_len;
  c->tied_lm_head = 1;
  for (const auto& t : f.tensors)
    if (t.name == "output.weight") c->tied_lm_head = 0;
  return FRN_OK;
}

extern "C" frn_status frn_model_load(const frn_gguf* g, int device, uint32_t max_ctx, uint32_t flags,
                                     frn_ctx** out) {
  if (!g || !out) return frn_fail(FRN_EINVAL, "frn_model_load: null argument");
  *out = nullptr;
  frn_config c{};
  frn_status st = frn_gguf_config(g, &c, nullptr);
  if (st) return st;
  c.max_ctx = max_ctx;
  c.flags = flags;
  frn_ctx* ctx = nullptr;
  if ((st = frn_create(&c, device, &ctx))) return st;
  // every tensor of the file goes up raw; finalize checks that the set
  // Model::load needs is present and consistently shaped
  for (const auto& t : g->f.tensors) {
    const frn_host::TensorInfo* info;
    const uint8_t* p;
    size_t bytes;
    if ((st = frn_host::tensor(g->f, t.name, &info, &p, &bytes))) break;
    // F16 (type 1) is an extension: the reference's Model::load rejects it
    // (src/quant.rs:279)
    if (t.type != 0 && t.type != 1 && t.type != 6 && t.type != 8 && t.type != 12 && t.type != 14) {
      st = frn_fail(FRN_EDTYPE, "tensor '%s': dequantization for ggml type %u is not implemented", t.name.c_str(), t.type);
      break;
    }
    uint64_t in = t.dims.empty() ? 1 : t.dims[0];
    if (in == 0) {  // a zero-length row would divide by zero below; Model::load errors on such shapes
      st = frn_fail(FRN_ESHAPE, "tensor '%s': dimension 0 is zero", t.name.c_str());
      break;
    }
    uint64_t outd = t.dims.size() > 1 ? t.n_elements() / in : 1;
    if ((st = frn_upload(ctx, t.name.c_str(), t.type, outd, in, p, bytes))) break;
  }
  if (!st) st = frn_finalize(ctx);
  if (st) {
    std::string msg = frn_last_error();
    frn_destroy(ctx);
    return frn_fail(st, "%s", msg.c_str());
  }
  *out = ctx;
  return FRN_OK;
}

static double now_s() {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + ts.tv_nsec * 1e-9;
}

extern "C" frn_status frn_generate_greedy(frn_ctx* ctx, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                                          const uint32_t* stop_ids, uint32_t n_stop, uint32_t* out_ids,
                                          frn_gen_stats* stats) {
  if (!ctx || !prompt || !out_ids) return frn_fail(FRN_EINVAL, "frn_generate_greedy: null argument");
  frn_gen_stats s{};
  uint32_t next = 0;
  double t0 = now_s();
  frn_status st = frn_prefill(ctx, prompt, n_prompt, &next);
  if (st) return st;
  s.prefill_s = now_s() - t0;
  if ((st = frn_timings_reset(ctx))) return st;  // generate.rs:119: the breakdown covers decode only
  auto is_stop = [&](uint32_t id) {
    for (uint32_t i = 0; i < n_stop; ++i)
      if (stop_ids[i] == id) return true;
    return false;
  };
  // generate.rs:122-141: sample (the prefill's argmax), stop on eos/bos,
  // push, then one forward per further token -- here all of them in one
  // frn_decode_greedy call, which ends after a step whose argmax is a stop id
  if (max_new > 0 && !is_stop(next)) {
    out_ids[s.n_generated++] = next;
    if (max_new > 1) {
      uint32_t done = 0;
      double t1 = now_s();
      if ((st = frn_decode_greedy(ctx, next, max_new - 1, stop_ids, n_stop, out_ids + 1, &done))) return st;
      s.decode_s = now_s() - t1;
      s.decode_steps = done;
      s.n_generated += done;
      if (done && is_stop(out_ids[done])) s.n_generated -= 1;  // the stop id is not pushed
    }
  }
  if (stats) *stats = s;
  return FRN_OK;
}

extern "C" frn_status frn_generate_sampled(frn_ctx* ctx, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                                           float temperature, uint32_t top_k, float top_p, float repeat_penalty,
                                           uint64_t seed, const uint32_t* stop_ids, uint32_t n_stop, uint32_t* out_ids,
                                           frn_gen_stats* stats, uint64_t* draws) {
  if (!ctx || !prompt || !out_ids) return frn_fail(FRN_EINVAL, "frn_generate_sampled: null argument");
  frn_status st = frn_sampler_init(ctx, temperature, top_k, top_p, repeat_penalty, seed);
  if (st) return st;
  frn_gen_stats s{};
  const uint32_t window = 64;  // Sampler::repeat_window (sampler.rs:75)
  std::vector<uint32_t> context(prompt, prompt + n_prompt);
  uint32_t next = 0;
  double t0 = now_s();
  if ((st = frn_prefill(ctx, prompt, n_prompt, &next))) return st;
  s.prefill_s = now_s() - t0;
  if ((st = frn_timings_reset(ctx))) return st;  // generate.rs:119: the breakdown covers decode only
  for (uint32_t step = 0; step < max_new; ++step) {
    const size_t w = context.size() > window ? context.size() - window : 0;  // generate.rs:123
    if ((st = frn_sample(ctx, context.data() + w, (uint32_t)(context.size() - w), &next))) return st;
    bool stop = false;
    for (uint32_t i = 0; i < n_stop; ++i) stop |= stop_ids[i] == next;
    if (stop) break;
    out_ids[s.n_generated++] = next;
    context.push_back(next);
    if (step + 1 == max_new) break;
    double t1 = now_s();
    if ((st = frn_decode(ctx, next, nullptr))) return st;
    s.decode_s += now_s() - t1;
    s.decode_steps += 1;
  }
  if (stats) *stats = s;
  if (draws && (st = frn_sampler_draws(ctx, draws))) return st;
  return FRN_OK;
}
