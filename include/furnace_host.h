/*
 * furnace_host.h -- host side above the engine ABI (C++ implementation,
 * C linkage).  furnace's Rust host does these steps itself; this library
 * restates them so the engine can be driven without Rust:
 *   GGUF mmap parsing          (src/gguf.rs:315-434)
 *   Config::from_gguf + load   (src/model.rs:41-60, 520-552) -> frn_upload
 *   the greedy token loop      (src/generate.rs:83-157)
 * plus a writer for seeded synthetic GGUF models (furnace ships no
 * quantizer; its block layouts, src/quant.rs:3-133, define the encoders).
 */
#ifndef FURNACE_HOST_H
#define FURNACE_HOST_H
#include "furnace_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct frn_gguf frn_gguf;

/* GgufFile::open (gguf.rs:366-380): read-only mmap + parse (gguf.rs:315-363). */
frn_status frn_gguf_open(const char* path, frn_gguf** out);
void frn_gguf_close(frn_gguf* g);
/* Config::from_gguf (model.rs:41-60); leaves cfg->max_ctx and
 * cfg->tied_lm_head from the tensor table (model.rs:541-545). */
frn_status frn_gguf_config(const frn_gguf* g, frn_config* cfg, uint32_t* context_length);
/* GgufFile::meta_u32 (gguf.rs:389-394) */
frn_status frn_gguf_meta_u32(const frn_gguf* g, const char* key, uint32_t* out);
/* GgufFile::tensor (gguf.rs:412-434): host pointer into the mapping. */
frn_status frn_gguf_tensor(const frn_gguf* g, const char* name, uint32_t* type, uint64_t dims[4], uint32_t* n_dims,
                           const void** data, size_t* bytes);

/* Model::load (model.rs:520-552) onto HIP device `device`: Config from the
 * metadata, one frn_upload per tensor of the model, frn_finalize.  flags are
 * FRN_FLAG_* of furnace_hip.h. */
frn_status frn_model_load(const frn_gguf* g, int device, uint32_t max_ctx, uint32_t flags, frn_ctx** out);

typedef struct frn_gen_stats {
  double prefill_s;      /* generate.rs:109-111 */
  double decode_s;       /* sum over timed decode forwards, :135-139 */
  uint32_t decode_steps; /* max_new - 1 unless a stop id ends the loop */
  uint32_t n_generated;
} frn_gen_stats;

/* generate (generate.rs:83-157) at temperature 0: prefill, then
 * sample (argmax) / stop check / decode, max_new samples and max_new - 1
 * timed decode forwards.  Writes up to max_new ids to out_ids.  The
 * context must be freshly reset; prompt + max_new must fit max_ctx. */
frn_status frn_generate_greedy(frn_ctx* ctx, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                               const uint32_t* stop_ids, uint32_t n_stop, uint32_t* out_ids, frn_gen_stats* stats);

/* generate (generate.rs:83-157) with the device sampler: prefill, then
 * sample with Sampler::new(temperature, top_k, top_p, repeat_penalty, seed)
 * over the last 64 context ids (generate.rs:123) / stop check / decode, as
 * frn_generate_greedy.  *draws receives Sampler::draws (may be NULL). */
frn_status frn_generate_sampled(frn_ctx* ctx, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                                float temperature, uint32_t top_k, float top_p, float repeat_penalty, uint64_t seed,
                                const uint32_t* stop_ids, uint32_t n_stop, uint32_t* out_ids, frn_gen_stats* stats,
                                uint64_t* draws);

/* ---- synthetic models ------------------------------------------------------ */
/* FRN_MIX_Q4_K_M: Q6_K attn_v / ffn_down on even layers; FRN_MIX_Q4_K_M_LLAMA:
 * llama.cpp's Q4_K_M rule for them (first and last eighth of the layers and
 * every third between) */
enum { FRN_MIX_ALL_Q8_0 = 0, FRN_MIX_Q4_K_M = 1, FRN_MIX_ALL_Q4_K = 2, FRN_MIX_ALL_Q6_K = 3, FRN_MIX_ALL_Q5_0 = 4,
       FRN_MIX_ALL_F32 = 5, FRN_MIX_Q4_K_M_LLAMA = 6, FRN_MIX_ALL_F16 = 7 };
typedef struct frn_synth_spec {
  uint32_t n_layers, n_heads, n_kv_heads, hidden, ffn, vocab, context_length;
  float rope_theta, rms_eps;
  uint32_t mix;          /* FRN_MIX_*: linear-weight types */
  uint32_t tied;         /* 1: no output.weight */
  uint32_t embd_type;    /* ggml type of token_embd.weight */
  uint32_t output_type;  /* ggml type of output.weight when untied */
  uint64_t seed;
  float weight_std;      /* N(0, std) for matrices and biases (0.02) */
  uint32_t threads;      /* 0: all hardware threads */
  uint32_t alignment;    /* 0: no general.alignment key (32); else a power of
                            two written as general.alignment, which the tensor
                            offsets and the data blob then follow */
} frn_synth_spec;
/* Writes a GGUF v3 file: qwen2 metadata, tokenizer stubs (vocab strings,
 * types, empty merges, eos 151645 / bos 151643 when in range), norm gains 1.0
 * (F32), biases and matrices drawn from N(0, std) per tensor from `seed`. */
frn_status frn_synth_write(const frn_synth_spec* spec, const char* path);
/* Encode n values (multiple of the block size) into ggml `type` blocks.
 * out must hold n / block * block_bytes bytes. */
frn_status frn_quantize(uint32_t type, const float* x, size_t n, uint8_t* out);
/* Seeded N(0, std) values, the generator frn_synth_write uses. */
frn_status frn_gaussian(uint64_t seed, float std, size_t n, float* out);

#ifdef __cplusplus
}
#endif
#endif
