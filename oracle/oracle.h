/*
 * oracle.h -- CPU restatement of furnace's token loop, used ONLY as the
 * test oracle: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it.  The product (furnace_amd/) never links, loads or calls it.
 *
 * Every function restates one reference function and cites it (paths are
 * relative to the furnace source tree).  Arithmetic order follows the Rust
 * code exactly: separate multiply and add (no FMA contraction -- the recipe
 * builds with -ffp-contract=off), the same accumulator grouping (8-lane dot,
 * sequential sums), the same glibc expf/powf/sinf/cosf calls that Rust's std
 * lowers to on linux-gnu.
 *
 * Parity pins (see tests/test_oracle_*.py): every dequantizer against the
 * reference's hand-computed known-answer tests plus closed-form checks;
 * fused matmul against dequantize-then-f64-dot; rmsnorm/softmax/swiglu/rope
 * against the reference's hand values; attention against the causal-mask,
 * GQA-routing and cached==uncached bit-identity invariants; argmax against
 * the first-max tie rule.  Nothing here is "parity unpinned" except the
 * last-ulp behaviour of glibc's libm versus Rust's (identical library calls,
 * so expected bit-equal, but only pinnable by running compiled furnace).
 */
#ifndef FURNACE_ORACLE_H
#define FURNACE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml on-disk type codes, src/gguf.rs:180-201 */
enum {
  ORC_F32 = 0, ORC_F16 = 1, ORC_Q5_0 = 6, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14
};

/* ---- quant.rs ---------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h);                                  /* half 2.7.1 f16::to_f32 */
int orc_block_layout(uint32_t type, size_t* elems, size_t* bytes); /* gguf.rs:206-216 */
/* quant.rs:261-281 -- returns 0, or -1 with orc_last_error() set */
int orc_dequantize(uint32_t type, const uint8_t* raw, size_t raw_len, size_t n, float* out);
/* quant.rs:170-193 (+ tensor.rs:86-137 loop structure).  a is [seq, d_in],
 * out is [seq, d_out].  Panics in the reference become return -1. */
int orc_matmul_quant(const float* a, size_t seq, const uint8_t* raw, size_t raw_len,
                     size_t d_out, size_t d_in, uint32_t type, float* out);
/* tensor.rs:74-80: f32 weights [d_out, d_in] */
void orc_matmul_f32(const float* a, size_t seq, const float* w, size_t d_out, size_t d_in, float* out);

/* Beyond the reference: F16 tensors widen exactly to f32 in orc_dequantize
 * (and so load as f32 weights) while switched on; off (the default), F16 is
 * the reference's "not implemented" error (quant.rs:279). */
void orc_set_f16_extension(int on);

/* ---- tensor.rs --------------------------------------------------------- */
float orc_dot(const float* a, const float* b, size_t n);                             /* :146-160 */
void orc_rmsnorm(const float* x, size_t rows, size_t cols, const float* w, float eps, float* out); /* :164-185 */
void orc_softmax(float* x, size_t rows, size_t cols);                                /* :188-203 */
void orc_silu(const float* x, size_t n, float* out);                                 /* :207-210 */
void orc_swiglu(const float* gate, const float* up, size_t n, float* out);           /* :213-227 */
void orc_add(const float* a, const float* b, size_t n, float* out);                  /* :229-234 */

/* ---- model.rs ops ------------------------------------------------------ */
void orc_rope(float* x, size_t seq, size_t n_heads, size_t head_dim, float theta, size_t start_pos); /* :193-217 */
/* :224-258 -- probs [n_heads, seq, seq] */
void orc_attention_scores(const float* q, const float* k, size_t seq, size_t n_heads,
                          size_t n_kv_heads, size_t head_dim, float* probs);
/* :262-290 -- out [seq, n_heads*head_dim] */
void orc_attention_apply(const float* probs, const float* v, size_t seq, size_t n_heads,
                         size_t n_kv_heads, size_t head_dim, float* out);

/* ---- generate.rs ------------------------------------------------------- */
uint32_t orc_argmax(const float* x, size_t n); /* :69-77 */

/* ---- sampler.rs --------------------------------------------------------- */
typedef struct orc_pcg32 {
  uint64_t state, inc;
} orc_pcg32;
/* O'Neill's pcg32_srandom_r; Pcg32::new(seed) = (seed, 0xda3e39cb94b95bdb) (:11-17) */
void orc_pcg32_seed(orc_pcg32* r, uint64_t initstate, uint64_t initseq);
uint32_t orc_pcg32_next_u32(orc_pcg32* r); /* :20-28 */
float orc_pcg32_next_f32(orc_pcg32* r);    /* :31-33 */
void orc_apply_repeat_penalty(float* logits, const uint32_t* recent, size_t n_recent, float penalty); /* :39-55 */
typedef struct orc_sampler {               /* Sampler (:57-66) */
  float temperature;
  uint32_t top_k; /* 0 disables the cut */
  float top_p;    /* 1.0 disables the cut */
  float repeat_penalty;
  uint32_t repeat_window;
  orc_pcg32 rng;
  uint64_t draws;
} orc_sampler;
void orc_sampler_new(orc_sampler* s, float temperature, uint32_t top_k, float top_p, float repeat_penalty,
                     uint64_t seed); /* :68-78 */
/* :117-155: (id, prob) by descending prob into ids/probs (room for n); returns the count */
size_t orc_sampler_filtered(const orc_sampler* s, const float* logits, size_t n, uint32_t* ids, float* probs);
/* :86-108 */
uint32_t orc_sampler_sample(orc_sampler* s, const float* logits, size_t n, const uint32_t* recent,
                            size_t n_recent);

/* ---- GGUF (gguf.rs) and model (model.rs) -------------------------------- */
typedef struct orc_config {            /* model.rs:26-38 */
  uint32_t n_layers, n_heads, n_kv_heads, hidden, ffn, head_dim, vocab, context_length;
  float rope_theta, rms_eps;
} orc_config;

typedef struct orc_model orc_model;
typedef struct orc_cache orc_cache;

/* Model::load (model.rs:520-552) over GgufFile::open (gguf.rs:366-380). */
orc_model* orc_model_load(const char* gguf_path);
void orc_model_free(orc_model* m);
int orc_model_get_config(const orc_model* m, orc_config* out);
/* eos/bos ids from tokenizer metadata (main.rs:246-249); -1 if absent */
int64_t orc_model_meta_u32(const orc_model* m, const char* key);
/* Raw tensor lookup (GgufFile::tensor, gguf.rs:412-434). */
int orc_model_tensor(const orc_model* m, const char* name, uint32_t* type, uint64_t dims[4],
                     uint32_t* n_dims, const uint8_t** data, size_t* bytes);
size_t orc_model_param_bytes(const orc_model* m); /* model.rs:555-563 */

/* KvCache (model.rs:321-363); max_ctx positions. */
orc_cache* orc_cache_new(const orc_model* m, size_t max_ctx);
void orc_cache_free(orc_cache* c);
size_t orc_cache_len(const orc_cache* c);
/* Read back one layer's cached K or V rows [0, n) (kv_dim floats each). */
int orc_cache_read(const orc_cache* c, size_t layer, int which_v, size_t n, float* out);

/* Model::forward_cached (model.rs:579-592): logits [vocab] of the last row. */
int orc_forward_cached(const orc_model* m, orc_cache* c, const uint32_t* tokens, size_t n, float* logits);
/* Model::forward_last (model.rs:569-575): uncached full recompute. */
int orc_forward_last(const orc_model* m, const uint32_t* tokens, size_t n, float* logits);
/* Final hidden state of the last row after all layers, before output norm
 * (debug aid for staged checks). */
int orc_forward_cached_hidden(const orc_model* m, orc_cache* c, const uint32_t* tokens, size_t n,
                              float* hidden_last);

/* generate (generate.rs:83-157) at temperature 0: prefill, then greedy
 * sample/decode.  Returns the number of generated ids written to out_ids;
 * prefill_s / decode_s receive the wall times as generate measures them. */
long orc_generate_greedy(const orc_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                         size_t max_ctx, const uint32_t* stop_ids, size_t n_stop, uint32_t* out_ids,
                         double* prefill_s, double* decode_s, size_t* decode_steps, float* last_logits);

/* Thread count for the row-parallel matmul (rayon pool, main.rs:167-176). */
void orc_set_threads(int n);
int orc_get_threads(void);
const char* orc_last_error(void);

/* Tiny single-layer harness mirroring model.rs tests (:658-729): build an
 * F32 layer from caller arrays and run layer_forward / layer_forward_cached. */
typedef struct orc_f32_layer {
  const float *attn_norm, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *ffn_norm, *w_gate, *w_up, *w_down;
} orc_f32_layer;
void orc_layer_forward_f32(const float* x, size_t seq, const orc_f32_layer* l, const orc_config* c, float* out);
/* k_cache/v_cache are [max_ctx * kv_dim] and updated in place. */
void orc_layer_forward_cached_f32(const float* x, size_t n_new, const orc_f32_layer* l, const orc_config* c,
                                  float* k_cache, float* v_cache, size_t max_ctx, size_t start_pos, float* out);

#ifdef __cplusplus
}
#endif
#endif
