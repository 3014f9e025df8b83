/*
 * furnace_hip.h -- C ABI of the MI355X (gfx950) token-loop engine.
 *
 * This is the drop-in boundary for furnace's decode/prefill path.  furnace
 * (Rust) keeps its host code -- GGUF mmap parsing, tokenizer, sampler, the
 * generate loop and CLI -- and replaces everything below `generate`'s calls
 * to Model::forward_cached + Sampler::sample with these entry points.
 * Plain C types only (fixed-width integers, float, pointers, sizes), so a
 * Rust `extern "C"` block binds them unchanged.
 *
 * Conventions
 *  - Every entry point returns frn_status (0 = success) and never aborts.
 *    The message for the last failure on the calling thread is
 *    frn_last_error().
 *  - A context is single-threaded: the caller serialises calls on it.
 *  - One HIP stream per context.  frn_decode's only host synchronisation is
 *    the 4-byte read-back of the next token id.
 *  - Quantized weights are uploaded once in their raw GGUF block layout
 *    (Q8_0 34 B / 32, Q5_0 22 B / 32, Q4_K 144 B / 256, Q6_K 210 B / 256);
 *    full-precision copies of them never exist on the device.
 */
#ifndef FURNACE_HIP_H
#define FURNACE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum frn_status {
  FRN_OK = 0,
  FRN_EINVAL = 1,        /* bad argument, missing tensor, wrong call order */
  FRN_EDTYPE = 2,        /* ggml type without a kernel (quant.rs:191, :279) */
  FRN_ESHAPE = 3,        /* shape/byte-count mismatch (quant.rs:18-32, :210-212) */
  FRN_ECTX_OVERFLOW = 4, /* start + n > max_ctx (model.rs:581-585, :348-352) */
  FRN_ETOKEN = 5,        /* token id >= vocab (model.rs:489) */
  FRN_EOOM = 6,          /* device allocation failed */
  FRN_EHIP = 7,          /* any other HIP runtime error */
  FRN_ENODEV = 8         /* no usable gfx950 device */
} frn_status;

/* ggml tensor type codes, src/gguf.rs:180-201 (the subset with kernels). */
enum { FRN_TYPE_F32 = 0, FRN_TYPE_Q5_0 = 6, FRN_TYPE_Q8_0 = 8, FRN_TYPE_Q4_K = 12, FRN_TYPE_Q6_K = 14 };

/* Model configuration: src/model.rs:26-38 Config, filled by the host from
 * GGUF metadata exactly as Config::from_gguf (model.rs:41-60) does.
 * max_ctx replaces KvCache::new's max_ctx (model.rs:330; generate.rs:91). */
typedef struct frn_config {
  uint32_t n_layers, n_heads, n_kv_heads, hidden, ffn, head_dim, vocab, max_ctx;
  float rope_theta, rms_eps;
  uint32_t tied_lm_head; /* 1 when output.weight is absent (model.rs:541-545) */
  uint32_t flags;        /* FRN_FLAG_* */
} frn_config;

/* Launch the step's kernels one by one instead of replaying a hipGraph
 * (same kernels; for profilers that do not follow graph launches). */
#define FRN_FLAG_EAGER 1u
/* Prefill one decode step per prompt position (the decode kernels) instead
 * of blocks of rows through the MFMA GEMMs.  For comparisons. */
#define FRN_FLAG_STEPWISE_PREFILL 2u
/* Decode with the per-step graphs even where the resident decode kernel
 * (frn_decode_engine) could run.  For comparisons. */
#define FRN_FLAG_NO_RESIDENT 4u
/* Decode with the resident decode kernel where it can run (frn_decode_engine);
 * without this flag or FRN_FLAG_NO_RESIDENT the engine picks the faster form
 * for the model. */
#define FRN_FLAG_RESIDENT 8u

typedef struct frn_ctx frn_ctx;

/* Allocate a context on HIP device `device`: the KV cache (f32,
 * [n_layers][max_ctx][n_kv_heads*head_dim] for K and V, model.rs:321-339),
 * activation buffers, the RoPE table and the prefill's row buffers
 * (min(max_ctx, 4096) rows of 3*hidden + 2*kv_dim + ffn floats: ~500 MB at
 * Qwen2-7B shape).  Replaces Model::load's allocation side
 * (model.rs:520-552) and KvCache::new (model.rs:330-339). */
frn_status frn_create(const frn_config* cfg, int device, frn_ctx** out);

/* Copy one GGUF tensor from host memory (e.g. the mmap) to HBM, raw.
 * `name` is the GGUF tensor name ("token_embd.weight", "blk.3.ffn_up.weight",
 * "output_norm.weight", ...); out_dim/in_dim are dims[1]/dims[0] (ggml order,
 * model.rs:123-124; 1-D tensors pass out_dim = 1).  The host may unmap the
 * source after the call.  Replaces load_weight / Tensor::from_gguf
 * (model.rs:112-126, tensor.rs:55-60). */
frn_status frn_upload(frn_ctx* ctx, const char* name, uint32_t ggml_type, uint64_t out_dim, uint64_t in_dim,
                      const void* host, size_t bytes);

/* Check that every tensor Model::load requires is present and
 * consistently shaped, then build the decode step.  Must follow the uploads
 * and precede prefill/decode. */
frn_status frn_finalize(frn_ctx* ctx);

/* Model::forward_cached(&prompt) + Sampler::sample at temperature 0
 * (model.rs:579-592, sampler.rs:91-94, generate.rs:69-77): runs the n ids at
 * positions ctx.len .. ctx.len+n, advances ctx.len by n and writes the
 * argmax of the last position's logits (first maximum on ties).  n >= 2
 * runs blocks of up to 4096 positions through fp32-MFMA GEMMs on the raw
 * weight blocks (dequantized exactly into LDS tiles). */
frn_status frn_prefill(frn_ctx* ctx, const uint32_t* ids, uint32_t n, uint32_t* next_id);

/* One decode step: Model::forward_cached(&[id]) + argmax
 * (generate.rs:136, :124).  Only the next id crosses back to the host. */
frn_status frn_decode(frn_ctx* ctx, uint32_t id, uint32_t* next_id);

/* Greedy decode of up to n steps (the loop of generate.rs:110-136 at
 * temperature 0, as n frn_decode calls where each feeds back the previous
 * next_id): step i runs at position ctx.len and decodes `id` (i = 0) or
 * out_ids[i-1], writing its argmax to out_ids[i].  The steps are enqueued
 * back to back, the argmax feeding the next step on the device, and the
 * host synchronises once per batch of up to 32 steps.  If out_ids[i] is one
 * of the n_stop stop_ids, the loop ends there (generate.rs:125-127) with
 * *n_done = i + 1 and ctx.len just past step i; steps of the batch that ran
 * beyond it are rolled back and frn_logits has nothing to return.  The ids
 * equal those of the frn_decode loop. */
frn_status frn_decode_greedy(frn_ctx* ctx, uint32_t id, uint32_t n, const uint32_t* stop_ids, uint32_t n_stop,
                             uint32_t* out_ids, uint32_t* n_done);

/* Which engine serves frn_decode / frn_decode_greedy (no counterpart in the
 * reference, which has one CPU path): *resident = 1 for the resident decode
 * kernel -- the whole greedy loop (every layer, lm_head, argmax, next
 * embedding) in one persistent launch of one block per CU, the 8 XCDs each
 * owning an eighth of the heads and of the FFN -- or 0 for the per-step
 * graphs of kernels, with the reason in reason[0..reason_len) (may be NULL).
 * The resident kernel needs an MI355X with 256 CUs, all matrices Q4_K/Q6_K
 * or all Q8_0, hidden <= 4096 (a multiple of 256 for the K-quants), ffn a
 * multiple of 128, head_dim 64 or 128.  A resident launch that fails (a
 * bounded wait gave up) returns FRN_EHIP and the context decodes with the
 * graphs from then on. */
frn_status frn_decode_engine(frn_ctx* ctx, uint32_t* resident, char* reason, size_t reason_len);

/* Profiling hook for the resident decode kernel (no counterpart in the
 * reference).  host_out == NULL arms the next resident launch to record, for
 * its first n_steps steps, a 100 MHz timestamp per block at the end of every
 * phase: [n_steps][n_layers + 1][16][256] uint64 (layer n_layers: the
 * lm_head, argmax and next embedding).  With host_out, copies the recorded
 * stamps of the last armed launch (n values at most). */
frn_status frn_resident_trace(frn_ctx* ctx, uint32_t n_steps, uint64_t* host_out, size_t n);

/* Sampler::new (sampler.rs:68-78) on the device: temperature, top_k, top_p,
 * repeat penalty (1.0 disables) and the PCG32 seed (Pcg32::new).  At
 * temperature 0 or top_k 1, frn_sample is the argmax of the penalized logits
 * and takes no RNG draw (sampler.rs:91-94).  top_k 2..64 keeps per-block
 * candidates; top_k 0 ("no cut") and top_k above 64 sort the whole
 * vocabulary on the device (the first such call allocates 4 buffers of
 * vocab entries and the sort's temporary storage). */
frn_status frn_sampler_init(frn_ctx* ctx, float temperature, uint32_t top_k, float top_p, float repeat_penalty,
                            uint64_t seed);

/* Sampler::sample(logits, recent) (sampler.rs:86-108) on the device logits of
 * the last frn_prefill / frn_decode: repeat penalty over the unique ids of
 * recent[0..n_recent) (generate.rs:123 passes the last repeat_window = 64
 * context ids; at most 256), temperature, top-k, softmax, top-p, renormalize,
 * one PCG32 draw.  The id also becomes the device's next token, so
 * frn_decode(ctx, *next_id) uploads nothing.  Equal scaled logits are taken
 * in ascending id order (the reference's unstable sort leaves them
 * unordered). */
frn_status frn_sample(frn_ctx* ctx, const uint32_t* recent, uint32_t n_recent, uint32_t* next_id);

/* Sampler::draws (sampler.rs:82-84): RNG draws taken since frn_sampler_init. */
frn_status frn_sampler_draws(frn_ctx* ctx, uint64_t* draws);

/* Copy the last step's logits [vocab] to host memory (the 1e-3 parity gate
 * and any host-side sampler).  n must be >= vocab. */
frn_status frn_logits(frn_ctx* ctx, float* host_out, size_t n);

/* Forget the cached positions (ctx.len = 0).  Weights stay resident. */
frn_status frn_reset(frn_ctx* ctx);
/* Current number of cached positions (KvCache::len, model.rs:324). */
frn_status frn_cache_len(frn_ctx* ctx, uint32_t* len);
/* Read layer `layer`'s cached K (which = 0) or V (which = 1) rows [0, n)
 * into host memory, n * n_kv_heads * head_dim floats (debug/parity). */
frn_status frn_cache_read(frn_ctx* ctx, uint32_t layer, uint32_t which, uint32_t n, float* host_out);

void frn_destroy(frn_ctx* ctx);

/* Message for the last failure on this thread ("" if none). */
const char* frn_last_error(void);

/* --timings dashboard (perf.rs:25-96): per-kernel GPU time of the steps run
 * since the last frn_timings_reset.  While enabled, steps run eagerly (not
 * as a graph) with a HIP event pair around every kernel.  Entries: embed,
 * qkv, rope_kv, attention, o_proj, gate_up, down, lm_head, step_end.
 * perf.rs's matmul counter is qkv + o_proj + gate_up + down + lm_head; its
 * rmsnorm, add/swiglu and sample work is fused into those kernels. */
typedef struct frn_timing {
  char name[16];
  double ms;
  uint64_t calls;
} frn_timing;
frn_status frn_timings_enable(frn_ctx* ctx, int enable);
frn_status frn_timings_reset(frn_ctx* ctx);
frn_status frn_timings(frn_ctx* ctx, frn_timing* out, uint32_t max, uint32_t* n);

/* Per-step decode times, for the `[decode N: seq M, X ms/token]` lines of
 * generate.rs:137-140.  While enabled, frn_decode and frn_decode_greedy
 * record a HIP event after every step (one graph launch per step; the
 * resident decode kernel is not used) and keep each step's duration in ms:
 * from the end of the previous step of the same batch (the batch's start
 * for its first step) to the step's end.  Enabling (or disabling) forgets
 * what was kept.  frn_step_times moves up to max kept durations, oldest
 * first, to ms_out; *n receives the count. */
frn_status frn_step_times_enable(frn_ctx* ctx, int enable);
frn_status frn_step_times(frn_ctx* ctx, float* ms_out, uint32_t max, uint32_t* n);

/* Measurement hook (no counterpart in the reference; used by the bench to
 * price one kernel without per-launch event overhead): launches the kernel
 * of timing category `name` (as in frn_timings) for `layer` `reps` times
 * back to back on the context's stream, between one event pair, and
 * returns the mean time per launch.  layer == FRN_ALL_LAYERS launches it
 * for every layer in order, reps rounds, so the weights stream from HBM as
 * in a decode step (one layer's weights replayed alone would stay in the
 * 256 MB last-level cache).  Leaves the context's activations and position
 * undefined: call frn_reset afterwards. */
#define FRN_ALL_LAYERS 0xFFFFFFFFu
frn_status frn_bench_kernel(frn_ctx* ctx, const char* name, uint32_t layer, uint32_t reps, float* avg_us);

/* ---- single-op entry points (device pointers, caller's stream) ----------- */

/* quant::dequantize (quant.rs:261-281) on device buffers: n_elems values of
 * `type` from raw_dev (raw_bytes long) into out_dev as f32.  Bit-exact with
 * the CPU path.  stream may be NULL (the default stream). */
frn_status frn_dequant(uint32_t type, const void* raw_dev, size_t raw_bytes, size_t n_elems, float* out_dev,
                       void* stream);

/* quant::matmul_quant (quant.rs:170-193): a_dev [seq, d_in] f32 times the
 * raw quantized weight w_dev [d_out, d_in] -> out_dev [seq, d_out] f32.
 * Each of the seq rows is one launch of the decode GEMV kernel for `type`.
 * w_bytes must equal d_out * (d_in / block) * block_bytes. */
frn_status frn_matmul_quant(uint32_t type, const void* w_dev, size_t w_bytes, const float* a_dev, uint32_t seq,
                            float* out_dev, uint32_t d_out, uint32_t d_in, void* stream);

/* Device argmax over n floats, first maximum on ties (generate.rs:69-77).
 * n at most 2^32 - 1. */
frn_status frn_argmax(const float* x_dev, size_t n, uint32_t* out_dev, void* stream);

/* frn_argmax without any allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * result and limit (n at most 2^32 - 1, else FRN_ESHAPE) as frn_argmax; its
 * 8-byte running key lives in a static 256-byte device array, one per GPU,
 * looked up on the first call on each device.  Calls that overlap on one
 * GPU (different streams or threads) share that array and race. */
frn_status frn_argmax_noalloc(const float* x_dev, size_t n, uint32_t* out_dev, void* stream);

#ifdef __cplusplus
}
#endif
#endif
