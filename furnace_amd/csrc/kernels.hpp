// Launch wrappers for the gfx950 kernels of the token loop.  All pointers
// are device pointers; every wrapper enqueues on `s` and returns the launch
// status.  Shapes are validated by the callers (engine.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frn {

// Per-context step state, resident in device memory so the decode step can
// be replayed as a graph with no host-side arguments.
struct StepState {
  uint32_t pos;        // position of the token being processed (KvCache::len)
  uint32_t tok;        // its id
  uint64_t best;       // packed (ordered logit, ~index) running argmax
  uint32_t next_tok;   // argmax of this step's logits
  uint32_t pad[3];
};

enum GemvMode : int { GEMV_STORE = 0, GEMV_RESID = 1, GEMV_SWIGLU = 2, GEMV_ARGMAX = 3 };

struct GemvArgs {
  const uint8_t* w;      // [rows, row_bytes] raw blocks
  const uint8_t* w2;     // SWIGLU: the up matrix (w is gate)
  uint32_t type, rows, in, row_bytes;
  const float* x;        // [in]
  const float* norm_w;   // optional rmsnorm gain applied to x first
  float eps;
  const float* bias;     // optional [rows]
  float* out;            // [rows]; RESID: out[r] += dot (in place)
  StepState* state;      // ARGMAX: running argmax target
};

hipError_t launch_dequant(uint32_t type, const uint8_t* raw, size_t n_elems, float* out, hipStream_t s);
hipError_t launch_gemv(const GemvArgs& a, GemvMode mode, hipStream_t s);
size_t gemv_lds_bytes(uint32_t type, uint32_t in);
hipError_t gemv_prepare(uint32_t max_in);  // raises dynamic-LDS limits once

hipError_t launch_embed(const uint8_t* table, uint32_t type, uint32_t hidden, uint32_t row_bytes, StepState* st,
                        float* x, hipStream_t s);
hipError_t launch_rope_kv(float* q, const float* k, const float* v, const float* rope_cs, uint32_t n_heads,
                          uint32_t n_kv_heads, uint32_t head_dim, float* k_cache, float* v_cache, const StepState* st,
                          hipStream_t s);
hipError_t launch_attention(const float* q, const float* k_cache, const float* v_cache, uint32_t n_heads,
                            uint32_t n_kv_heads, uint32_t head_dim, uint32_t max_ctx, float scale, float* part,
                            float* att, const StepState* st, hipStream_t s);
size_t attention_part_floats(uint32_t n_heads, uint32_t head_dim, uint32_t max_ctx);
hipError_t launch_step_end(StepState* st, int has_logits, hipStream_t s);
hipError_t launch_argmax(const float* x, size_t n, uint64_t* scratch, uint32_t* out, hipStream_t s);

}  // namespace frn
