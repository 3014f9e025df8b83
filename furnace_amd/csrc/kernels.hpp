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
  uint32_t next_tok;   // argmax of this step's logits
  uint32_t pad[5];
};

// RESID_ATT: RESID whose x is the attention output, merged from the
// attention kernel's per-split partials while staging.
enum GemvMode : int { GEMV_STORE = 0, GEMV_RESID = 1, GEMV_SWIGLU = 2, GEMV_ARGMAX = 3, GEMV_RESID_ATT = 4 };

// One weight matrix of a (possibly multi-matrix) GEMV launch.  All segments
// of a launch share the input vector x and its optional rmsnorm.
struct GemvSeg {
  const uint8_t* w;   // [rows, row_bytes] raw blocks
  const uint8_t* w2;  // SWIGLU: the up matrix (w is gate)
  uint32_t type, rows, row_bytes, block0;  // block0: first block of this segment
  const float* bias;  // optional [rows]
  float* out;         // [rows]; RESID: out[r] = resid[r] + dot
  const float* resid; // RESID: residual input (may equal out)
  float* out2;        // RESID: optional second copy of the result
};

struct GemvArgs {
  GemvSeg seg[3];
  int n_seg;
  uint32_t in;
  const float* x;       // [in]
  const float* norm_w;  // optional rmsnorm gain applied to x first (tensor.rs:164-185)
  float eps;
  uint64_t* best;       // ARGMAX: one packed (logit, ~row) candidate per block
  // RESID_ATT: partials [n_heads][att_ms][att_hd + 2] = (o[att_hd], m, l) of
  // the step's splits (attention_split_len positions each; st->pos + 1
  // positions in all)
  const float* att_part;
  const StepState* st;
  uint32_t att_ms, att_hd, att_part_bytes;
};

hipError_t launch_dequant(uint32_t type, const uint8_t* raw, size_t n_elems, float* out, hipStream_t s);
// Launches one GEMV over args.n_seg segments (mode applies to all).
// Returns the number of blocks launched through *blocks when non-null.
hipError_t launch_gemv(GemvArgs a, GemvMode mode, hipStream_t s, uint32_t* blocks = nullptr);
size_t gemv_lds_bytes(uint32_t in, bool norm);
hipError_t gemv_prepare(size_t max_lds_bytes);  // raises dynamic-LDS limits once
// Blocks launch_gemv uses for a single segment of `rows` rows and in `in`.
uint32_t gemv_blocks(uint32_t type, uint32_t rows, uint32_t in);

// Embedding row of st->tok into x; also copies row st->pos of the RoPE
// table (hd floats, cos | sin) to rope_cur for the step's attention launches.
hipError_t launch_embed(const uint8_t* table, uint32_t type, uint32_t hidden, uint32_t row_bytes, StepState* st,
                        float* x, const float* rope, uint32_t hd, float* rope_cur, hipStream_t s);
constexpr uint32_t ATTENTION_CHUNK = 64;  // positions per attention sub-tile
// At most 16 splits while the o-proj GEMV merges them in its staging
// (GEMV_RESID_ATT: one or two batches of loads); at most 128 in the
// long-context step, whose splits k_attn_merge merges once (one 64-position
// sub-tile per block up to 8192 positions).
constexpr uint32_t ATTENTION_MAX_SPLITS = 16;
constexpr uint32_t ATTENTION_MAX_SPLITS_LONG = 128;
// Steps over more positions than this (pos + 1) run the long-context form.
constexpr uint32_t ATTENTION_LONG_FROM = 1024;
// RoPE(q), RoPE(k) at the step's position (rope_cur: that position's
// cos | sin row), KV-cache append and split-sequence GQA attention in one
// launch, with at most `cap` splits;
// writes the per-split partials that a GEMV_RESID_ATT launch (cap 16) or
// launch_attn_merge (cap 128) merges (layout in GemvArgs).  live > 0 (cap
// 16 only): the launch serves only steps with exactly `live` splits (T in
// (64 (live - 1), 64 live]); its grid holds those splits alone and every
// block streams its K/V rows before it reads the step position.
hipError_t launch_attention(const float* q, const float* k, const float* v, const float* rope_cur, float* k_cache,
                            float* v_cache, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                            uint32_t max_ctx, float scale, float* part, const StepState* st, uint32_t cap,
                            uint32_t live, hipStream_t s);
// The long-context merge: out[h][d] = sum_s e^(m_s - M) o_s[d] / sum_s
// e^(m_s - M) l_s over the step's splits, one block per query head.
hipError_t launch_attn_merge(const float* part, float* out, uint32_t n_heads, uint32_t head_dim, uint32_t max_ctx,
                             const StepState* st, hipStream_t s);
// partials buffer: n_heads x attention_splits(max_ctx, 128) x (head_dim + 2)
size_t attention_part_floats(uint32_t n_heads, uint32_t head_dim, uint32_t max_ctx);
// the most splits a step can have with at most `cap` (att_ms for cap 16)
uint32_t attention_splits(uint32_t max_ctx, uint32_t cap = ATTENTION_MAX_SPLITS);
// Positions per split for a step over T positions: whole 64-position
// sub-tiles, as few as keep the step at <= cap splits.
__host__ __device__ inline uint32_t attention_split_len(uint32_t T, uint32_t cap = ATTENTION_MAX_SPLITS) {
  const uint32_t tiles = (T + ATTENTION_CHUNK - 1) / ATTENTION_CHUNK;
  return ATTENTION_CHUNK * ((tiles + cap - 1) / cap);
}
// Query heads of one kv head's group that one attention block handles
// (the launch's grid z covers the group in blocks of this many).
uint32_t attention_heads_per_block(uint32_t gq, uint32_t cap);
// Shapes the attention kernel handles: head_dim 64 or 128, at most 8 query
// heads per kv head.
bool attention_supported(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim);
// Ends a step: reduces the lm_head kernel's per-block argmax candidates
// (best == nullptr for a step without logits) into next_tok/tok, records
// the id at hist[pos] when hist is given, and advances the position.
hipError_t launch_step_end(StepState* st, const uint64_t* best, uint32_t n_best, uint32_t* hist, hipStream_t s);
hipError_t launch_argmax(const float* x, size_t n, uint64_t* scratch, uint32_t* out, hipStream_t s);

// ---- prefill (prefill.hip) ----------------------------------------------------
enum GemmMode : int { GEMM_STORE = 0, GEMM_RESID = 1, GEMM_SWIGLU = 2 };

// C[P][N] = A[P][K] . W[N][K]^T on bf16 MFMA.  A comes split into two bf16
// planes, a_hi + a_lo (row stride K; launch_rows_split, the attention rows
// and the SwiGLU epilogue write that form).  STORE: out = C (+ bias);
// RESID: out += C; SWIGLU: silu(C(w)) * C(w2), split into the planes
// o_hi / o_lo (row stride ldo).  Q4_K weights also read the sums of A's
// 32-value groups, x_hi + x_lo (launch_group_sums).
struct GemmArgs {
  const uint16_t* a_hi;  // [P][K] bf16
  const uint16_t* a_lo;  // [P][K] bf16
  const uint16_t* x_hi;  // Q4_K: [P][K / 32] bf16, group sums of a_hi + a_lo
  const uint16_t* x_lo;
  const uint8_t* w;      // [N] rows of row_bytes raw blocks
  const uint8_t* w2;     // SWIGLU: the up matrix
  uint32_t type, row_bytes;
  const float* bias;     // optional [N]
  float* out;            // STORE / RESID: [P][ldo] f32
  uint16_t* o_hi;        // SWIGLU: [P][ldo] bf16 planes
  uint16_t* o_lo;
  uint32_t ldo, P, N, K;
  // Few output tiles (short prompts): the K range may be split over blocks
  // (grid z) that store partial products to `partial` (STORE [z][P][all
  // segments' columns], RESID [z][P][N], SWIGLU [z][2][P][N] f32, at most
  // partial_floats), summed in z order afterwards; nullptr: no split
  float* partial;
  size_t partial_floats;
  uint32_t ksplit, kchunk;  // set by launch_gemm
  // STORE: up to two more weight matrices of the same type and K on the
  // same A (a layer's q, k and v), with their own bias, output and ldo; one
  // launch, their tiles after segment 0's
  uint32_t n_more;
  struct More {
    const uint8_t* w;
    const float* bias;
    float* out;
    uint32_t N, ldo;
  } more[2];
};
hipError_t launch_gemm(const GemmArgs& g, GemmMode mode, hipStream_t s);
// Raises the GEMM kernels' dynamic LDS limit (up to 120 KiB per block) on
// the current device; once per device before the first launch_gemm.
hipError_t gemm_prepare();
// Rows of x [rows][cols] -- rmsnorm'd with gain nw (tensor.rs:164-185) when
// nw is given -- split into the bf16 planes hi + lo that the GEMM reads;
// with xh/xl given (cols % 32 == 0), also their 32-value group sums (the
// Q4_K GEMMs' x_hi/x_lo).
hipError_t launch_rows_split(const float* x, uint32_t rows, uint32_t cols, const float* nw, float eps, uint16_t* hi,
                             uint16_t* lo, uint16_t* xh, uint16_t* xl, hipStream_t s);
// Sums of the 32-value groups of rows [rows][cols] given as bf16 planes
// hi + lo, each sum split into the planes xh + xl ([rows][cols / 32]).
hipError_t launch_group_sums(const uint16_t* hi, const uint16_t* lo, uint32_t rows, uint32_t cols, uint16_t* xh,
                             uint16_t* xl, hipStream_t s);
hipError_t launch_embed_rows(const uint8_t* table, uint32_t type, uint32_t hidden, uint32_t row_bytes,
                             const uint32_t* ids, uint32_t n, float* x, hipStream_t s);
// RoPE of n q rows (in place) and k rows (into the cache) at positions
// pos0.., v rows into the cache.
hipError_t launch_rope_kv_rows(float* q, const float* k, const float* v, const float* rope_cs, float* k_cache,
                               float* v_cache, uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                               uint32_t pos0, uint32_t n, hipStream_t s);
// A layer's keys 0 .. T of the cache as the attention's bf16 planes
// (kv_split_elems(T, kvd) 16-bit values at `planes`).
inline size_t kv_split_elems(uint32_t T, uint32_t kvd) { return 4ull * ((T + 31) / 32 * 32) * kvd; }
hipError_t launch_kv_split(const float* k_cache, const float* v_cache, uint32_t T, uint32_t kvd, uint16_t* planes,
                           hipStream_t s);
// Causal attention of n query rows at positions pos0.. over keys 0 ..
// pos0 + n (launch_kv_split's planes); the output rows [n][n_heads *
// head_dim] as the GEMM's bf16 planes.
hipError_t launch_attn_rows(const float* q, const uint16_t* kv_planes, uint16_t* out_hi, uint16_t* out_lo,
                            uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t pos0, uint32_t n,
                            float scale, float* part, hipStream_t s);
// Past 512 keys the late query blocks' keys run in up to ATTN_ROWS_CHUNKS
// chunks (blocks of their own) whose partials (`part`, attn_rows_part_floats
// floats; nullptr: no chunks) a merge kernel combines.
constexpr uint32_t ATTN_ROWS_CHUNKS = 4;
size_t attn_rows_part_floats(uint32_t n_heads, uint32_t head_dim, uint32_t rows);
// Argmax of the lm_head candidates into next_tok/tok, position += n.
hipError_t launch_prefill_end(StepState* st, const uint64_t* best, uint32_t n_best, uint32_t n, hipStream_t s);

}  // namespace frn
