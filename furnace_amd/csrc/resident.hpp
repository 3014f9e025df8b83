// Resident decode: the greedy token loop as one persistent launch (see
// resident.hip).  Host-side structures shared with engine.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"

namespace frn {

// The launch: one block of RES_THREADS threads per CU, RES_XCDS XCDs of
// RES_CUS CUs each (MI355X: 8 x 32).
constexpr uint32_t RES_XCDS = 8, RES_CUS = 32, RES_BLOCKS = RES_XCDS * RES_CUS, RES_THREADS = 256;
// Attention splits per query head at most (each split is one block's job).
constexpr uint32_t RES_MAX_SPLITS = 16;
// Largest vector a block stages (hidden size, one XCD's FFN slice).
constexpr uint32_t RES_MAX_K = 4096;
// Stop ids the kernel checks itself.
constexpr uint32_t RES_MAX_STOP = 16;
// Dynamic LDS per block: above half of the CU's 160 KiB, so that exactly one
// block runs per CU.
constexpr uint32_t RES_LDS_BYTES = 96 * 1024;

// One layer's weights: raw GGUF blocks, their ggml types and row strides.
struct ResLayer {
  const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  const float *bq, *bk, *bv, *an, *fn;  // biases, attn_norm, ffn_norm
  uint32_t tq, tk, tv, to, tg, td;
  uint32_t rq, rk, rv, ro, rg, rd;
};

// Launch control, cleared before every launch.  Each counter sits on its own
// 128-byte line.
struct ResCtl {
  uint32_t ticket[RES_XCDS * 32];  // blocks seen per XCD (ticket[32 x])
  uint32_t abort, pad0[31];        // set by a block that gives up a wait
  uint32_t err, n_done, pad1[30];  // first failure (code | layer | phase), steps completed
};
enum : uint32_t { RES_ERR_LAYOUT = 1u << 24, RES_ERR_WAIT = 2u << 24 };

// Exchange buffers, in 8-byte (value, epoch) pairs:
//  local, per XCD and layer parity: x, q|k|v, attention partials, x after
//   the attention block, the FFN activation;
//  cross-XCD, per parity: the o-proj and down partial sums of every XCD,
//   the lm_head blocks' argmax candidates.
struct ResLayout {
  uint32_t o_x, o_qkv, o_att, o_x2, o_act, loc_stride;
  uint32_t o_po, o_pd, o_lmc, glb_stride;
};

enum : uint32_t { RES_FS_KQUANT = 0, RES_FS_Q8_0 = 1 };

struct ResArgs {
  const ResLayer* layers;
  uint32_t L, H, F, nh, nkv, hd, V, max_ctx;
  float eps, scale;
  const uint8_t* embd;
  uint32_t te, rbe;
  const uint8_t* lm;
  uint32_t tl, rbl;
  const float* onorm;
  float *kc, *vc;
  const float* rope;
  float* logits;
  uint32_t* hist;
  StepState* st;
  uint2 *loc, *glb;
  ResLayout lay;
  ResCtl* ctl;
  uint32_t n_steps, n_stop;
  uint32_t stop[RES_MAX_STOP];
  uint32_t epoch0;
  uint32_t fset;
  // profiling: for steps < trace_steps every block records a 100 MHz
  // timestamp at the end of each phase: trace[step][layer][k][block],
  // k as RES_TR_*; layer n_layers holds the lm_head, argmax and embedding
  uint64_t* trace;
  uint32_t trace_steps;
  uint32_t opts;  // RES_OPT_*
};
// Schedule options (measurement switches).
enum : uint32_t { RES_OPT_ALL_WAVES = 1, RES_OPT_LATE_WEIGHTS = 2, RES_OPT_SHALLOW = 4 };
enum : uint32_t {
  RES_TR_START = 0, RES_TR_A_IN = 1, RES_TR_A = 2, RES_TR_B = 3, RES_TR_C_IN = 4, RES_TR_C = 5, RES_TR_D = 6,
  RES_TR_E_IN = 7, RES_TR_E = 8, RES_TR_F_IN = 9, RES_TR_F = 10, RES_TR_G = 11,
  // input arrived (before staging) for A, E, F, C
  RES_TR_A_POLL = 12, RES_TR_E_POLL = 13, RES_TR_F_POLL = 14, RES_TR_C_POLL = 15,
  // layer n_layers: lm_head input staged, lm_head done, argmax done, next embedding done
  RES_TR_H_IN = 1, RES_TR_H = 2, RES_TR_I = 3, RES_TR_EMBED = 4, RES_TR_K = 16
};

ResLayout res_layout(uint32_t H, uint32_t F, uint32_t nh, uint32_t nkv, uint32_t hd);
// pairs of exchange memory the layout needs (local regions, then cross)
size_t res_exchange_pairs(const ResLayout& l);
// Shape and format checks: nullptr when the resident kernel can run this
// model, else the reason it cannot.  types: every matrix's ggml type;
// o_gran: the column granularity of the o-proj items (128 when any o-proj
// is Q6_K, else 64).
const char* res_unsupported(uint32_t H, uint32_t F, uint32_t nh, uint32_t nkv, uint32_t hd, const uint32_t* types,
                            size_t n_types, uint32_t lm_type, uint32_t o_gran, uint32_t* fset);
hipError_t res_prepare();
// host: the arguments in pinned host memory (left untouched until the copy
// has run); dev: their device copy, which the kernel reads.
hipError_t launch_resident(const ResArgs* host, ResArgs* dev, hipStream_t s);
// epochs one launch of n steps uses (the next launch starts past them)
inline uint32_t res_epochs(uint32_t n_steps, uint32_t L) { return (n_steps * (L + 1) + 1) << 3; }

}  // namespace frn
