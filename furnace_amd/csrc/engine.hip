// Engine context and C ABI (include/furnace_hip.h).
//
// A context owns, on one gfx950 device: the raw GGUF weight blocks (one
// allocation per tensor, uploaded once), the f32 KV cache, activation
// buffers, the host-computed RoPE table and a StepState.  finalize() records
// the decode step -- embedding, 28x (norm+QKV, RoPE+KV write, attention,
// o-proj+residual, norm+gate/up+SwiGLU, down+residual), final norm + lm_head
// + argmax -- into a hipGraph that is replayed once per token.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/furnace_hip.h"
#include "common.hpp"
#include "formats.hpp"
#include "kernels.hpp"
#include "resident.hpp"
#include "sampler.hpp"

using namespace frn;

#define fail frn_fail

static frn_status hip_fail(hipError_t e, const char* what) {
  return fail(e == hipErrorOutOfMemory ? FRN_EOOM : FRN_EHIP, "%s: %s", what, hipGetErrorString(e));
}
#define HIP_TRY(expr, what)                  \
  do {                                       \
    hipError_t e_ = (expr);                  \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)


namespace {

struct DevTensor {
  uint32_t type = 0;
  uint64_t out = 0, in = 0;
  size_t bytes = 0;
  uint8_t* ptr = nullptr;  // raw blocks, or f32 for 1-D tensors
};

struct LayerPtrs {
  const float *attn_norm, *bq, *bk, *bv, *ffn_norm;
  const DevTensor *wq, *wk, *wv, *wo, *gate, *up, *down;
};

size_t type_row_bytes(uint32_t t, uint64_t in) { return (size_t)(in / blk_elems(t)) * blk_bytes(t); }
// F16 is an extension: the reference's dequantize has no F16 arm and its
// Model::load rejects such tensors (src/quant.rs:279)
bool known_type(uint32_t t) {
  return t == T_F32 || t == T_F16 || t == T_Q5_0 || t == T_Q8_0 || t == T_Q4_K || t == T_Q6_K;
}

// Kernel categories of the --timings dashboard.  furnace's perf.rs counters
// (matmul, rmsnorm, rope, attn, add/swiglu, embed, sample) map onto these
// fused kernels: rmsnorm runs in the GEMV prologues, bias/residual/SwiGLU
// in their epilogues, the sampler's argmax in the lm_head kernel.
enum { CAT_EMBED, CAT_QKV, CAT_ROPE, CAT_ATTN, CAT_OPROJ, CAT_GATEUP, CAT_DOWN, CAT_LMHEAD, CAT_STEP, N_CAT };
const char* const CAT_NAMES[N_CAT] = {"embed", "qkv", "rope_kv", "attention", "o_proj", "gate_up", "down",
                                      "lm_head", "step_end"};

}  // namespace

struct frn_ctx {
  frn_config cfg{};
  int device = 0;
  hipStream_t stream = nullptr;
  std::map<std::string, DevTensor> tensors;
  std::vector<LayerPtrs> layers;
  const DevTensor *embd = nullptr, *lm_head = nullptr;
  const float* out_norm = nullptr;
  float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *act = nullptr, *logits = nullptr;
  float *part = nullptr, *kcache = nullptr, *vcache = nullptr, *rope = nullptr;
  float* rope_cur = nullptr;  // the step position's row of `rope`, copied by the embed kernel
  uint64_t* best_part = nullptr;  // per-block argmax candidates of the lm_head kernel
  uint32_t n_best = 0;
  StepState* st = nullptr;
  StepState* h_st = nullptr;  // pinned mirror for read-back
  uint32_t* hist = nullptr;    // [max_ctx] argmax id of each decoded position (frn_decode_greedy)
  uint32_t* h_hist = nullptr;  // pinned [GREEDY_BATCH] read-back of one batch
  // device sampler (frn_sampler_init / frn_sample)
  SamplerRng* rng = nullptr;                           // Pcg32 state and draw count
  float* cand_v = nullptr;                             // per-block candidates
  uint32_t *cand_id = nullptr, *recent = nullptr;      // [SAMPLER_MAX_RECENT] recent ids
  uint32_t* h_recent = nullptr;                        // pinned staging of the recent ids
  SamplerRng* h_rng = nullptr;                         // pinned staging of the RNG state
  bool sampler_ready = false;
  float s_temperature = 0.f, s_top_p = 1.f, s_penalty = 1.f;
  uint32_t s_top_k = 0;
  bool s_full = false;  // top_k 0 or above SAMPLER_MAX_K: the whole-vocabulary path
  SamplerFull full;     // its buffers, allocated by the first frn_sampler_init that needs them
  // prefill rows: blocks of up to pf_rows prompt tokens through all layers
  uint32_t pf_rows = 0;
  float *pf_x = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr;
  // the GEMM operands as bf16 hi + lo planes: rmsnorm'd x, attention rows, SwiGLU activation
  uint16_t *pf_xs = nullptr, *pf_att = nullptr, *pf_act = nullptr;
  uint16_t* pf_xg = nullptr;  // group sums of a Q4_K GEMM's input planes (launch_group_sums)
  float* pf_part = nullptr;   // split-K partial products of the short prompts' residual GEMMs
  float* pf_attp = nullptr;   // the prefill attention's key-chunk partials
  uint16_t* pf_kvs = nullptr;  // a layer's K and V as the prefill attention's bf16 planes (max_ctx keys)
  uint32_t* pf_ids = nullptr;
  uint32_t len = 0;           // host view of KvCache::len
  uint32_t last_next = 0xFFFFFFFFu;
  bool finalized = false, have_logits = false;
  // captured steps: [0] short contexts, [1] past ATTENTION_LONG_FROM positions
  hipGraphExec_t g_step[2] = {}, g_prefill[2] = {}, g_multi[2] = {};
  hipGraph_t graph_step[2] = {}, graph_prefill[2] = {}, graph_multi[2] = {};
  // short-context steps by their exact attention split count n (T in
  // (64 (n - 1), 64 n]): index n - 1; one step, and GREEDY_MULTI steps
  hipGraphExec_t g_exact[ATTENTION_MAX_SPLITS] = {}, g_exact_multi[ATTENTION_MAX_SPLITS] = {};
  hipGraph_t graph_exact[ATTENTION_MAX_SPLITS] = {}, graph_exact_multi[ATTENTION_MAX_SPLITS] = {};
  bool rec_long = false;  // the form record_step records (long-context attention)
  uint32_t rec_splits = 0;  // > 0: record the short form with exactly this many splits
  float* att = nullptr;   // [n_heads * head_dim] merged attention output (long-context form)
  // --timings: the step runs eagerly with an event pair around each kernel
  bool timing = false;
  std::vector<hipEvent_t> ev;
  std::vector<int> ev_cat;
  double t_ms[N_CAT] = {0};
  uint64_t t_calls[N_CAT] = {0};
  // frn_step_times: an event after every decode step, durations kept here
  bool step_timing = false;
  std::vector<hipEvent_t> st_ev;  // GREEDY_BATCH + 1
  std::vector<float> step_ms;
  // resident decode (resident.hip): the whole greedy loop in one launch
  bool res_ok = false;
  std::string res_why = "not finalized";
  ResArgs* h_res = nullptr;   // pinned: the launch arguments, copied to d_res per launch
  ResArgs* d_res = nullptr;
  ResLayer* d_layers = nullptr;
  uint2* res_ex = nullptr;    // exchange pairs
  size_t res_ex_bytes = 0;
  ResCtl* res_ctl = nullptr;
  ResCtl* h_ctl = nullptr;    // pinned read-back
  uint32_t* h_ids = nullptr;  // pinned [RES_STEPS] ids of one launch
  uint32_t res_epoch = 0;     // first epoch of the next launch
  uint64_t* res_trace = nullptr;  // frn_resident_trace buffer
  size_t res_trace_n = 0;         // its length in stamps
  uint32_t res_trace_arm = 0;     // steps the next launch records
};

static void free_ctx(frn_ctx* c) {
  if (!c) return;
  for (int i = 0; i < 2; ++i) {
    if (c->g_step[i]) (void)hipGraphExecDestroy(c->g_step[i]);
    if (c->g_prefill[i]) (void)hipGraphExecDestroy(c->g_prefill[i]);
    if (c->graph_step[i]) (void)hipGraphDestroy(c->graph_step[i]);
    if (c->graph_prefill[i]) (void)hipGraphDestroy(c->graph_prefill[i]);
    if (c->g_multi[i]) (void)hipGraphExecDestroy(c->g_multi[i]);
    if (c->graph_multi[i]) (void)hipGraphDestroy(c->graph_multi[i]);
  }
  for (uint32_t i = 0; i < ATTENTION_MAX_SPLITS; ++i) {
    if (c->g_exact[i]) (void)hipGraphExecDestroy(c->g_exact[i]);
    if (c->graph_exact[i]) (void)hipGraphDestroy(c->graph_exact[i]);
    if (c->g_exact_multi[i]) (void)hipGraphExecDestroy(c->g_exact_multi[i]);
    if (c->graph_exact_multi[i]) (void)hipGraphDestroy(c->graph_exact_multi[i]);
  }
  for (auto& kv : c->tensors) (void)hipFree(kv.second.ptr);
  for (hipEvent_t e : c->ev) (void)hipEventDestroy(e);
  for (hipEvent_t e : c->st_ev) (void)hipEventDestroy(e);
  void* bufs[] = {c->x, c->q, c->k, c->v, c->act, c->logits, c->part, c->kcache, c->vcache, c->rope, c->rope_cur, c->st, c->best_part, c->hist, c->att, c->rng, c->cand_v, c->cand_id, c->recent, c->full.keys, c->full.terms, c->pf_x, c->pf_q, c->pf_k, c->pf_v, c->pf_xs, c->pf_att, c->pf_act, c->pf_kvs, c->pf_ids, c->pf_xg, c->pf_part, c->pf_attp};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  if (c->h_st) (void)hipHostFree(c->h_st);
  if (c->h_hist) (void)hipHostFree(c->h_hist);
  if (c->h_recent) (void)hipHostFree(c->h_recent);
  if (c->h_rng) (void)hipHostFree(c->h_rng);
  if (c->h_res) (void)hipHostFree(c->h_res);
  if (c->h_ctl) (void)hipHostFree(c->h_ctl);
  if (c->h_ids) (void)hipHostFree(c->h_ids);
  void* rbufs[] = {c->d_res, c->d_layers, c->res_ex, c->res_ctl, c->res_trace};
  for (void* p : rbufs)
    if (p) (void)hipFree(p);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
}

template <typename T>
static hipError_t dmalloc(T** p, size_t bytes) {
  return hipMalloc((void**)p, bytes ? bytes : 16);
}

// Prefill works on blocks of up to PREFILL_ROWS tokens (64-row GEMM tiles).
// Every GEMM's grid grows with the block's rows: at 256 rows the 1.5B
// hidden-size GEMMs ran 96 blocks on 256 CUs.  Measured (MI355X): 7B
// 2048-token prompt 5,120 / 6,460 / 7,270 / 8,110 prefill tokens/s at
// 256 / 512 / 1024 / 2048 rows; 1.5B 4096-token prompt 10,756 / 19,105 /
// 26,500 / 32,050 / 34,680 at 256 ... 4096.  The scratch is
// min(max_ctx, 4096) x (3 hidden + 2 kv + ffn) floats: ~500 MB at 7B.
constexpr uint32_t PREFILL_ROWS = 4096;
// frn_decode_greedy's steps per host synchronisation (and the most steps
// that run past a stop id before the host sees it).
constexpr uint32_t GREEDY_BATCH = 32;
// split-K partial products of the prefill's residual GEMMs (32 MiB)
constexpr size_t PREFILL_PARTIAL_FLOATS = 8u << 20;
// decode steps per captured multi-step graph of frn_decode_greedy
// (8 or 16 steps per graph measured the same: 1,100 tokens/s at 1.5B)
constexpr uint32_t GREEDY_MULTI = 4;
// decode steps per resident launch (one host synchronisation each)
constexpr uint32_t RES_STEPS = 128;
// whether models the resident kernel supports use it without FRN_FLAG_RESIDENT
constexpr bool kResidentDefault = false;

static hipError_t alloc_prefill(frn_ctx* x) {
  const frn_config& c = x->cfg;
  const size_t P = std::min(c.max_ctx, PREFILL_ROWS), qd = (size_t)c.n_heads * c.head_dim,
               kvd = (size_t)c.n_kv_heads * c.head_dim;
  x->pf_rows = (uint32_t)P;
  hipError_t e;
  if ((e = dmalloc(&x->pf_x, P * c.hidden * 4)) || (e = dmalloc(&x->pf_q, P * qd * 4)) ||
      (e = dmalloc(&x->pf_k, P * kvd * 4)) || (e = dmalloc(&x->pf_v, P * kvd * 4)) ||
      (e = dmalloc(&x->pf_xs, P * c.hidden * 4)) || (e = dmalloc(&x->pf_att, P * qd * 4)) ||
      (e = dmalloc(&x->pf_act, P * c.ffn * 4)) || (e = dmalloc(&x->pf_ids, P * 4)) ||
      (e = dmalloc(&x->pf_xg, P * std::max<size_t>(std::max<size_t>(c.hidden, qd), c.ffn) / 32 * 4)) ||
      (e = dmalloc(&x->pf_part, PREFILL_PARTIAL_FLOATS * 4)) ||
      (e = dmalloc(&x->pf_attp, attn_rows_part_floats(c.n_heads, c.head_dim, (uint32_t)P) * 4)) ||
      (e = dmalloc(&x->pf_kvs, kv_split_elems(c.max_ctx, (uint32_t)kvd) * 2)))
    return e;
  return hipSuccess;
}

extern "C" frn_status frn_create(const frn_config* cfg, int device, frn_ctx** out) {
  if (!cfg || !out) return fail(FRN_EINVAL, "frn_create: null argument");
  *out = nullptr;
  const frn_config& c = *cfg;
  if (!c.n_layers || !c.n_heads || !c.n_kv_heads || !c.hidden || !c.ffn || !c.head_dim || !c.vocab || !c.max_ctx)
    return fail(FRN_EINVAL, "frn_create: zero dimension in config");
  if (c.hidden % c.n_heads || c.hidden / c.n_heads != c.head_dim)
    return fail(FRN_ESHAPE, "frn_create: head_dim %u != hidden %u / n_heads %u", c.head_dim, c.hidden, c.n_heads);
  if (c.n_heads % c.n_kv_heads) return fail(FRN_ESHAPE, "frn_create: %u heads not divisible by %u kv heads", c.n_heads, c.n_kv_heads);
  if (c.head_dim != 64 && c.head_dim != 128) return fail(FRN_ESHAPE, "frn_create: head_dim %u unsupported (64, 128)", c.head_dim);
  if (!attention_supported(c.n_heads, c.n_kv_heads, c.head_dim))
    return fail(FRN_ESHAPE, "frn_create: %u query heads per kv head unsupported (at most 8)", c.n_heads / c.n_kv_heads);
  // activation vectors are staged with 16-byte loads in 16-value chunks;
  // per-format block divisibility is checked per tensor at upload/finalize
  if (c.hidden % 32 || c.ffn % 32) return fail(FRN_ESHAPE, "frn_create: hidden and ffn must be multiples of 32");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= device || device < 0)
    return fail(FRN_ENODEV, "frn_create: no HIP device %d", device);
  HIP_TRY(hipSetDevice(device), "hipSetDevice");
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(FRN_ENODEV, "frn_create: device %d is %s, this library targets gfx950", device, prop.gcnArchName);
  frn_ctx* x = new frn_ctx();
  x->cfg = c;
  x->device = device;

  size_t kvd = (size_t)c.n_kv_heads * c.head_dim, qd = (size_t)c.n_heads * c.head_dim;
  size_t kv_bytes = (size_t)c.n_layers * c.max_ctx * kvd * 4;
  hipError_t e;
  if ((e = hipStreamCreateWithFlags(&x->stream, hipStreamNonBlocking)) || (e = dmalloc(&x->x, c.hidden * 4)) ||
      (e = dmalloc(&x->q, qd * 4)) || (e = dmalloc(&x->k, kvd * 4)) || (e = dmalloc(&x->v, kvd * 4)) ||
      (e = dmalloc(&x->act, (size_t)c.ffn * 4)) ||
      (e = dmalloc(&x->logits, (size_t)c.vocab * 4)) ||
      (e = dmalloc(&x->part, attention_part_floats(c.n_heads, c.head_dim, c.max_ctx) * 4)) ||
      (e = dmalloc(&x->kcache, kv_bytes)) || (e = dmalloc(&x->vcache, kv_bytes)) ||
      (e = dmalloc(&x->rope, (size_t)c.max_ctx * c.head_dim * 4)) || (e = dmalloc(&x->rope_cur, c.head_dim * 4)) ||
      (e = dmalloc(&x->st, sizeof(StepState))) ||
      (e = dmalloc(&x->best_part, ((size_t)c.vocab + 3) / 4 * 8)) ||  // >= lm_head blocks (4+ rows each)
      (e = alloc_prefill(x)) ||
      (e = dmalloc(&x->hist, (size_t)c.max_ctx * 4)) ||
      (e = hipHostMalloc((void**)&x->h_hist, GREEDY_BATCH * 4, hipHostMallocDefault)) ||
      (e = dmalloc(&x->rng, sizeof(SamplerRng))) || (e = dmalloc(&x->att, qd * 4)) ||
      (e = dmalloc(&x->cand_v, (size_t)sampler_blocks(c.vocab) * SAMPLER_MAX_K * 4)) ||
      (e = dmalloc(&x->cand_id, (size_t)sampler_blocks(c.vocab) * SAMPLER_MAX_K * 4)) ||
      (e = dmalloc(&x->recent, SAMPLER_MAX_RECENT * 4)) ||
      (e = hipHostMalloc((void**)&x->h_recent, SAMPLER_MAX_RECENT * 4, hipHostMallocDefault)) ||
      (e = hipHostMalloc((void**)&x->h_rng, sizeof(SamplerRng), hipHostMallocDefault)) ||
      (e = hipHostMalloc((void**)&x->h_st, sizeof(StepState), hipHostMallocDefault))) {
    free_ctx(x);
    return hip_fail(e, "frn_create: allocation");
  }
  // RoPE table (model.rs:207-210): freq = theta^(-2i/hd) via powf, angle in
  // f32, sin/cos from the host libm -- the same calls the CPU path makes.
  std::vector<float> tab((size_t)c.max_ctx * c.head_dim);
  uint32_t half = c.head_dim / 2;
  std::vector<float> freq(half);
  for (uint32_t i = 0; i < half; ++i) freq[i] = powf(c.rope_theta, -2.0f * (float)i / (float)c.head_dim);
  for (uint32_t p = 0; p < c.max_ctx; ++p)
    for (uint32_t i = 0; i < half; ++i) {
      volatile float angle = (float)p * freq[i];
      tab[(size_t)p * c.head_dim + i] = cosf(angle);
      tab[(size_t)p * c.head_dim + half + i] = sinf(angle);
    }
  StepState init{};
  if ((e = hipMemcpy(x->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice)) ||
      (e = hipMemcpy(x->st, &init, sizeof init, hipMemcpyHostToDevice)) ||
      (e = hipMemset(x->kcache, 0, kv_bytes)) || (e = hipMemset(x->vcache, 0, kv_bytes)) ||
      (e = gemv_prepare(std::max(gemv_lds_bytes(c.hidden, true),
                                 std::max(gemv_lds_bytes(c.ffn, false), gemv_lds_bytes(c.n_heads * c.head_dim, false))))) ||
      (e = gemm_prepare())) {
    free_ctx(x);
    return hip_fail(e, "frn_create: init");
  }
  *out = x;
  return FRN_OK;
}

extern "C" void frn_destroy(frn_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  free_ctx(ctx);
}

extern "C" frn_status frn_upload(frn_ctx* ctx, const char* name, uint32_t type, uint64_t out_dim, uint64_t in_dim,
                                 const void* host, size_t bytes) {
  if (!ctx || !name || (!host && bytes)) return fail(FRN_EINVAL, "frn_upload: null argument");
  if (ctx->finalized) return fail(FRN_EINVAL, "frn_upload: context already finalized");
  if (!known_type(type)) return fail(FRN_EDTYPE, "frn_upload: '%s' has ggml type %u without a kernel", name, type);
  uint64_t n = out_dim * in_dim;
  if (in_dim == 0 || out_dim == 0 || n % blk_elems(type))
    return fail(FRN_ESHAPE, "frn_upload: '%s' has %llu elements, not a multiple of %d", name, (unsigned long long)n,
                blk_elems(type));
  if (type != T_F32 && in_dim % blk_elems(type))
    return fail(FRN_ESHAPE, "frn_upload: '%s' in dim %llu not a multiple of %d", name, (unsigned long long)in_dim,
                blk_elems(type));
  size_t want = (size_t)(n / blk_elems(type)) * blk_bytes(type);
  if (bytes != want)
    return fail(FRN_ESHAPE, "frn_upload: '%s' is %zu bytes, expected %zu", name, bytes, want);
  HIP_TRY(hipSetDevice(ctx->device), "hipSetDevice");
  DevTensor t;
  t.type = type;
  t.out = out_dim;
  t.in = in_dim;
  bool vec = out_dim == 1;  // norms and biases: stored dequantized (Tensor::from_gguf)
  t.bytes = vec ? (size_t)n * 4 : bytes;
  // 256 B of slack: allocation granularity keeps tails readable by 16-byte loads
  HIP_TRY(hipMalloc((void**)&t.ptr, t.bytes + 256), "frn_upload: hipMalloc");
  hipError_t e = hipSuccess;
  if (vec && type != T_F32) {
    uint8_t* tmp = nullptr;
    if (!(e = hipMalloc((void**)&tmp, bytes + 256)) && !(e = hipMemcpy(tmp, host, bytes, hipMemcpyHostToDevice)) &&
        !(e = launch_dequant(type, tmp, n, (float*)t.ptr, ctx->stream)))
      e = hipStreamSynchronize(ctx->stream);
    if (tmp) (void)hipFree(tmp);
    t.type = T_F32;
  } else {
    e = hipMemcpy(t.ptr, host, bytes, hipMemcpyHostToDevice);
  }
  if (e) {
    (void)hipFree(t.ptr);
    return hip_fail(e, "frn_upload: copy");
  }
  auto it = ctx->tensors.find(name);
  if (it != ctx->tensors.end()) (void)hipFree(it->second.ptr);
  ctx->tensors[name] = t;
  return FRN_OK;
}

static frn_status need(frn_ctx* c, const std::string& name, uint64_t out, uint64_t in, bool matrix,
                       const DevTensor** dst) {
  auto it = c->tensors.find(name);
  if (it == c->tensors.end()) return fail(FRN_EINVAL, "no tensor named '%s'", name.c_str());
  const DevTensor& t = it->second;
  if (t.out != out || t.in != in)
    return fail(FRN_ESHAPE, "'%s' is [%llu, %llu], expected [%llu, %llu]", name.c_str(), (unsigned long long)t.out,
                (unsigned long long)t.in, (unsigned long long)out, (unsigned long long)in);
  if (matrix && t.type != T_F32 && (in % blk_elems(t.type)))
    return fail(FRN_ESHAPE, "'%s' in dim not a multiple of the block", name.c_str());
  *dst = &t;
  return FRN_OK;
}

// Event pair around one kernel when the step runs eagerly for --timings.
// Replay mode (rcat >= 0): launch only category rcat of layer rlayer (the
// per-step kernels match any layer), reps times back to back.
struct Tick {
  frn_ctx* c;
  bool on;
  size_t n = 0;
  int rcat = -1, rlayer = -1, layer = -1;  // rlayer -1: every layer
  int counted = -2;                        // the last layer counted in `launched`
  uint32_t reps = 0, launched = 0;         // category instances replayed (one per layer)
  template <class F>
  hipError_t replay(int cat, F&& launch) {
    if (cat != rcat || (layer >= 0 && rlayer >= 0 && layer != rlayer)) return hipSuccess;
    if (layer != counted || layer < 0) {  // a category of two launches in a layer counts once
      launched += reps;
      counted = layer;
    }
    for (uint32_t r = 0; r < reps; ++r)
      if (hipError_t e = launch()) return e;
    return hipSuccess;
  }
  hipError_t begin(int cat) {
    if (!on) return hipSuccess;
    if (c->ev.size() < 2 * (n + 1)) {
      for (int k = 0; k < 2; ++k) {
        hipEvent_t e;
        hipError_t r = hipEventCreate(&e);
        if (r) return r;
        c->ev.push_back(e);
      }
      c->ev_cat.resize(c->ev.size() / 2);
    }
    c->ev_cat[n] = cat;
    return hipEventRecord(c->ev[2 * n], c->stream);
  }
  hipError_t end(hipError_t launch) {
    if (!on || launch) return launch;
    hipError_t r = hipEventRecord(c->ev[2 * n + 1], c->stream);
    ++n;
    return r;
  }
};

// Record one decode step on ctx->stream: under stream capture for the
// replayed graphs, or eagerly with per-kernel events when tk.on.
static hipError_t record_step(frn_ctx* c, bool with_logits, Tick& tk) {
  const frn_config& g = c->cfg;
  tk.counted = -2;
  hipStream_t s = c->stream;
  hipError_t e;
  float scale = 1.0f / sqrtf((float)g.head_dim);  // model.rs:384
#define TIMED(cat, call) \
  (tk.rcat >= 0 ? (e = tk.replay(cat, [&]() { return (call); })) : ((e = tk.begin(cat)) ? e : (e = tk.end(call))))
  if (TIMED(CAT_EMBED, launch_embed(c->embd->ptr, c->embd->type, g.hidden,
                                    (uint32_t)type_row_bytes(c->embd->type, g.hidden), c->st, c->x, c->rope,
                                    g.head_dim, c->rope_cur, s)))
    return e;
  auto seg = [&](const DevTensor* w, const DevTensor* w2, const float* bias, float* out, const float* resid) {
    GemvSeg sg{};
    sg.w = w->ptr;
    sg.w2 = w2 ? w2->ptr : nullptr;
    sg.type = w->type;
    sg.rows = (uint32_t)w->out;
    sg.row_bytes = (uint32_t)type_row_bytes(w->type, w->in);
    sg.bias = bias;
    sg.out = out;
    sg.resid = resid;
    return sg;
  };
  auto args = [&](uint32_t in, const float* xin, const float* norm) {
    GemvArgs a{};
    a.in = in;
    a.x = xin;
    a.norm_w = norm;
    a.eps = g.rms_eps;
    a.n_seg = 1;
    return a;
  };
  const uint32_t H = g.hidden, QD = g.n_heads * g.head_dim;
  for (uint32_t l = 0; l < g.n_layers; ++l) {
    const LayerPtrs& L = c->layers[l];
    tk.layer = (int)l;
    // rmsnorm + q/k/v GEMVs + biases in one launch (model.rs:456-459)
    GemvArgs qkv = args(H, c->x, L.attn_norm);
    qkv.n_seg = 3;
    qkv.seg[0] = seg(L.wq, nullptr, L.bq, c->q, nullptr);
    qkv.seg[1] = seg(L.wk, nullptr, L.bk, c->k, nullptr);
    qkv.seg[2] = seg(L.wv, nullptr, L.bv, c->v, nullptr);
    if (TIMED(CAT_QKV, launch_gemv(qkv, GEMV_STORE, s))) return e;
    // rope, KV append, attention (model.rs:460-467)
    size_t lo = (size_t)l * g.max_ctx * g.n_kv_heads * g.head_dim;
    const uint32_t cap = c->rec_long ? ATTENTION_MAX_SPLITS_LONG : ATTENTION_MAX_SPLITS;
    if (TIMED(CAT_ATTN, launch_attention(c->q, c->k, c->v, c->rope_cur, c->kcache + lo, c->vcache + lo, g.n_heads,
                                         g.n_kv_heads, g.head_dim, g.max_ctx, scale, c->part, c->st, cap,
                                         c->rec_long ? 0u : c->rec_splits, s)))
      return e;
    if (c->rec_long) {
      // long contexts: up to 128 splits, merged once (model.rs:436-438),
      // then o-proj + residual on the merged rows (model.rs:469-470)
      if (TIMED(CAT_ATTN, launch_attn_merge(c->part, c->att, g.n_heads, g.head_dim, g.max_ctx, c->st, s))) return e;
      GemvArgs o = args(QD, c->att, nullptr);
      o.seg[0] = seg(L.wo, nullptr, nullptr, c->x, c->x);
      if (TIMED(CAT_OPROJ, launch_gemv(o, GEMV_RESID, s))) return e;
    } else {
      // merge of the attention splits + o-proj + residual (model.rs:436-438, 469-470)
      GemvArgs o = args(QD, nullptr, nullptr);
      o.seg[0] = seg(L.wo, nullptr, nullptr, c->x, c->x);
      o.att_part = c->part;
      o.st = c->st;
      o.att_ms = attention_splits(g.max_ctx);
      o.att_hd = g.head_dim;
      o.att_part_bytes = (uint32_t)(attention_part_floats(g.n_heads, g.head_dim, g.max_ctx) * 4);
      if (TIMED(CAT_OPROJ, launch_gemv(o, GEMV_RESID_ATT, s))) return e;
    }
    // rmsnorm + gate/up + SwiGLU (model.rs:473-476)
    GemvArgs gu = args(H, c->x, L.ffn_norm);
    gu.seg[0] = seg(L.gate, L.up, nullptr, c->act, nullptr);
    if (TIMED(CAT_GATEUP, launch_gemv(gu, GEMV_SWIGLU, s))) return e;
    // down + residual (model.rs:476-477)
    GemvArgs dn = args(g.ffn, c->act, nullptr);
    dn.seg[0] = seg(L.down, nullptr, nullptr, c->x, c->x);
    if (TIMED(CAT_DOWN, launch_gemv(dn, GEMV_RESID, s))) return e;
  }
  tk.layer = -1;
  if (with_logits) {  // last_row_logits + argmax (model.rs:594-600, generate.rs:69-77)
    GemvArgs lm = args(H, c->x, c->out_norm);
    lm.seg[0] = seg(c->lm_head, nullptr, nullptr, c->logits, nullptr);
    lm.best = c->best_part;
    if (TIMED(CAT_LMHEAD, launch_gemv(lm, GEMV_ARGMAX, s, &c->n_best))) return e;
  }
  TIMED(CAT_STEP, launch_step_end(c->st, with_logits ? c->best_part : nullptr, c->n_best,
                                  with_logits ? c->hist : nullptr, s));
#undef TIMED
  return e;
}

// Eager step with per-kernel events, accumulated into the dashboard.
static hipError_t timed_step(frn_ctx* c, bool with_logits) {
  Tick tk{c, true};
  hipError_t e = record_step(c, with_logits, tk);
  if (e) return e;
  if ((e = hipEventSynchronize(c->ev[2 * tk.n - 1]))) return e;
  for (size_t i = 0; i < tk.n; ++i) {
    float ms = 0.f;
    if ((e = hipEventElapsedTime(&ms, c->ev[2 * i], c->ev[2 * i + 1]))) return e;
    c->t_ms[c->ev_cat[i]] += ms;
    c->t_calls[c->ev_cat[i]] += 1;
  }
  return hipSuccess;
}

// Short-context split counts that get their own step graphs: every count a
// step within max_ctx can have (at most 16, up to ATTENTION_LONG_FROM).
static uint32_t exact_forms(const frn_ctx* c) {
  const uint32_t t = std::min<uint32_t>(c->cfg.max_ctx, ATTENTION_LONG_FROM);
  return std::min<uint32_t>((t + ATTENTION_CHUNK - 1) / ATTENTION_CHUNK, ATTENTION_MAX_SPLITS);
}
// The exact-split graph index + 1 for a step over T positions, 0 for none.
static uint32_t exact_splits(const frn_ctx* c, uint32_t T) {
  if (T > ATTENTION_LONG_FROM) return 0;
  const uint32_t n = (T + ATTENTION_CHUNK - 1) / ATTENTION_CHUNK;
  return n <= exact_forms(c) && c->g_exact[n - 1] ? n : 0;
}

static frn_status capture(frn_ctx* c, bool with_logits, hipGraph_t* graph, hipGraphExec_t* exec,
                          uint32_t steps = 1) {
  HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  Tick tk{c, false};
  hipError_t e = hipSuccess;
  for (uint32_t i = 0; i < steps && !e; ++i) e = record_step(c, with_logits, tk);
  hipGraph_t gr = nullptr;
  hipError_t e2 = hipStreamEndCapture(c->stream, &gr);
  if (e) {
    if (gr) hipGraphDestroy(gr);
    return hip_fail(e, "recording decode step");
  }
  if (e2) return hip_fail(e2, "hipStreamEndCapture");
  *graph = gr;
  HIP_TRY(hipGraphInstantiate(exec, gr, nullptr, nullptr, 0), "hipGraphInstantiate");
  return FRN_OK;
}

// Decides whether the resident decode kernel serves this model and
// prepares it: the per-layer weight table, the exchange buffers and the
// launch arguments.  Unsupported shapes keep the step graphs (res_why).
static frn_status setup_resident(frn_ctx* c) {
  const frn_config& g = c->cfg;
  c->res_ok = false;
  if (g.flags & FRN_FLAG_NO_RESIDENT) {
    c->res_why = "disabled by FRN_FLAG_NO_RESIDENT";
    return FRN_OK;
  }
  if (!(g.flags & FRN_FLAG_RESIDENT) && !kResidentDefault) {
    c->res_why = "the step graphs are the default (FRN_FLAG_RESIDENT selects the resident kernel)";
    return FRN_OK;
  }
  if (g.flags & FRN_FLAG_EAGER) {
    c->res_why = "FRN_FLAG_EAGER runs the step kernels one by one";
    return FRN_OK;
  }
  hipDeviceProp_t prop;
  int coop = 0;
  HIP_TRY(hipGetDeviceProperties(&prop, c->device), "hipGetDeviceProperties");
  HIP_TRY(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, c->device), "hipDeviceGetAttribute");
  if (prop.multiProcessorCount != (int)RES_BLOCKS || !coop) {
    c->res_why = "needs 256 CUs and cooperative launches";
    return FRN_OK;
  }
  std::vector<uint32_t> types;
  uint32_t o_gran = 64;
  for (const LayerPtrs& L : c->layers) {
    for (const DevTensor* t : {L.wq, L.wk, L.wv, L.wo, L.gate, L.up, L.down}) types.push_back(t->type);
    if (L.wo->type == T_Q6_K) o_gran = 128;
  }
  uint32_t fset = 0;
  if (const char* why = res_unsupported(g.hidden, g.ffn, g.n_heads, g.n_kv_heads, g.head_dim, types.data(),
                                        types.size(), c->lm_head->type, o_gran, &fset)) {
    c->res_why = why;
    return FRN_OK;
  }
  const ResLayout lay = res_layout(g.hidden, g.ffn, g.n_heads, g.n_kv_heads, g.head_dim);
  c->res_ex_bytes = res_exchange_pairs(lay) * 8;
  std::vector<ResLayer> tab(g.n_layers);
  for (uint32_t l = 0; l < g.n_layers; ++l) {
    const LayerPtrs& L = c->layers[l];
    ResLayer& r = tab[l];
    r.wq = L.wq->ptr; r.wk = L.wk->ptr; r.wv = L.wv->ptr; r.wo = L.wo->ptr;
    r.wg = L.gate->ptr; r.wu = L.up->ptr; r.wd = L.down->ptr;
    r.bq = L.bq; r.bk = L.bk; r.bv = L.bv; r.an = L.attn_norm; r.fn = L.ffn_norm;
    r.tq = L.wq->type; r.tk = L.wk->type; r.tv = L.wv->type; r.to = L.wo->type; r.tg = L.gate->type;
    r.td = L.down->type;
    r.rq = (uint32_t)type_row_bytes(r.tq, L.wq->in); r.rk = (uint32_t)type_row_bytes(r.tk, L.wk->in);
    r.rv = (uint32_t)type_row_bytes(r.tv, L.wv->in); r.ro = (uint32_t)type_row_bytes(r.to, L.wo->in);
    r.rg = (uint32_t)type_row_bytes(r.tg, L.gate->in); r.rd = (uint32_t)type_row_bytes(r.td, L.down->in);
  }
  hipError_t e;
  if ((e = dmalloc(&c->d_layers, tab.size() * sizeof(ResLayer))) || (e = dmalloc(&c->d_res, sizeof(ResArgs))) ||
      (e = dmalloc(&c->res_ex, c->res_ex_bytes)) || (e = dmalloc(&c->res_ctl, sizeof(ResCtl))) ||
      (e = hipHostMalloc((void**)&c->h_res, sizeof(ResArgs), hipHostMallocDefault)) ||
      (e = hipHostMalloc((void**)&c->h_ctl, sizeof(ResCtl), hipHostMallocDefault)) ||
      (e = hipHostMalloc((void**)&c->h_ids, RES_STEPS * 4, hipHostMallocDefault)) ||
      (e = hipMemcpy(c->d_layers, tab.data(), tab.size() * sizeof(ResLayer), hipMemcpyHostToDevice)) ||
      (e = hipMemset(c->res_ex, 0, c->res_ex_bytes)) || (e = res_prepare()))
    return hip_fail(e, "resident decode setup");
  ResArgs& a = *c->h_res;
  memset(&a, 0, sizeof a);
  a.layers = c->d_layers;
  a.L = g.n_layers; a.H = g.hidden; a.F = g.ffn; a.nh = g.n_heads; a.nkv = g.n_kv_heads; a.hd = g.head_dim;
  a.V = g.vocab; a.max_ctx = g.max_ctx;
  a.eps = g.rms_eps;
  a.scale = 1.0f / sqrtf((float)g.head_dim);  // model.rs:384
  a.embd = c->embd->ptr; a.te = c->embd->type; a.rbe = (uint32_t)type_row_bytes(c->embd->type, g.hidden);
  a.lm = c->lm_head->ptr; a.tl = c->lm_head->type; a.rbl = (uint32_t)type_row_bytes(c->lm_head->type, g.hidden);
  a.onorm = c->out_norm;
  a.kc = c->kcache; a.vc = c->vcache; a.rope = c->rope;
  a.logits = c->logits; a.hist = c->hist; a.st = c->st;
  a.loc = c->res_ex;
  a.glb = c->res_ex + (size_t)RES_XCDS * 2 * lay.loc_stride;
  a.lay = lay;
  a.ctl = c->res_ctl;
  a.fset = fset;
  if (const char* o = getenv("FRN_RESIDENT_OPTS")) a.opts = (uint32_t)strtoul(o, nullptr, 0);
  c->res_epoch = 0;
  c->res_ok = true;
  c->res_why = "";
  return FRN_OK;
}

extern "C" frn_status frn_resident_trace(frn_ctx* c, uint32_t n_steps, uint64_t* host_out, size_t n) {
  if (!c) return fail(FRN_EINVAL, "frn_resident_trace: null context");
  if (!c->res_ok) return fail(FRN_EINVAL, "frn_resident_trace: the resident decode kernel is not in use");
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  const size_t need = (size_t)n_steps * (c->cfg.n_layers + 1) * RES_TR_K * RES_BLOCKS;
  if (!host_out) {
    if (need > c->res_trace_n) {
      if (c->res_trace) HIP_TRY(hipFree(c->res_trace), "hipFree");
      c->res_trace = nullptr;
      c->res_trace_n = 0;
      HIP_TRY(hipMalloc((void**)&c->res_trace, need * 8), "trace buffer");
      c->res_trace_n = need;
    }
    if (need) HIP_TRY(hipMemset(c->res_trace, 0, need * 8), "trace clear");
    c->res_trace_arm = n_steps;
    return FRN_OK;
  }
  const size_t k = std::min(n, std::min(need, c->res_trace_n));
  HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  if (k) HIP_TRY(hipMemcpy(host_out, c->res_trace, k * 8, hipMemcpyDeviceToHost), "trace copy");
  return FRN_OK;
}

extern "C" frn_status frn_decode_engine(frn_ctx* c, uint32_t* resident, char* reason, size_t reason_len) {
  if (!c || !resident) return fail(FRN_EINVAL, "frn_decode_engine: null argument");
  *resident = c->res_ok ? 1u : 0u;
  if (reason && reason_len) snprintf(reason, reason_len, "%s", c->res_why.c_str());
  return FRN_OK;
}

// n greedy steps through resident launches of up to RES_STEPS steps; the
// kernel itself stops after a step whose id is a stop id.  Ids go to out.
static frn_status res_decode(frn_ctx* c, uint32_t id, uint32_t n, const uint32_t* stop_ids, uint32_t n_stop,
                             uint32_t* out, uint32_t* n_done) {
  const frn_config& g = c->cfg;
  *n_done = 0;
  if (id != c->last_next) {
    c->h_st->tok = id;
    HIP_TRY(hipMemcpyAsync((char*)c->st + offsetof(StepState, tok), &c->h_st->tok, 4, hipMemcpyHostToDevice, c->stream),
            "token upload");
  }
  uint32_t done = 0;
  while (done < n) {
    const uint32_t b = std::min(n - done, RES_STEPS), p0 = c->len;
    if ((uint64_t)c->res_epoch + res_epochs(b, g.n_layers) >= 0x7FFFFFFFull) {  // epochs restart on cleared pairs
      HIP_TRY(hipMemsetAsync(c->res_ex, 0, c->res_ex_bytes, c->stream), "exchange reset");
      c->res_epoch = 0;
    }
    ResArgs& a = *c->h_res;
    a.n_steps = b;
    a.n_stop = n_stop;
    for (uint32_t k = 0; k < n_stop; ++k) a.stop[k] = stop_ids[k];
    a.epoch0 = c->res_epoch;
    c->res_epoch += res_epochs(b, g.n_layers);
    a.trace = c->res_trace_arm ? c->res_trace : nullptr;
    a.trace_steps = c->res_trace_arm;
    c->res_trace_arm = 0;
    HIP_TRY(launch_resident(c->h_res, c->d_res, c->stream), "resident decode launch");
    HIP_TRY(hipMemcpyAsync(c->h_ctl, c->res_ctl, sizeof(ResCtl), hipMemcpyDeviceToHost, c->stream), "status read-back");
    HIP_TRY(hipMemcpyAsync(c->h_ids, c->hist + p0, (size_t)b * 4, hipMemcpyDeviceToHost, c->stream), "id read-back");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    const uint32_t k = c->h_ctl->n_done;
    if (c->h_ctl->err || k == 0 || k > b) {
      const uint32_t err = c->h_ctl->err;
      c->res_ok = false;
      c->res_why = "a resident launch failed";
      c->last_next = 0xFFFFFFFFu;
      c->have_logits = false;
      return fail(FRN_EHIP,
                  "resident decode: %s (code %u, layer %u, phase %u); the context decodes with the step graphs from now on",
                  (err >> 24) == (RES_ERR_LAYOUT >> 24) ? "blocks not spread 32 per XCD" : "a wait gave up",
                  err >> 24, (err >> 8) & 0xFFFFu, err & 0xFFu);
    }
    memcpy(out + done, c->h_ids, (size_t)k * 4);
    done += k;
    c->len += k;
    if (k < b) break;  // stopped at a stop id (generate.rs:125-127)
  }
  *n_done = done;
  c->last_next = out[done - 1];
  c->have_logits = true;
  return FRN_OK;
}

extern "C" frn_status frn_finalize(frn_ctx* c) {
  if (!c) return fail(FRN_EINVAL, "frn_finalize: null context");
  if (c->finalized) return FRN_OK;
  const frn_config& g = c->cfg;
  uint64_t H = g.hidden, qd = (uint64_t)g.n_heads * g.head_dim, kd = (uint64_t)g.n_kv_heads * g.head_dim;
  frn_status st;
  const DevTensor* t;
  // Model::load's tensor set (model.rs:147-161, 522-545)
  if ((st = need(c, "token_embd.weight", g.vocab, H, true, &c->embd))) return st;
  if ((st = need(c, "output_norm.weight", 1, H, false, &t))) return st;
  c->out_norm = (const float*)t->ptr;
  if (c->tensors.count("output.weight")) {
    if ((st = need(c, "output.weight", g.vocab, H, true, &c->lm_head))) return st;
  } else {
    c->lm_head = c->embd;
  }
  c->layers.resize(g.n_layers);
  char nm[96];
  for (uint32_t l = 0; l < g.n_layers; ++l) {
    LayerPtrs& L = c->layers[l];
    auto vec = [&](const char* suf, uint64_t n, const float** dst) {
      snprintf(nm, sizeof nm, "blk.%u.%s", l, suf);
      const DevTensor* tt;
      frn_status s2 = need(c, nm, 1, n, false, &tt);
      if (!s2) *dst = (const float*)tt->ptr;
      return s2;
    };
    auto mat = [&](const char* suf, uint64_t o, uint64_t i, const DevTensor** dst) {
      snprintf(nm, sizeof nm, "blk.%u.%s", l, suf);
      return need(c, nm, o, i, true, dst);
    };
    if ((st = vec("attn_norm.weight", H, &L.attn_norm)) || (st = mat("attn_q.weight", qd, H, &L.wq)) ||
        (st = vec("attn_q.bias", qd, &L.bq)) || (st = mat("attn_k.weight", kd, H, &L.wk)) ||
        (st = vec("attn_k.bias", kd, &L.bk)) || (st = mat("attn_v.weight", kd, H, &L.wv)) ||
        (st = vec("attn_v.bias", kd, &L.bv)) || (st = mat("attn_output.weight", H, qd, &L.wo)) ||
        (st = vec("ffn_norm.weight", H, &L.ffn_norm)) || (st = mat("ffn_gate.weight", g.ffn, H, &L.gate)) ||
        (st = mat("ffn_up.weight", g.ffn, H, &L.up)) || (st = mat("ffn_down.weight", H, g.ffn, &L.down)))
      return st;
    if (L.gate->type != L.up->type)
      return fail(FRN_EDTYPE, "blk.%u: ffn_gate and ffn_up must share a type for the fused SwiGLU kernel", l);
  }
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  if ((st = setup_resident(c))) return st;
  if (!(g.flags & FRN_FLAG_EAGER)) {
    for (int lng = 0; lng < (g.max_ctx > ATTENTION_LONG_FROM ? 2 : 1); ++lng) {
      c->rec_long = lng;
      if ((st = capture(c, true, &c->graph_step[lng], &c->g_step[lng]))) return st;
      if ((st = capture(c, false, &c->graph_prefill[lng], &c->g_prefill[lng]))) return st;
      if ((st = capture(c, true, &c->graph_multi[lng], &c->g_multi[lng], GREEDY_MULTI))) return st;
    }
    c->rec_long = false;
    // decode steps whose attention grid is exactly their splits
    for (uint32_t n = 1; n <= exact_forms(c); ++n) {
      c->rec_splits = n;
      if ((st = capture(c, true, &c->graph_exact[n - 1], &c->g_exact[n - 1]))) break;
      if ((st = capture(c, true, &c->graph_exact_multi[n - 1], &c->g_exact_multi[n - 1], GREEDY_MULTI))) break;
    }
    c->rec_splits = 0;
    if (st) return st;
  }
  c->finalized = true;
  return FRN_OK;
}

// Run one position with token `tok` (already validated); with_logits picks
// the graph that ends in lm_head + argmax (the exact-split graph of the
// step's position where there is one).  on_device: the token is the
// previous step's argmax, already in StepState::tok.
static frn_status run_step(frn_ctx* c, uint32_t tok, bool with_logits, bool on_device = false) {
  if (!on_device && tok != c->last_next) {
    c->h_st->tok = tok;
    HIP_TRY(hipMemcpyAsync((char*)c->st + offsetof(StepState, tok), &c->h_st->tok, 4, hipMemcpyHostToDevice, c->stream),
            "token upload");
  }
  // the long-context form once the step covers more than ATTENTION_LONG_FROM positions
  c->rec_long = c->len + 1 > ATTENTION_LONG_FROM;
  if (c->timing) {
    HIP_TRY(timed_step(c, with_logits), "timed step");
  } else if (c->cfg.flags & FRN_FLAG_EAGER) {
    Tick tk{c, false};
    HIP_TRY(record_step(c, with_logits, tk), "eager step");
  } else {
    const uint32_t n = with_logits ? exact_splits(c, c->len + 1) : 0u;
    HIP_TRY(hipGraphLaunch(n ? c->g_exact[n - 1] : with_logits ? c->g_step[c->rec_long] : c->g_prefill[c->rec_long],
                           c->stream),
            "hipGraphLaunch");
  }
  c->len += 1;
  c->last_next = 0xFFFFFFFFu;
  return FRN_OK;
}

static frn_status check_ready(frn_ctx* c, uint32_t n) {
  if (!c) return fail(FRN_EINVAL, "null context");
  if (!c->finalized) return fail(FRN_EINVAL, "context not finalized");
  if ((uint64_t)c->len + n > c->cfg.max_ctx)
    return fail(FRN_ECTX_OVERFLOW, "context overflow: %u + %u > max_ctx %u", c->len, n, c->cfg.max_ctx);
  return FRN_OK;
}

static frn_status read_next(frn_ctx* c, uint32_t* next_id) {
  HIP_TRY(hipMemcpyAsync(&c->h_st->next_tok, (char*)c->st + offsetof(StepState, next_tok), 4, hipMemcpyDeviceToHost,
                         c->stream),
          "next-id read-back");
  HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  c->last_next = c->h_st->next_tok;
  c->have_logits = true;
  if (next_id) *next_id = c->last_next;
  return FRN_OK;
}

// The prompt as blocks of rows (forward_cached with seq > 1, model.rs:579-592):
// each block goes through every layer -- rmsnorm + q/k/v GEMMs (MFMA), RoPE
// + KV append, causal attention over the cache, o-proj + residual, rmsnorm +
// gate/up + SwiGLU, down + residual -- then the last row of the last block
// gets the final norm, the lm_head GEMV and the argmax.
static hipError_t prefill_rows(frn_ctx* c, const uint32_t* ids, uint32_t n) {
  const frn_config& g = c->cfg;
  hipStream_t s = c->stream;
  hipError_t e;
  const uint32_t H = g.hidden, QD = g.n_heads * g.head_dim, KVD = g.n_kv_heads * g.head_dim;
  const float scale = 1.0f / sqrtf((float)g.head_dim);  // model.rs:384
  uint32_t m = 0;
  for (uint32_t c0 = 0; c0 < n; c0 += c->pf_rows) {
    m = std::min(c->pf_rows, n - c0);
    const uint32_t pos0 = c->len + c0;
    if ((e = hipMemcpyAsync(c->pf_ids, ids + c0, (size_t)m * 4, hipMemcpyHostToDevice, s))) return e;
    if ((e = launch_embed_rows(c->embd->ptr, c->embd->type, H, (uint32_t)type_row_bytes(c->embd->type, H), c->pf_ids,
                               m, c->pf_x, s)))
      return e;
    // the planes of an operand [m][K]: hi first, lo after
    auto lo_of = [&](uint16_t* hi, uint32_t K) { return hi + (size_t)m * K; };
    // the group sums a Q4_K weight reads beside its input planes
    auto group_sums = [&](GemmArgs& ga, uint16_t* a, uint32_t K) {
      ga.x_hi = c->pf_xg;
      ga.x_lo = c->pf_xg + (size_t)m * (K / 32);
      return launch_group_sums(a, lo_of(a, K), m, K, c->pf_xg, c->pf_xg + (size_t)m * (K / 32), s);
    };
    auto gemm = [&](const DevTensor* w, const DevTensor* w2, uint16_t* a, uint32_t K, const float* bias, float* out,
                    uint16_t* o_planes, uint32_t ldo, GemmMode mode) {
      GemmArgs ga{};
      ga.a_hi = a;
      ga.a_lo = lo_of(a, K);
      if (w->type == T_Q4_K) {
        if (a == c->pf_xs) {  // written with its group sums by launch_rows_split
          ga.x_hi = c->pf_xg;
          ga.x_lo = c->pf_xg + (size_t)m * (K / 32);
        } else if (hipError_t r = group_sums(ga, a, K)) {
          return r;
        }
      }
      ga.partial = c->pf_part;
      ga.partial_floats = PREFILL_PARTIAL_FLOATS;
      ga.w = w->ptr;
      ga.w2 = w2 ? w2->ptr : nullptr;
      ga.type = w->type;
      ga.row_bytes = (uint32_t)type_row_bytes(w->type, w->in);
      ga.bias = bias;
      ga.out = out;
      ga.o_hi = o_planes;
      ga.o_lo = o_planes ? lo_of(o_planes, ldo) : nullptr;
      ga.ldo = ldo;
      ga.P = m;
      ga.N = (uint32_t)w->out;
      ga.K = K;
      return launch_gemm(ga, mode, s);
    };
    // q, k and v: one launch for the matrices that share a format
    auto qkv = [&](const LayerPtrs& L) {
      const DevTensor* w[3] = {L.wq, L.wk, L.wv};
      const float* b[3] = {L.bq, L.bk, L.bv};
      float* o[3] = {c->pf_q, c->pf_k, c->pf_v};
      const uint32_t ld[3] = {QD, KVD, KVD};
      bool done[3] = {false, false, false};
      for (int i = 0; i < 3; ++i) {
        if (done[i]) continue;
        GemmArgs ga{};
        ga.a_hi = c->pf_xs;
        ga.a_lo = lo_of(c->pf_xs, H);
        ga.x_hi = c->pf_xg;  // the group sums launch_rows_split wrote with pf_xs
        ga.x_lo = c->pf_xg + (size_t)m * (H / 32);
        ga.partial = c->pf_part;
        ga.partial_floats = PREFILL_PARTIAL_FLOATS;
        ga.w = w[i]->ptr;
        ga.type = w[i]->type;
        ga.row_bytes = (uint32_t)type_row_bytes(w[i]->type, w[i]->in);
        ga.bias = b[i];
        ga.out = o[i];
        ga.ldo = ld[i];
        ga.P = m;
        ga.N = (uint32_t)w[i]->out;
        ga.K = H;
        done[i] = true;
        for (int k = i + 1; k < 3; ++k)
          if (!done[k] && w[k]->type == w[i]->type) {
            ga.more[ga.n_more++] = GemmArgs::More{w[k]->ptr, b[k], o[k], (uint32_t)w[k]->out, ld[k]};
            done[k] = true;
          }
        if (hipError_t r = launch_gemm(ga, GEMM_STORE, s)) return r;
      }
      return hipSuccess;
    };
    for (uint32_t l = 0; l < g.n_layers; ++l) {
      const LayerPtrs& L = c->layers[l];
      const size_t lo = (size_t)l * g.max_ctx * KVD;
      uint16_t* xsh = H % 32 ? nullptr : c->pf_xg;  // group sums beside the split rows
      uint16_t* xsl = xsh ? c->pf_xg + (size_t)m * (H / 32) : nullptr;
      if ((e = launch_rows_split(c->pf_x, m, H, L.attn_norm, g.rms_eps, c->pf_xs, lo_of(c->pf_xs, H), xsh, xsl, s)) ||
          (e = qkv(L)) ||
          (e = launch_rope_kv_rows(c->pf_q, c->pf_k, c->pf_v, c->rope, c->kcache + lo, c->vcache + lo, g.n_heads,
                                   g.n_kv_heads, g.head_dim, pos0, m, s)) ||
          (e = launch_kv_split(c->kcache + lo, c->vcache + lo, pos0 + m, KVD, c->pf_kvs, s)) ||
          (e = launch_attn_rows(c->pf_q, c->pf_kvs, c->pf_att, lo_of(c->pf_att, QD), g.n_heads, g.n_kv_heads,
                                g.head_dim, pos0, m, scale, c->pf_attp, s)) ||
          (e = gemm(L.wo, nullptr, c->pf_att, QD, nullptr, c->pf_x, nullptr, H, GEMM_RESID)) ||
          (e = launch_rows_split(c->pf_x, m, H, L.ffn_norm, g.rms_eps, c->pf_xs, lo_of(c->pf_xs, H), xsh, xsl, s)) ||
          (e = gemm(L.gate, L.up, c->pf_xs, H, nullptr, nullptr, c->pf_act, g.ffn, GEMM_SWIGLU)) ||
          (e = gemm(L.down, nullptr, c->pf_act, g.ffn, nullptr, c->pf_x, nullptr, H, GEMM_RESID)))
        return e;
    }
  }
  // last_row_logits (model.rs:594-600) + argmax (generate.rs:69-77)
  GemvArgs lm{};
  lm.in = H;
  lm.x = c->pf_x + (size_t)(m - 1) * H;
  lm.norm_w = c->out_norm;
  lm.eps = g.rms_eps;
  lm.n_seg = 1;
  lm.seg[0].w = c->lm_head->ptr;
  lm.seg[0].type = c->lm_head->type;
  lm.seg[0].rows = (uint32_t)c->lm_head->out;
  lm.seg[0].row_bytes = (uint32_t)type_row_bytes(c->lm_head->type, c->lm_head->in);
  lm.seg[0].out = c->logits;
  lm.best = c->best_part;
  uint32_t nb = 0;
  if ((e = launch_gemv(lm, GEMV_ARGMAX, s, &nb))) return e;
  return launch_prefill_end(c->st, c->best_part, nb, n, s);
}

extern "C" frn_status frn_prefill(frn_ctx* c, const uint32_t* ids, uint32_t n, uint32_t* next_id) {
  frn_status st;
  if ((st = check_ready(c, n))) return st;
  if (!ids || n == 0) return fail(FRN_EINVAL, "frn_prefill: empty prompt");
  for (uint32_t i = 0; i < n; ++i)
    if (ids[i] >= c->cfg.vocab) return fail(FRN_ETOKEN, "token id %u out of range (vocab %u)", ids[i], c->cfg.vocab);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  c->last_next = 0xFFFFFFFFu;
  if (n == 1 || (c->cfg.flags & FRN_FLAG_STEPWISE_PREFILL)) {  // one decode step per position
    for (uint32_t i = 0; i < n; ++i) {
      // per-position token upload: make sure the previous copy has landed
      if (i) HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
      if ((st = run_step(c, ids[i], i + 1 == n))) return st;
    }
  } else {
    HIP_TRY(prefill_rows(c, ids, n), "prefill");
    c->len += n;
  }
  return read_next(c, next_id);
}

extern "C" frn_status frn_decode(frn_ctx* c, uint32_t id, uint32_t* next_id) {
  frn_status st;
  if ((st = check_ready(c, 1))) return st;
  if (id >= c->cfg.vocab) return fail(FRN_ETOKEN, "token id %u out of range (vocab %u)", id, c->cfg.vocab);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  if (c->res_ok && !c->timing && !c->step_timing) {
    uint32_t nxt = 0, k = 0;
    if ((st = res_decode(c, id, 1, nullptr, 0, &nxt, &k))) return st;
    if (next_id) *next_id = nxt;
    return FRN_OK;
  }
  if (c->step_timing) HIP_TRY(hipEventRecord(c->st_ev[0], c->stream), "hipEventRecord");
  // run_step skips the upload when id is the device's own argmax
  if ((st = run_step(c, id, true))) return st;
  if (c->step_timing) HIP_TRY(hipEventRecord(c->st_ev[1], c->stream), "hipEventRecord");
  if ((st = read_next(c, next_id))) return st;
  if (c->step_timing) {
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, c->st_ev[0], c->st_ev[1]), "hipEventElapsedTime");
    c->step_ms.push_back(ms);
  }
  return FRN_OK;
}

// Greedy decode without a host round trip per step (generate.rs:110-136 at
// temperature 0): the step graphs go out back to back, each step's embed
// reading the previous step's argmax from StepState::tok, and the host
// reads one batch of ids (hist[pos], written by the step-end kernel) per
// synchronisation.  A stop id ends the loop after the step that produced
// it, as generate.rs:125-127 would; the position count is rolled back over
// the steps of the batch that ran past it (their KV rows lie beyond the
// cache length, where no later step reads before overwriting them).
extern "C" frn_status frn_decode_greedy(frn_ctx* c, uint32_t id, uint32_t n, const uint32_t* stop_ids,
                                        uint32_t n_stop, uint32_t* out_ids, uint32_t* n_done) {
  frn_status st;
  if (n_done) *n_done = 0;
  if ((st = check_ready(c, n))) return st;
  if (n && !out_ids) return fail(FRN_EINVAL, "frn_decode_greedy: null out_ids");
  if (n_stop && !stop_ids) return fail(FRN_EINVAL, "frn_decode_greedy: null stop_ids");
  if (id >= c->cfg.vocab) return fail(FRN_ETOKEN, "token id %u out of range (vocab %u)", id, c->cfg.vocab);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  if (n == 0) return FRN_OK;
  if (c->res_ok && !c->timing && !c->step_timing && n_stop <= RES_MAX_STOP) {
    uint32_t k = 0;
    st = res_decode(c, id, n, stop_ids, n_stop, out_ids, &k);
    if (n_done) *n_done = k;
    return st;
  }
  uint32_t done = 0;
  bool stopped = false, rolled = false;
  while (done < n && !stopped) {
    const uint32_t b = std::min<uint32_t>(n - done, GREEDY_BATCH), p0 = c->len;
    if (c->step_timing) HIP_TRY(hipEventRecord(c->st_ev[0], c->stream), "hipEventRecord");
    for (uint32_t i = 0; i < b;) {
      // GREEDY_MULTI steps in one graph when the token is already on the
      // device and all of them run the same attention form (one graph per
      // step while step times are recorded)
      const bool same_form = (c->len + 1 > ATTENTION_LONG_FROM) == (c->len + GREEDY_MULTI > ATTENTION_LONG_FROM);
      if (done + i > 0 && b - i >= GREEDY_MULTI && same_form && !c->timing && !c->step_timing &&
          !(c->cfg.flags & FRN_FLAG_EAGER)) {
        c->rec_long = c->len + 1 > ATTENTION_LONG_FROM;
        const uint32_t n = exact_splits(c, c->len + 1);
        const bool exact = n && n == exact_splits(c, c->len + GREEDY_MULTI);
        HIP_TRY(hipGraphLaunch(exact ? c->g_exact_multi[n - 1] : c->g_multi[c->rec_long], c->stream), "hipGraphLaunch");
        c->len += GREEDY_MULTI;
        c->last_next = 0xFFFFFFFFu;
        i += GREEDY_MULTI;
        continue;
      }
      if ((st = run_step(c, id, true, done + i > 0))) return st;
      if (c->step_timing) HIP_TRY(hipEventRecord(c->st_ev[i + 1], c->stream), "hipEventRecord");
      ++i;
    }
    HIP_TRY(hipMemcpyAsync(c->h_hist, c->hist + p0, (size_t)b * 4, hipMemcpyDeviceToHost, c->stream),
            "id read-back");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    uint32_t used = b;
    for (uint32_t i = 0; i < b && !stopped; ++i) {
      out_ids[done + i] = c->h_hist[i];
      for (uint32_t k = 0; k < n_stop; ++k)
        if (c->h_hist[i] == stop_ids[k]) {
          stopped = true;
          used = i + 1;
        }
    }
    for (uint32_t i = 0; c->step_timing && i < used; ++i) {
      float ms = 0.f;
      HIP_TRY(hipEventElapsedTime(&ms, c->st_ev[i], c->st_ev[i + 1]), "hipEventElapsedTime");
      c->step_ms.push_back(ms);
    }
    done += used;
    if (used < b) {  // roll the position back to just after the stop id's step
      rolled = true;
      c->len = p0 + used;
      c->h_st->pos = c->len;
      HIP_TRY(hipMemcpyAsync((char*)c->st + offsetof(StepState, pos), &c->h_st->pos, 4, hipMemcpyHostToDevice,
                             c->stream),
              "position roll-back");
      HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    }
  }
  if (n_done) *n_done = done;
  if (done) {
    // the device's tok/next_tok hold the last step that ran; after a
    // roll-back that is not the last one kept, so the next call uploads
    c->last_next = rolled ? 0xFFFFFFFFu : out_ids[done - 1];
    c->have_logits = !rolled;
  }
  return FRN_OK;
}

extern "C" frn_status frn_logits(frn_ctx* c, float* host_out, size_t n) {
  if (!c || !host_out) return fail(FRN_EINVAL, "frn_logits: null argument");
  if (!c->have_logits) return fail(FRN_EINVAL, "frn_logits: no logits yet");
  if (n < c->cfg.vocab) return fail(FRN_EINVAL, "frn_logits: buffer holds %zu < vocab %u", n, c->cfg.vocab);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  HIP_TRY(hipMemcpyAsync(host_out, c->logits, (size_t)c->cfg.vocab * 4, hipMemcpyDeviceToHost, c->stream), "logits copy");
  HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return FRN_OK;
}

// ---- sampler (sampler.rs) -----------------------------------------------------
// Pcg32::new(seed) (sampler.rs:11-17) on the host: O'Neill's
// pcg32_srandom_r with initstate = seed, initseq = 0xda3e39cb94b95bdb.
static uint32_t pcg32_step(SamplerRng& r) {
  const uint64_t old = r.state;
  r.state = old * 6364136223846793005ull + r.inc;
  const uint32_t xs = (uint32_t)(((old >> 18) ^ old) >> 27), rot = (uint32_t)(old >> 59);
  return (xs >> rot) | (xs << ((32u - rot) & 31u));
}

extern "C" frn_status frn_sampler_init(frn_ctx* c, float temperature, uint32_t top_k, float top_p,
                                       float repeat_penalty, uint64_t seed) {
  if (!c) return fail(FRN_EINVAL, "frn_sampler_init: null context");
  if (!c->finalized) return fail(FRN_EINVAL, "frn_sampler_init: context not finalized");
  if (!(temperature >= 0.0f) || !std::isfinite(temperature))
    return fail(FRN_EINVAL, "frn_sampler_init: temperature %g must be finite and >= 0", (double)temperature);
  if (!std::isfinite(top_p)) return fail(FRN_EINVAL, "frn_sampler_init: top_p must be finite");
  if (!(repeat_penalty > 0.0f) || !std::isfinite(repeat_penalty))
    return fail(FRN_EINVAL, "frn_sampler_init: repeat_penalty %g must be finite and > 0", (double)repeat_penalty);
  const bool draw = !(temperature == 0.0f || top_k == 1);
  // top_k 0 (no cut) and top_k above SAMPLER_MAX_K sort the whole vocabulary
  const bool full = draw && (top_k == 0 || top_k > SAMPLER_MAX_K);
  if (!full && sampler_sort_size(c->cfg.vocab, draw ? top_k : 1) > SAMPLER_MAX_SORT)
    return fail(FRN_EINVAL, "frn_sampler_init: vocab %u x top_k %u candidates exceed the %u the sampler sorts",
                c->cfg.vocab, top_k, SAMPLER_MAX_SORT);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  if (full && !c->full.keys) {
    SamplerFull f;
    f.n2 = sampler_full_size(c->cfg.vocab);
    hipError_t e;
    if ((e = dmalloc(&f.keys, (size_t)f.n2 * 8)) || (e = dmalloc(&f.terms, (size_t)c->cfg.vocab * 4))) {
      if (f.keys) (void)hipFree(f.keys);
      return fail(e == hipErrorOutOfMemory ? FRN_EOOM : FRN_EHIP, "frn_sampler_init: whole-vocabulary buffers: %s",
                  hipGetErrorString(e));
    }
    c->full = f;
  }
  // the candidate path's sort for the k it will run (the whole-vocabulary path needs none)
  if (!full) HIP_TRY(sampler_prepare(c->cfg.vocab, draw ? std::min(top_k, SAMPLER_MAX_K) : 1u), "sampler LDS limit");
  SamplerRng r{0, (0xda3e39cb94b95bdbull << 1) | 1u, 0};
  pcg32_step(r);
  r.state += seed;
  pcg32_step(r);
  *c->h_rng = r;
  HIP_TRY(hipMemcpyAsync(c->rng, c->h_rng, sizeof r, hipMemcpyHostToDevice, c->stream), "sampler state upload");
  HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  c->s_temperature = temperature;
  c->s_top_k = top_k;
  c->s_full = full;
  c->s_top_p = top_p;
  c->s_penalty = repeat_penalty;
  c->sampler_ready = true;
  return FRN_OK;
}

// Sampler::sample (sampler.rs:86-108) on the device logits of the last
// frn_prefill / frn_decode step; the id also becomes the device's next
// token, so a following frn_decode(ctx, id) uploads nothing.
extern "C" frn_status frn_sample(frn_ctx* c, const uint32_t* recent, uint32_t n_recent, uint32_t* next_id) {
  if (!c) return fail(FRN_EINVAL, "frn_sample: null context");
  if (!c->sampler_ready) return fail(FRN_EINVAL, "frn_sample: call frn_sampler_init first");
  if (!c->have_logits) return fail(FRN_EINVAL, "frn_sample: no logits yet");
  if (n_recent > SAMPLER_MAX_RECENT)
    return fail(FRN_EINVAL, "frn_sample: %u recent ids exceed %u", n_recent, SAMPLER_MAX_RECENT);
  if (n_recent && !recent) return fail(FRN_EINVAL, "frn_sample: null recent ids");
  for (uint32_t i = 0; i < n_recent; ++i)
    if (recent[i] >= c->cfg.vocab) return fail(FRN_ETOKEN, "frn_sample: recent id %u out of range", recent[i]);
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  const bool draw = !(c->s_temperature == 0.0f || c->s_top_k == 1);
  if (n_recent) {
    memcpy(c->h_recent, recent, (size_t)n_recent * 4);
    HIP_TRY(hipMemcpyAsync(c->recent, c->h_recent, (size_t)n_recent * 4, hipMemcpyHostToDevice, c->stream),
            "recent ids upload");
  }
  if (draw && c->s_full)
    HIP_TRY(launch_sample_full(c->logits, c->cfg.vocab, c->recent, n_recent, c->s_penalty, c->s_temperature,
                               c->s_top_k, c->s_top_p, c->full, c->rng, c->st, c->stream),
            "sampler launch (whole vocabulary)");
  else
    HIP_TRY(launch_sample(c->logits, c->cfg.vocab, c->recent, n_recent, c->s_penalty,
                          draw ? c->s_temperature : 1.0f, draw ? std::min(c->s_top_k, SAMPLER_MAX_K) : 1u,
                          c->s_top_p, draw, c->cand_v, c->cand_id, c->rng, c->st, c->stream),
            "sampler launch");
  frn_status st = read_next(c, next_id);
  // the host buffer is reused by the next call: the copy above has run
  return st;
}

extern "C" frn_status frn_sampler_draws(frn_ctx* c, uint64_t* draws) {
  if (!c || !draws) return fail(FRN_EINVAL, "frn_sampler_draws: null argument");
  if (!c->sampler_ready) return fail(FRN_EINVAL, "frn_sampler_draws: call frn_sampler_init first");
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  HIP_TRY(hipMemcpyAsync(c->h_rng, c->rng, sizeof(SamplerRng), hipMemcpyDeviceToHost, c->stream), "draws read-back");
  HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  *draws = c->h_rng->draws;
  return FRN_OK;
}

extern "C" frn_status frn_reset(frn_ctx* c) {
  if (!c) return fail(FRN_EINVAL, "frn_reset: null context");
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  StepState init{};
  HIP_TRY(hipMemcpy(c->st, &init, sizeof init, hipMemcpyHostToDevice), "state reset");
  c->len = 0;
  c->last_next = 0xFFFFFFFFu;
  c->have_logits = false;
  return FRN_OK;
}

extern "C" frn_status frn_cache_len(frn_ctx* c, uint32_t* len) {
  if (!c || !len) return fail(FRN_EINVAL, "frn_cache_len: null argument");
  *len = c->len;
  return FRN_OK;
}

extern "C" frn_status frn_cache_read(frn_ctx* c, uint32_t layer, uint32_t which, uint32_t n, float* host_out) {
  if (!c || !host_out) return fail(FRN_EINVAL, "frn_cache_read: null argument");
  if (layer >= c->cfg.n_layers || n > c->cfg.max_ctx || which > 1) return fail(FRN_EINVAL, "frn_cache_read: out of range");
  size_t kvd = (size_t)c->cfg.n_kv_heads * c->cfg.head_dim;
  const float* src = (which ? c->vcache : c->kcache) + (size_t)layer * c->cfg.max_ctx * kvd;
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  HIP_TRY(hipMemcpy(host_out, src, (size_t)n * kvd * 4, hipMemcpyDeviceToHost), "cache copy");
  return FRN_OK;
}

// ---- --timings (perf.rs) -----------------------------------------------------
extern "C" frn_status frn_timings_enable(frn_ctx* c, int enable) {
  if (!c) return fail(FRN_EINVAL, "null context");
  c->timing = enable != 0;
  return FRN_OK;
}
extern "C" frn_status frn_timings_reset(frn_ctx* c) {
  if (!c) return fail(FRN_EINVAL, "null context");
  memset(c->t_ms, 0, sizeof c->t_ms);
  memset(c->t_calls, 0, sizeof c->t_calls);
  return FRN_OK;
}
extern "C" frn_status frn_step_times_enable(frn_ctx* c, int enable) {
  if (!c) return fail(FRN_EINVAL, "null context");
  if (enable && c->st_ev.empty()) {
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    for (uint32_t i = 0; i <= GREEDY_BATCH; ++i) {
      hipEvent_t e;
      HIP_TRY(hipEventCreate(&e), "hipEventCreate");
      c->st_ev.push_back(e);
    }
  }
  c->step_timing = enable != 0;
  c->step_ms.clear();
  return FRN_OK;
}
extern "C" frn_status frn_step_times(frn_ctx* c, float* ms_out, uint32_t max, uint32_t* n) {
  if (!c || !n || (max && !ms_out)) return fail(FRN_EINVAL, "frn_step_times: null argument");
  const uint32_t k = (uint32_t)std::min<size_t>(max, c->step_ms.size());
  std::copy(c->step_ms.begin(), c->step_ms.begin() + k, ms_out);
  c->step_ms.erase(c->step_ms.begin(), c->step_ms.begin() + k);
  *n = k;
  return FRN_OK;
}
extern "C" frn_status frn_timings(frn_ctx* c, frn_timing* out, uint32_t max, uint32_t* n) {
  if (!c || !n || (max && !out)) return fail(FRN_EINVAL, "null argument");
  uint32_t k = 0;
  for (int i = 0; i < N_CAT && k < max; ++i) {
    snprintf(out[k].name, sizeof out[k].name, "%s", CAT_NAMES[i]);
    out[k].ms = c->t_ms[i];
    out[k].calls = c->t_calls[i];
    ++k;
  }
  *n = k;
  return FRN_OK;
}

extern "C" frn_status frn_bench_kernel(frn_ctx* c, const char* name, uint32_t layer, uint32_t reps, float* avg_us) {
  if (!c || !name || !avg_us || reps == 0) return fail(FRN_EINVAL, "frn_bench_kernel: bad argument");
  int cat = -1;
  for (int i = 0; i < N_CAT; ++i)
    if (!strcmp(name, CAT_NAMES[i])) cat = i;
  if (cat < 0) return fail(FRN_EINVAL, "frn_bench_kernel: no kernel category '%s'", name);
  if (layer != FRN_ALL_LAYERS && layer >= c->cfg.n_layers)
    return fail(FRN_EINVAL, "frn_bench_kernel: layer %u out of range", layer);
  // the replayed kernels run a step at position len (and write its KV row)
  if (frn_status st = check_ready(c, 1)) return st;
  HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0), "hipEventCreate");
  if (hipError_t r = hipEventCreate(&e1)) {
    (void)hipEventDestroy(e0);
    return fail(FRN_EHIP, "hipEventCreate: %s", hipGetErrorString(r));
  }
  c->rec_long = c->len + 1 > ATTENTION_LONG_FROM;  // the form the next step runs
  Tick tk{c, false};
  tk.rcat = cat;
  tk.rlayer = layer == FRN_ALL_LAYERS ? -1 : (int)layer;
  tk.reps = layer == FRN_ALL_LAYERS ? 1 : reps;
  hipError_t r = hipEventRecord(e0, c->stream);
  for (uint32_t k = 0; !r && k < (layer == FRN_ALL_LAYERS ? reps : 1u); ++k) r = record_step(c, true, tk);
  if (!r) r = hipEventRecord(e1, c->stream);
  if (!r) r = hipEventSynchronize(e1);
  float ms = 0.f;
  if (!r) r = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (r) return fail(FRN_EHIP, "frn_bench_kernel: %s", hipGetErrorString(r));
  *avg_us = tk.launched ? ms * 1000.0f / (float)tk.launched : 0.f;
  return FRN_OK;
}

// ---- single-op entry points ------------------------------------------------------
namespace {
// Per-device state the single-op entry points prepare on first use on a
// device (the current device of the calling thread).
constexpr int OP_MAX_DEVICES = 64;
// argmax keys carry the index in 32 bits
constexpr size_t ARGMAX_MAX_N = 0xFFFFFFFFull;
struct OpDevice {
  size_t gemv_lds = 0;             // dynamic LDS the GEMV kernels are prepared for
  uint64_t* argmax_key = nullptr;  // frn_argmax's running key (allocated once)
  uint64_t* scratch = nullptr;     // this device's copy of `scratch` (frn_argmax_noalloc)
};
std::mutex g_op_mu;
OpDevice g_op_dev[OP_MAX_DEVICES];
}  // namespace

extern "C" frn_status frn_dequant(uint32_t type, const void* raw_dev, size_t raw_bytes, size_t n, float* out_dev,
                                  void* stream) {
  if (!known_type(type)) return fail(FRN_EDTYPE, "dequantization for type %u is not implemented", type);
  if (n % blk_elems(type)) return fail(FRN_ESHAPE, "element count %zu is not a multiple of %d", n, blk_elems(type));
  size_t want = n / blk_elems(type) * blk_bytes(type);
  if (raw_bytes != want)
    return fail(FRN_ESHAPE, "data is %zu bytes, expected %zu (%zu blocks of %d)", raw_bytes, want,
                n / blk_elems(type), blk_bytes(type));
  if (n && (!raw_dev || !out_dev)) return fail(FRN_EINVAL, "frn_dequant: null pointer");
  HIP_TRY(launch_dequant(type, (const uint8_t*)raw_dev, n, out_dev, (hipStream_t)stream), "dequant launch");
  return FRN_OK;
}

extern "C" frn_status frn_matmul_quant(uint32_t type, const void* w_dev, size_t w_bytes, const float* a_dev,
                                       uint32_t seq, float* out_dev, uint32_t d_out, uint32_t d_in, void* stream) {
  if (!known_type(type)) return fail(FRN_EDTYPE, "no fused matmul kernel for type %u", type);
  if (type != T_F32 && d_in % blk_elems(type))
    return fail(FRN_ESHAPE, "matmul: in dim %u not a multiple of %d", d_in, blk_elems(type));
  if (d_in % 32) return fail(FRN_ESHAPE, "matmul: in dim %u not a multiple of 32", d_in);
  size_t want = (size_t)d_out * type_row_bytes(type, d_in);
  if (w_bytes != want) return fail(FRN_ESHAPE, "matmul: bad weight byte count %zu, expected %zu", w_bytes, want);
  if (!w_dev || !a_dev || !out_dev) return fail(FRN_EINVAL, "frn_matmul_quant: null pointer");
  // the kernels use 16-byte loads of rows and of the activation vector
  if (((uintptr_t)w_dev | (uintptr_t)a_dev) & 15)
    return fail(FRN_EINVAL, "frn_matmul_quant: w_dev and a_dev must be 16-byte aligned");
  if (gemv_lds_bytes(d_in, false) > 160 * 1024)
    return fail(FRN_ESHAPE, "matmul: in dim %u exceeds the 160 KiB LDS staging limit", d_in);
  if (seq == 0 || d_out == 0) return FRN_OK;
  {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= OP_MAX_DEVICES) return fail(FRN_EINVAL, "frn_matmul_quant: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_op_mu);
    const size_t need = gemv_lds_bytes(d_in, false);
    if (need > g_op_dev[dev].gemv_lds) {
      HIP_TRY(gemv_prepare(need), "gemv_prepare");
      g_op_dev[dev].gemv_lds = need;
    }
  }
  for (uint32_t s = 0; s < seq; ++s) {
    GemvArgs a{};
    a.n_seg = 1;
    a.in = d_in;
    a.x = a_dev + (size_t)s * d_in;
    a.seg[0].w = (const uint8_t*)w_dev;
    a.seg[0].type = type;
    a.seg[0].rows = d_out;
    a.seg[0].row_bytes = (uint32_t)type_row_bytes(type, d_in);
    a.seg[0].out = out_dev + (size_t)s * d_out;
    HIP_TRY(launch_gemv(a, GEMV_STORE, (hipStream_t)stream), "gemv launch");
  }
  return FRN_OK;
}

extern "C" frn_status frn_argmax(const float* x_dev, size_t n, uint32_t* out_dev, void* stream) {
  if (!x_dev || !out_dev || n == 0) return fail(FRN_EINVAL, "frn_argmax: bad argument");
  if (n > ARGMAX_MAX_N) return fail(FRN_ESHAPE, "frn_argmax: %zu values exceed the 32-bit index limit", n);
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= OP_MAX_DEVICES) return fail(FRN_EINVAL, "frn_argmax: device %d out of range", dev);
  uint64_t* key = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_op_mu);
    if (!g_op_dev[dev].argmax_key) HIP_TRY(hipMalloc((void**)&g_op_dev[dev].argmax_key, 256), "argmax scratch");
    key = g_op_dev[dev].argmax_key;
  }
  HIP_TRY(launch_argmax(x_dev, n, key, out_dev, (hipStream_t)stream), "argmax launch");
  return FRN_OK;
}

// frn_argmax_noalloc's scratch: a file-scope device array, one copy per GPU,
// held until the process ends.  On the host its name is not a device
// address: host code uses only the per-device address that
// hipGetSymbolAddress returns (OpDevice::scratch).
constexpr size_t NOALLOC_SCRATCH_BYTES = 256;
static __device__ __align__(256) uint64_t scratch[NOALLOC_SCRATCH_BYTES / sizeof(uint64_t)];
// argmax keeps one 64-bit running key there, for any n up to ARGMAX_MAX_N
static_assert(sizeof(uint64_t) <= NOALLOC_SCRATCH_BYTES, "argmax key exceeds the scratch array");

extern "C" frn_status frn_argmax_noalloc(const float* x_dev, size_t n, uint32_t* out_dev, void* stream) {
  if (!x_dev || !out_dev || n == 0) return fail(FRN_EINVAL, "frn_argmax_noalloc: bad argument");
  if (n > ARGMAX_MAX_N)
    return fail(FRN_ESHAPE, "frn_argmax_noalloc: %zu values exceed the maximum of %zu (32-bit index)", n,
                ARGMAX_MAX_N);
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= OP_MAX_DEVICES) return fail(FRN_EINVAL, "frn_argmax_noalloc: device %d out of range", dev);
  uint64_t* key = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_op_mu);
    if (!g_op_dev[dev].scratch) {
      void* p = nullptr;
      HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
      if (!p) return fail(FRN_EHIP, "frn_argmax_noalloc: no device address for the scratch array");
      g_op_dev[dev].scratch = (uint64_t*)p;
    }
    key = g_op_dev[dev].scratch;
  }
  // the key is cleared by the first of the three launches (a kernel, no memset)
  HIP_TRY(launch_argmax(x_dev, n, key, out_dev, (hipStream_t)stream), "argmax launch");
  return FRN_OK;
}
