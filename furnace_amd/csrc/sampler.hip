// gfx950 sampler for temperature > 0: Sampler::sample (src/sampler.rs:86-155)
// on the device logits -- repeat penalty -> temperature -> top-k -> softmax
// -> top-p -> renormalize -> PCG32 draw, in the reference's order.
//
//  k_sample_cand: block b takes logits [1024 b, 1024 b + 1024): penalty for
//    ids in the recent set (set membership, so once per unique id), divide by
//    the temperature (IEEE division), bitonic sort in LDS by (value desc,
//    id asc), write the block's first k candidates.
//  k_sample_pick: one block sorts all blocks' candidates the same way; the
//    global top k are then the first k.  One thread then runs the
//    sequential part exactly as the reference orders it (softmax sum,
//    top-p cumulative sum, renormalization, cumulative draw), with the
//    PCG32 state in device memory.
//
// top_k 0 ("no cut") and top_k above 64 take the whole-vocabulary path:
//  k_sample_full_keys: the penalty and temperature per logit, as unique
//    sort keys (value descending, then id ascending);
//  a bitonic sort of the keys (k_bitonic_run in LDS, k_bitonic_step over
//    global memory);
//  k_sample_full_pick: the softmax terms in parallel, then one thread runs
//    the same sequential sums over the sorted vocabulary while the block
//    stages each next stretch of terms (or probabilities) through LDS.
//
// Ties among equal scaled logits are taken in ascending id order; the
// reference's select_nth_unstable_by / sort_unstable_by leave their order
// unspecified.  exp is evaluated in f64 and rounded to f32, which agrees with
// the glibc expf the CPU path calls to within its last-ulp behaviour.
#include "kernels.hpp"
#include "sampler.hpp"

#include <math.h>

namespace frn {

namespace {

constexpr int CAND_BLOCK = 1024;  // logits per candidate block

__device__ __forceinline__ bool before(float va, uint32_t ia, float vb, uint32_t ib) {
  return va > vb || (va == vb && ia < ib);
}

// Bitonic sort of n (a power of two) (value, id) pairs in LDS into
// (value desc, id asc) order, by all threads of the block.
__device__ void bitonic_sort(float* v, uint32_t* id, uint32_t n) {
  for (uint32_t k = 2; k <= n; k <<= 1)
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t l = i ^ j;
        if (l > i) {
          const float vi = v[i], vl = v[l];
          const uint32_t ii = id[i], il = id[l];
          const bool swap = (i & k) == 0 ? before(vl, il, vi, ii) : before(vi, ii, vl, il);
          if (swap) {
            v[i] = vl;
            v[l] = vi;
            id[i] = il;
            id[l] = ii;
          }
        }
      }
      __syncthreads();
    }
}

__global__ __launch_bounds__(256) void k_sample_cand(const float* __restrict__ logits, uint32_t vocab,
                                                     const uint32_t* __restrict__ recent, uint32_t n_recent,
                                                     float penalty, float temperature, uint32_t k,
                                                     float* __restrict__ cand_v, uint32_t* __restrict__ cand_id) {
  __shared__ float v[CAND_BLOCK];
  __shared__ uint32_t id[CAND_BLOCK];
  __shared__ uint32_t rec[SAMPLER_MAX_RECENT];
  for (uint32_t i = threadIdx.x; i < n_recent; i += blockDim.x) rec[i] = recent[i];
  __syncthreads();
  const uint32_t base = blockIdx.x * CAND_BLOCK;
  for (uint32_t i = threadIdx.x; i < CAND_BLOCK; i += blockDim.x) {
    const uint32_t t = base + i;
    float x = -INFINITY;
    if (t < vocab) {
      x = logits[t];
      if (penalty != 1.0f) {  // apply_repeat_penalty (sampler.rs:39-55)
        bool hit = false;
        for (uint32_t r = 0; r < n_recent; ++r) hit |= rec[r] == t;
        if (hit) x = x > 0.0f ? x / penalty : x * penalty;
      }
      if (temperature != 1.0f) x = x / temperature;  // filtered(), sampler.rs:121-125
    }
    v[i] = x;
    id[i] = t < vocab ? t : 0xFFFFFFFFu;
  }
  __syncthreads();
  bitonic_sort(v, id, CAND_BLOCK);
  for (uint32_t i = threadIdx.x; i < k; i += blockDim.x) {
    cand_v[(size_t)blockIdx.x * k + i] = v[i];
    cand_id[(size_t)blockIdx.x * k + i] = id[i];
  }
}

__device__ __forceinline__ uint32_t pcg32_next(SamplerRng* r) {  // Pcg32::next_u32 (sampler.rs:20-28)
  const uint64_t old = r->state;
  r->state = old * 6364136223846793005ull + r->inc;
  const uint32_t xorshifted = (uint32_t)(((old >> 18) ^ old) >> 27);
  const uint32_t rot = (uint32_t)(old >> 59);
  return (xorshifted >> rot) | (xorshifted << ((32u - rot) & 31u));
}

// dynamic LDS: n2 floats then n2 ids
__global__ __launch_bounds__(1024) void k_sample_pick(const float* __restrict__ cand_v,
                                                      const uint32_t* __restrict__ cand_id, uint32_t n_cand,
                                                      uint32_t n2, uint32_t k, float top_p, uint32_t draw,
                                                      SamplerRng* rng, StepState* st) {
  extern __shared__ float smem[];
  float* v = smem;
  uint32_t* id = (uint32_t*)(smem + n2);
  for (uint32_t i = threadIdx.x; i < n2; i += blockDim.x) {
    v[i] = i < n_cand ? cand_v[i] : -INFINITY;
    id[i] = i < n_cand ? cand_id[i] : 0xFFFFFFFFu;
  }
  __syncthreads();
  bitonic_sort(v, id, n2);
  if (threadIdx.x != 0) return;
  uint32_t pick = id[0];
  if (draw) {
    uint32_t len = k;
    while (len > 1 && id[len - 1] == 0xFFFFFFFFu) --len;  // fewer real candidates than k
    // softmax over the survivors, max-subtracted (sampler.rs:131-141)
    const float mx = v[0];
    float sum = 0.0f;
    for (uint32_t i = 0; i < len; ++i) {
      v[i] = (float)exp((double)(v[i] - mx));
      sum += v[i];
    }
    for (uint32_t i = 0; i < len; ++i) v[i] /= sum;
    if (top_p < 1.0f) {  // sampler.rs:143-153: keep through the crossing token
      float cum = 0.0f;
      uint32_t keep = len;
      for (uint32_t i = 0; i < len; ++i) {
        cum += v[i];
        if (cum >= top_p) {
          keep = i + 1;
          break;
        }
      }
      len = keep;
      float s = 0.0f;
      for (uint32_t i = 0; i < len; ++i) s += v[i];
      for (uint32_t i = 0; i < len; ++i) v[i] /= s;
    }
    // the draw (sampler.rs:97-107): u in [0, 1) from the top 24 bits
    SamplerRng r = *rng;
    const float u = (float)(pcg32_next(&r) >> 8) / (float)(1u << 24);
    r.draws += 1;
    *rng = r;
    float cum = 0.0f;
    pick = id[len - 1];
    for (uint32_t i = 0; i < len; ++i) {
      cum += v[i];
      if (u < cum) {
        pick = id[i];
        break;
      }
    }
  }
  st->next_tok = pick;
  st->tok = pick;
}

// ---- whole-vocabulary path (top_k 0 or above SAMPLER_MAX_K) -----------------------
// Every candidate gets a unique 64-bit key, (descending value key << 32) |
// id, so that ascending keys are the reference's sorted order (larger
// scaled logit first; equal values by ascending id).  A bitonic sort puts
// them in order: blocks sort runs of FULL_RUN keys in LDS, then every
// merge step whose partner distance is at least FULL_RUN runs as a pass
// over global memory and the shorter ones of each merge in LDS again.
// The reference's sums are then taken in that order, one by one in f32,
// as it takes them: they are not associative, and over ~10^5 small terms
// their rounding moves the cumulative probabilities well beyond an ulp, so
// any other summation order would pick other ids.
constexpr uint32_t FULL_RUN = 4096;  // keys per block-local run (32 KB of LDS)

__device__ __forceinline__ uint32_t order_key(float v) {  // larger v -> larger key
  if (v == 0.0f) v = 0.0f;                                 // -0 sorts with +0: the reference compares them equal
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint64_t key) {  // the scaled logit of a sorted key
  const uint32_t k = ~(uint32_t)(key >> 32);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// the penalty and temperature of every logit (as k_sample_cand), as sort
// keys; [vocab, n2) padded with keys that sort last
__global__ __launch_bounds__(256) void k_sample_full_keys(const float* __restrict__ logits, uint32_t vocab,
                                                          uint32_t n2, const uint32_t* __restrict__ recent,
                                                          uint32_t n_recent, float penalty, float temperature,
                                                          uint64_t* __restrict__ keys) {
  __shared__ uint32_t rec[SAMPLER_MAX_RECENT];
  for (uint32_t i = threadIdx.x; i < n_recent; i += blockDim.x) rec[i] = recent[i];
  __syncthreads();
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n2) return;
  if (t >= vocab) {
    keys[t] = ~0ull;
    return;
  }
  float x = logits[t];
  if (penalty != 1.0f) {  // apply_repeat_penalty (sampler.rs:39-55)
    bool hit = false;
    for (uint32_t r = 0; r < n_recent; ++r) hit |= rec[r] == t;
    if (hit) x = x > 0.0f ? x / penalty : x * penalty;
  }
  x = x / temperature;  // filtered(), sampler.rs:121-125
  keys[t] = ((uint64_t)~order_key(x) << 32) | t;
}

// bitonic steps on n2 keys, ascending where (index & k) == 0
__device__ __forceinline__ void bitonic_cas(uint64_t& a, uint64_t& b, bool up) {
  if ((a > b) == up) {
    const uint64_t t = a;
    a = b;
    b = t;
  }
}
// a run of FULL_RUN keys in LDS: the merges k = k0 .. k1 (powers of two), each
// with its partner distances below min(k, FULL_RUN)
__global__ __launch_bounds__(1024) void k_bitonic_run(uint64_t* __restrict__ keys, uint32_t k0, uint32_t k1) {
  __shared__ uint64_t s[FULL_RUN];
  const uint32_t base = blockIdx.x * FULL_RUN;
  for (uint32_t i = threadIdx.x; i < FULL_RUN; i += blockDim.x) s[i] = keys[base + i];
  __syncthreads();
  for (uint32_t k = k0; k <= k1; k <<= 1)
    for (uint32_t j = min(k, FULL_RUN) >> 1; j > 0; j >>= 1) {
      for (uint32_t i = threadIdx.x; i < FULL_RUN / 2; i += blockDim.x) {
        const uint32_t lo = 2 * i - (i & (j - 1)), hi = lo + j;  // the pair (lo, lo ^ j), lo's bit j clear
        bitonic_cas(s[lo], s[hi], ((base + lo) & k) == 0);
      }
      __syncthreads();
    }
  for (uint32_t i = threadIdx.x; i < FULL_RUN; i += blockDim.x) keys[base + i] = s[i];
}
// one merge step with partner distance j >= FULL_RUN, over global memory
__global__ __launch_bounds__(256) void k_bitonic_step(uint64_t* __restrict__ keys, uint32_t n2, uint32_t k,
                                                      uint32_t j) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n2 / 2) return;
  const uint32_t lo = 2 * i - (i & (j - 1)), hi = lo + j;
  uint64_t a = keys[lo], b = keys[hi];
  const bool up = (lo & k) == 0;
  if ((a > b) == up) {
    keys[lo] = b;
    keys[hi] = a;
  }
}

// Sequential passes over the sorted candidates (Sampler::filtered and the
// draw, sampler.rs:97-154) in the reference's order.  The block stages
// FULL_CHUNK values at a time through LDS, computing each pass's
// per-element values (terms, terms / sum, their renormalization) in
// parallel with the same single divisions; thread 0 then folds them in
// order, 16 at a time (four float4 LDS reads, the next group's issued
// before this group is added, then 16 dependent f32 adds).  The terms only
// shrink along the order, so a pass also ends once a group's last term is
// below half an ulp of the running sum: every later addition would leave
// it unchanged.
constexpr uint32_t FULL_CHUNK = 8192;
constexpr int FOLD = 16;
__device__ __forceinline__ float half_ulp(float a) {  // a > 0, normal, exponent above -102
  return __uint_as_float((__float_as_uint(a) & 0x7F800000u) - (24u << 23));
}
__global__ __launch_bounds__(1024) void k_sample_full_pick(const uint64_t* __restrict__ keys,
                                                           float* __restrict__ e, uint32_t vocab, uint32_t k,
                                                           float top_p, SamplerRng* rng, StepState* st) {
  __shared__ __align__(16) float buf[FULL_CHUNK];
  __shared__ float sh_val;
  __shared__ uint32_t sh_idx, sh_done;
  const uint32_t len0 = (k > 0 && k < vocab) ? k : vocab;  // top-k cut, else every candidate
  // softmax terms e^(v_i - max), max = v_0 (sampler.rs:131-137)
  const float mx = key_value(keys[0]);
  for (uint32_t i = threadIdx.x; i < len0; i += blockDim.x) e[i] = (float)exp((double)(key_value(keys[i]) - mx));
  __syncthreads();
  // pass: stage f(i) for i < len in chunks; thread 0 runs acc += x over
  // them in order.  With `stop`, the pass ends at the first i where
  // crossed(acc) holds and returns that i; else (or once the rest cannot
  // change acc) it returns len.
  auto pass = [&](uint32_t len, float& acc, bool stop, auto&& f, auto&& crossed) -> uint32_t {
    if (threadIdx.x == 0) {
      sh_done = 0;
      sh_idx = len;
    }
    __syncthreads();
    for (uint32_t c0 = 0; c0 < len; c0 += FULL_CHUNK) {
      const uint32_t n = min(FULL_CHUNK, len - c0);
      for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) buf[i] = f(c0 + i);
      __syncthreads();
      if (threadIdx.x == 0) {
        const float4* b4 = (const float4*)buf;
        const uint32_t ng = n / FOLD;
        float4 q[FOLD / 4];
#pragma unroll
        for (int w = 0; w < FOLD / 4; ++w) q[w] = b4[w];  // group 0 (inside buf even when ng == 0)
        for (uint32_t g = 0; g < ng; ++g) {
          float x[FOLD];
#pragma unroll
          for (int w = 0; w < FOLD / 4; ++w) {
            x[4 * w] = q[w].x;
            x[4 * w + 1] = q[w].y;
            x[4 * w + 2] = q[w].z;
            x[4 * w + 3] = q[w].w;
          }
          if (g + 1 < ng)
#pragma unroll
            for (int w = 0; w < FOLD / 4; ++w) q[w] = b4[(g + 1) * (FOLD / 4) + w];
          const float a0 = acc;
#pragma unroll
          for (int j = 0; j < FOLD; ++j) acc += x[j];
          if (stop && crossed(acc)) {  // the sums only grow: the crossing lies in this group
            float a = a0;
            int j = 0;
            for (; j < FOLD; ++j) {
              a += x[j];
              if (crossed(a)) break;
            }
            acc = a;
            sh_idx = c0 + g * FOLD + j;
            sh_done = 1;
            break;
          }
          if (x[FOLD - 1] < half_ulp(acc)) {  // the rest is absorbed: acc is final
            sh_done = 1;
            break;
          }
        }
        if (!sh_done)
          for (uint32_t i = ng * FOLD; i < n; ++i) {  // the chunk's tail
            acc += buf[i];
            if (stop && crossed(acc)) {
              sh_idx = c0 + i;
              sh_done = 1;
              break;
            }
          }
      }
      __syncthreads();
      if (sh_done) break;
    }
    return sh_idx;
  };
  auto never = [](float) { return false; };
  float sum = 0.0f;  // thread 0's running values
  pass(len0, sum, false, [&](uint32_t i) { return e[i]; }, never);
  if (threadIdx.x == 0) sh_val = sum;
  __syncthreads();
  sum = sh_val;
  uint32_t len = len0;
  float t = 1.0f;
  if (top_p < 1.0f) {
    // keep through the crossing token, then renormalize (sampler.rs:143-153);
    // the renormalizing sum adds the same terms in the same order as the
    // cumulative sum up to the crossing, so it is that cumulative sum
    float cum = 0.0f;
    const uint32_t at = pass(len0, cum, true, [&](uint32_t i) { return e[i] / sum; },
                             [&](float c) { return c >= top_p; });
    len = at < len0 ? at + 1 : len0;
    if (threadIdx.x == 0) sh_val = cum;
    __syncthreads();
    t = sh_val;
  }
  // the draw (sampler.rs:97-107): u in [0, 1) from the top 24 bits
  float u = 0.0f;
  if (threadIdx.x == 0) {
    SamplerRng r = *rng;
    u = (float)(pcg32_next(&r) >> 8) / (float)(1u << 24);
    r.draws += 1;
    *rng = r;
  }
  float cum = 0.0f;
  const bool renorm = top_p < 1.0f;
  const uint32_t at = pass(len, cum, true, [&](uint32_t i) { const float p = e[i] / sum; return renorm ? p / t : p; },
                           [&](float c) { return u < c; });
  if (threadIdx.x == 0) {
    const uint32_t pick = (uint32_t)keys[at < len ? at : len - 1];  // candidates.last() when the sum never passes u
    st->next_tok = pick;
    st->tok = pick;
  }
}

}  // namespace

uint32_t sampler_blocks(uint32_t vocab) { return (vocab + CAND_BLOCK - 1) / CAND_BLOCK; }

uint32_t sampler_full_size(uint32_t vocab) {
  uint32_t n2 = FULL_RUN;
  while (n2 < vocab) n2 <<= 1;
  return n2;
}

hipError_t launch_sample_full(const float* logits, uint32_t vocab, const uint32_t* recent, uint32_t n_recent,
                              float penalty, float temperature, uint32_t k, float top_p, const SamplerFull& f,
                              SamplerRng* rng, StepState* st, hipStream_t s) {
  const uint32_t n2 = sampler_full_size(vocab);
  if (n_recent > SAMPLER_MAX_RECENT || !f.keys || !f.terms || vocab == 0 || n2 > f.n2) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample_full_keys, dim3((n2 + 255) / 256), dim3(256), 0, s, logits, vocab, n2, recent, n_recent,
                     penalty, temperature, f.keys);
  // bitonic sort: runs of FULL_RUN in LDS, then each longer merge's global steps and its LDS tail
  hipLaunchKernelGGL(k_bitonic_run, dim3(n2 / FULL_RUN), dim3(1024), 0, s, f.keys, 2u, FULL_RUN);
  for (uint32_t kk = 2 * FULL_RUN; kk <= n2; kk <<= 1) {
    for (uint32_t j = kk / 2; j >= FULL_RUN; j >>= 1)
      hipLaunchKernelGGL(k_bitonic_step, dim3((n2 / 2 + 255) / 256), dim3(256), 0, s, f.keys, n2, kk, j);
    hipLaunchKernelGGL(k_bitonic_run, dim3(n2 / FULL_RUN), dim3(1024), 0, s, f.keys, kk, kk);
  }
  hipLaunchKernelGGL(k_sample_full_pick, dim3(1), dim3(1024), 0, s, f.keys, f.terms, vocab, k, top_p, rng, st);
  return hipGetLastError();
}

uint32_t sampler_sort_size(uint32_t vocab, uint32_t k) {
  uint32_t n = sampler_blocks(vocab) * k, n2 = 1;
  while (n2 < n) n2 <<= 1;
  return n2 < 2 ? 2 : n2;
}

hipError_t sampler_prepare(uint32_t vocab, uint32_t k_max) {
  const size_t bytes = (size_t)sampler_sort_size(vocab, k_max) * 8;
  return hipFuncSetAttribute((const void*)k_sample_pick, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

hipError_t launch_sample(const float* logits, uint32_t vocab, const uint32_t* recent, uint32_t n_recent,
                         float penalty, float temperature, uint32_t k, float top_p, bool draw, float* cand_v,
                         uint32_t* cand_id, SamplerRng* rng, StepState* st, hipStream_t s) {
  const uint32_t nb = sampler_blocks(vocab), n2 = sampler_sort_size(vocab, k);
  if (k < 1 || k > SAMPLER_MAX_K || n_recent > SAMPLER_MAX_RECENT || n2 > SAMPLER_MAX_SORT) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_sample_cand, dim3(nb), dim3(256), 0, s, logits, vocab, recent, n_recent, penalty, temperature,
                     k, cand_v, cand_id);
  hipError_t e = hipGetLastError();
  if (e) return e;
  hipLaunchKernelGGL(k_sample_pick, dim3(1), dim3(1024), (size_t)n2 * 8, s, cand_v, cand_id, nb * k, n2, k, top_p,
                     draw ? 1u : 0u, rng, st);
  return hipGetLastError();
}

}  // namespace frn
