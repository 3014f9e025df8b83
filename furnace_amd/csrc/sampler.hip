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

}  // namespace

uint32_t sampler_blocks(uint32_t vocab) { return (vocab + CAND_BLOCK - 1) / CAND_BLOCK; }

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
