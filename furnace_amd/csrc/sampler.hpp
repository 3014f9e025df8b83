// Device sampler for temperature > 0 (src/sampler.rs): launch interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"

namespace frn {

constexpr uint32_t SAMPLER_MAX_K = 64;         // top-k the device sampler supports (1..64)
constexpr uint32_t SAMPLER_MAX_RECENT = 256;   // recent ids for the repeat penalty
constexpr uint32_t SAMPLER_MAX_SORT = 16384;   // candidates sorted in one block's LDS (128 KB)

// Pcg32 (sampler.rs:5-35) and the draw count (Sampler::draws), in device memory.
struct SamplerRng {
  uint64_t state, inc, draws;
};

uint32_t sampler_blocks(uint32_t vocab);
// power-of-two size of the candidate sort for top-k k
uint32_t sampler_sort_size(uint32_t vocab, uint32_t k);
hipError_t sampler_prepare(uint32_t vocab, uint32_t k_max);
// Samples from logits[vocab] into st->tok/next_tok: with draw,
// the full pipeline and one RNG draw; without, the argmax of the penalized
// logits (temperature ignored) and no draw.  cand_v/cand_id hold
// sampler_blocks(vocab) * k entries.
hipError_t launch_sample(const float* logits, uint32_t vocab, const uint32_t* recent, uint32_t n_recent,
                         float penalty, float temperature, uint32_t k, float top_p, bool draw, float* cand_v,
                         uint32_t* cand_id, SamplerRng* rng, StepState* st, hipStream_t s);

// The whole-vocabulary path, for top_k 0 ("no cut") and top_k above
// SAMPLER_MAX_K: every candidate sorted (sort keys of sampler_full_size
// entries), then the reference's sequential softmax sum, top-p cumulative
// sum and draw (terms of `vocab` entries).
struct SamplerFull {
  uint64_t* keys = nullptr;  // (descending value key << 32) | id
  float* terms = nullptr;    // softmax terms in sorted order
  uint32_t n2 = 0;           // keys' capacity
};
// the sort's size for a vocabulary: a power of two, at least one LDS run
uint32_t sampler_full_size(uint32_t vocab);
hipError_t launch_sample_full(const float* logits, uint32_t vocab, const uint32_t* recent, uint32_t n_recent,
                              float penalty, float temperature, uint32_t k, float top_p, const SamplerFull& f,
                              SamplerRng* rng, StepState* st, hipStream_t s);

}  // namespace frn
