/* Test infrastructure only (the oracle).  Restates src/sampler.rs of furnace:
 * PCG32 (O'Neill), the llama.cpp-convention repeat penalty and
 * Sampler::{sample, filtered} -- repeat penalty -> temperature -> top-k ->
 * softmax -> top-p -> renormalize -> draw, in that fixed order.
 *
 * Ties: the reference selects and sorts with select_nth_unstable_by and
 * sort_unstable_by, which leave the order of equal scaled logits
 * unspecified.  Here equal values are ordered by ascending id, one of the
 * orders the reference may produce. */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Pcg32::next_u32 (sampler.rs:20-28): LCG step, XSH-RR output of the old state */
uint32_t orc_pcg32_next_u32(orc_pcg32* r) {
  const uint64_t old = r->state;
  r->state = old * 6364136223846793005ull + r->inc;
  const uint32_t xorshifted = (uint32_t)(((old >> 18) ^ old) >> 27);
  const uint32_t rot = (uint32_t)(old >> 59);
  return (xorshifted >> rot) | (xorshifted << ((32u - rot) & 31u));
}

/* O'Neill's pcg32_srandom_r; Pcg32::new(seed) (sampler.rs:11-17) is
 * (initstate = seed, initseq = 0xda3e39cb94b95bdb) */
void orc_pcg32_seed(orc_pcg32* r, uint64_t initstate, uint64_t initseq) {
  r->state = 0;
  r->inc = (initseq << 1) | 1u;
  orc_pcg32_next_u32(r);
  r->state += initstate;
  orc_pcg32_next_u32(r);
}

/* Pcg32::next_f32 (sampler.rs:31-33): 24 bits, uniform in [0, 1) */
float orc_pcg32_next_f32(orc_pcg32* r) {
  return (float)(orc_pcg32_next_u32(r) >> 8) / (float)(1u << 24);
}

/* apply_repeat_penalty (sampler.rs:39-55): once per unique recent token,
 * positive logits divided by the penalty, the others multiplied */
void orc_apply_repeat_penalty(float* logits, const uint32_t* recent, size_t n_recent, float penalty) {
  if (penalty == 1.0f) return;
  for (size_t i = 0; i < n_recent; ++i) {
    int seen = 0;
    for (size_t j = 0; j < i; ++j) seen |= recent[j] == recent[i];
    if (seen) continue;
    float* l = &logits[recent[i]];
    if (*l > 0.0f)
      *l /= penalty;
    else
      *l *= penalty;
  }
}

/* Sampler::new (sampler.rs:68-78) */
void orc_sampler_new(orc_sampler* s, float temperature, uint32_t top_k, float top_p, float repeat_penalty,
                     uint64_t seed) {
  s->temperature = temperature;
  s->top_k = top_k;
  s->top_p = top_p;
  s->repeat_penalty = repeat_penalty;
  s->repeat_window = 64;
  orc_pcg32_seed(&s->rng, seed, 0xda3e39cb94b95bdbull);
  s->draws = 0;
}

typedef struct {
  uint32_t id;
  float v;
} cand_t;

/* descending value, then ascending id */
static int cand_cmp(const void* a, const void* b) {
  const cand_t *x = (const cand_t*)a, *y = (const cand_t*)b;
  if (x->v > y->v) return -1;
  if (x->v < y->v) return 1;
  return x->id < y->id ? -1 : x->id > y->id;
}

/* Sampler::filtered (sampler.rs:117-155): writes (id, prob) sorted by
 * descending probability into ids/probs (n entries of room) and returns
 * the count */
size_t orc_sampler_filtered(const orc_sampler* s, const float* logits, size_t n, uint32_t* ids, float* probs) {
  cand_t* c = (cand_t*)malloc(n * sizeof(cand_t));
  if (!c || n == 0) {
    free(c);
    return 0;
  }
  for (size_t i = 0; i < n; ++i) {
    c[i].id = (uint32_t)i;
    c[i].v = logits[i] / s->temperature;
  }
  /* select_nth_unstable + truncate, then sort_unstable, both descending */
  qsort(c, n, sizeof(cand_t), cand_cmp);
  size_t len = (s->top_k > 0 && s->top_k < n) ? s->top_k : n;
  /* softmax over the surviving candidates only, max-subtracted */
  const float max = c[0].v;
  float sum = 0.0f;
  for (size_t i = 0; i < len; ++i) {
    c[i].v = expf(c[i].v - max);
    sum += c[i].v;
  }
  for (size_t i = 0; i < len; ++i) c[i].v /= sum;
  if (s->top_p < 1.0f) {
    float cum = 0.0f;
    size_t keep = len;
    for (size_t i = 0; i < len; ++i) {
      cum += c[i].v;
      if (cum >= s->top_p) {
        keep = i + 1; /* the crossing token is included */
        break;
      }
    }
    len = keep;
    float t = 0.0f;
    for (size_t i = 0; i < len; ++i) t += c[i].v;
    for (size_t i = 0; i < len; ++i) c[i].v /= t;
  }
  for (size_t i = 0; i < len; ++i) {
    ids[i] = c[i].id;
    probs[i] = c[i].v;
  }
  free(c);
  return len;
}

/* Sampler::sample (sampler.rs:86-108) */
uint32_t orc_sampler_sample(orc_sampler* s, const float* logits, size_t n, const uint32_t* recent,
                            size_t n_recent) {
  float* lg = (float*)malloc(n * sizeof(float));
  uint32_t* ids = (uint32_t*)malloc(n * sizeof(uint32_t));
  float* pr = (float*)malloc(n * sizeof(float));
  uint32_t out = 0;
  if (!lg || !ids || !pr) goto done;
  memcpy(lg, logits, n * sizeof(float));
  orc_apply_repeat_penalty(lg, recent, n_recent, s->repeat_penalty);
  if (s->temperature == 0.0f || s->top_k == 1) { /* argmax, no RNG draw */
    out = orc_argmax(lg, n);
    goto done;
  }
  size_t len = orc_sampler_filtered(s, lg, n, ids, pr);
  const float u = orc_pcg32_next_f32(&s->rng);
  s->draws += 1;
  float cum = 0.0f;
  out = len ? ids[len - 1] : 0;
  for (size_t i = 0; i < len; ++i) {
    cum += pr[i];
    if (u < cum) {
      out = ids[i];
      break;
    }
  }
done:
  free(lg);
  free(ids);
  free(pr);
  return out;
}
