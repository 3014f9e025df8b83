/* Test infrastructure only (the oracle).  Restates the f32 ops of furnace's
 * src/tensor.rs and the position/attention ops of src/model.rs. */
#include <math.h>
#include <string.h>
#include "oracle.h"

/* tensor.rs:146-160: 8 independent lanes over chunks of 8, lanes summed in
 * order (Sum for f32 folds from -0.0), then the remainder sequentially. */
float orc_dot(const float* a, const float* b, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t full = n / 8 * 8;
  for (size_t i = 0; i < full; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] += a[i + j] * b[i + j];
  float sum = -0.0f;
  for (int j = 0; j < 8; ++j) sum += acc[j];
  for (size_t i = full; i < n; ++i) sum += a[i] * b[i];
  return sum;
}

/* tensor.rs:74-80 matmul (f32 weights) over matmul_with */
void orc_matmul_f32(const float* a, size_t seq, const float* w, size_t d_out, size_t d_in, float* out) {
  long n_chunks = (long)((d_out + 63) / 64);
#pragma omp parallel for schedule(dynamic, 1)
  for (long c = 0; c < n_chunks; ++c) {
    size_t o_end = (size_t)(c + 1) * 64 < d_out ? (size_t)(c + 1) * 64 : d_out;
    for (size_t o = (size_t)c * 64; o < o_end; ++o)
      for (size_t s = 0; s < seq; ++s) out[s * d_out + o] = orc_dot(a + s * d_in, w + o * d_in, d_in);
  }
}

/* tensor.rs:164-185 */
void orc_rmsnorm(const float* x, size_t rows, size_t cols, const float* w, float eps, float* out) {
  for (size_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    float ss = -0.0f;
    for (size_t i = 0; i < cols; ++i) ss += row[i] * row[i];
    float mean_sq = ss / (float)cols;
    float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    float* o = out + r * cols;
    for (size_t i = 0; i < cols; ++i) o[i] = row[i] * inv_rms * w[i];
  }
}

/* tensor.rs:188-203: fold(-inf, f32::max), exp(v - max), sequential sum
 * from 0.0, divide. */
void orc_softmax(float* x, size_t rows, size_t cols) {
  /* rows are independent: threads split them, each row's order unchanged */
#pragma omp parallel for schedule(static) if (rows * cols > (1u << 16))
  for (size_t r = 0; r < rows; ++r) {
    float* row = x + r * cols;
    float mx = -INFINITY;
    for (size_t i = 0; i < cols; ++i) mx = fmaxf(mx, row[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < cols; ++i) {
      row[i] = expf(row[i] - mx);
      sum += row[i];
    }
    for (size_t i = 0; i < cols; ++i) row[i] /= sum;
  }
}

/* tensor.rs:207-210 */
void orc_silu(const float* x, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = x[i] / (1.0f + expf(-x[i]));
}

/* tensor.rs:213-227: g / (1 + exp(-g)) * u */
void orc_swiglu(const float* gate, const float* up, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = gate[i] / (1.0f + expf(-gate[i])) * up[i];
}

/* tensor.rs:229-234 */
void orc_add(const float* a, const float* b, size_t n, float* out) {
  for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* model.rs:193-217: NeoX half-split pairing; freq = theta^(-2i/hd) via powf,
 * angle = (start_pos + s) as f32 * freq, sin/cos from libm. */
void orc_rope(float* x, size_t seq, size_t n_heads, size_t head_dim, float theta, size_t start_pos) {
  size_t half = head_dim / 2;
  for (size_t s = 0; s < seq; ++s) {
    float* row = x + s * n_heads * head_dim;
    for (size_t h = 0; h < n_heads; ++h) {
      float* head = row + h * head_dim;
      for (size_t i = 0; i < half; ++i) {
        float freq = powf(theta, -2.0f * (float)i / (float)head_dim);
        float angle = (float)(start_pos + s) * freq;
        float sn = sinf(angle), cs = cosf(angle);
        float a = head[i], b = head[i + half];
        head[i] = a * cs - b * sn;
        head[i + half] = a * sn + b * cs;
      }
    }
  }
}

/* Sequential dot of model.rs:248/:396 (`iter().zip().map().sum()`). */
static float seq_dot(const float* a, const float* b, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
  return s;
}

/* model.rs:371-407 attention_scores_cached; with start_pos = 0 and
 * total = n_new it is model.rs:224-258 attention_scores. */
void orc_attention_scores_cached(const float* q, size_t n_new, const float* k_cache, size_t total,
                                 size_t start_pos, size_t nh, size_t nkv, size_t hd, float* probs) {
  size_t kv_dim = nkv * hd, group = nh / nkv;
  float scale = 1.0f / sqrtf((float)hd);
  /* (head, row) pairs are independent: threads split them, each dot's order unchanged */
#pragma omp parallel for collapse(2) schedule(static) if (nh * n_new * total > (1u << 16))
  for (size_t h = 0; h < nh; ++h) {
    for (size_t s = 0; s < n_new; ++s) {
      size_t kv = h / group;
      const float* qh = q + s * nh * hd + h * hd;
      float* row = probs + (h * n_new + s) * total;
      for (size_t t = 0; t < total; ++t)
        row[t] = t <= start_pos + s ? seq_dot(qh, k_cache + t * kv_dim + kv * hd, hd) * scale : -INFINITY;
    }
  }
  orc_softmax(probs, nh * n_new, total);
}

/* model.rs:410-438 attention_apply_cached (= :262-290 attention_apply). */
void orc_attention_apply_cached(const float* probs, size_t n_new, size_t total, const float* v_cache,
                                size_t nh, size_t nkv, size_t hd, float* out) {
  size_t kv_dim = nkv * hd, group = nh / nkv;
  memset(out, 0, n_new * nh * hd * sizeof(float));
  /* each (head, row) pair writes its own output row: threads split them */
#pragma omp parallel for collapse(2) schedule(static) if (nh * n_new * total > (1u << 16))
  for (size_t h = 0; h < nh; ++h) {
    for (size_t s = 0; s < n_new; ++s) {
      size_t kv = h / group;
      const float* row = probs + (h * n_new + s) * total;
      float* oh = out + s * nh * hd + h * hd;
      for (size_t t = 0; t < total; ++t) {
        float p = row[t];
        const float* vh = v_cache + t * kv_dim + kv * hd;
        for (size_t d = 0; d < hd; ++d) oh[d] += p * vh[d];
      }
    }
  }
}

void orc_attention_scores(const float* q, const float* k, size_t seq, size_t n_heads, size_t n_kv_heads,
                          size_t head_dim, float* probs) {
  orc_attention_scores_cached(q, seq, k, seq, 0, n_heads, n_kv_heads, head_dim, probs);
}

void orc_attention_apply(const float* probs, const float* v, size_t seq, size_t n_heads, size_t n_kv_heads,
                         size_t head_dim, float* out) {
  orc_attention_apply_cached(probs, seq, seq, v, n_heads, n_kv_heads, head_dim, out);
}

/* generate.rs:69-77: strict `>` keeps the first maximum. */
uint32_t orc_argmax(const float* x, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return (uint32_t)best;
}
