/* Test infrastructure only (the oracle).  Restates src/quant.rs of furnace.
 * Built with -ffp-contract=off: every product and sum rounds separately, as
 * Rust's f32 arithmetic does. */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include "oracle.h"
#include "oracle_internal.h"

static __thread char g_err[512];
const char* orc_last_error(void) { return g_err; }
void orc_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

/* half 2.7.1 f16::to_f32 (Cargo.lock:198-199; used at quant.rs:36,54,94-95,
 * 115,243): exact IEEE binary16 -> binary32 widening, subnormals included. */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t ex = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
  if (ex == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = 0;
      while (!(man & 0x400u)) { man <<= 1; ++e; }
      bits = sign | ((uint32_t)(127 - 15 + 1 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (ex == 31) {
    bits = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0u);
  } else {
    bits = sign | ((ex + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline float f16le(const uint8_t* p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* gguf.rs:206-216 GgmlType::block_layout */
int orc_block_layout(uint32_t type, size_t* elems, size_t* bytes) {
  switch (type) {
    case ORC_F32: *elems = 1; *bytes = 4; return 0;
    case ORC_F16: *elems = 1; *bytes = 2; return 0;
    case ORC_Q8_0: *elems = 32; *bytes = 34; return 0;
    case ORC_Q5_0: *elems = 32; *bytes = 22; return 0;
    case ORC_Q4_K: *elems = 256; *bytes = 144; return 0;
    case ORC_Q6_K: *elems = 256; *bytes = 210; return 0;
    default: return -1;
  }
}

/* quant.rs:53-63 dequant_block_q5_0 */
void orc_dequant_block_q5_0(const uint8_t* b, float* out) {
  float d = f16le(b);
  uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
  const uint8_t* qs = b + 6;
  for (int j = 0; j < 16; ++j) {
    uint32_t hi0 = ((qh >> j) & 1u) << 4;
    uint32_t hi1 = ((qh >> (j + 16)) & 1u) << 4;
    out[j] = d * (float)((int32_t)((qs[j] & 0x0Fu) | hi0) - 16);
    out[j + 16] = d * (float)((int32_t)((uint32_t)(qs[j] >> 4) | hi1) - 16);
  }
}

/* quant.rs:78-88 q4k_scale_min */
static void q4k_scale_min(int j, const uint8_t* s, float* sc, float* m) {
  uint8_t a, b;
  if (j < 4) {
    a = s[j] & 63;
    b = s[j + 4] & 63;
  } else {
    a = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
    b = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
  *sc = (float)a;
  *m = (float)b;
}

/* quant.rs:93-109 dequant_block_q4_k */
void orc_dequant_block_q4_k(const uint8_t* b, float* out) {
  float d = f16le(b), dmin = f16le(b + 2);
  const uint8_t* scales = b + 4;
  const uint8_t* qs = b + 16;
  for (int j64 = 0; j64 < 4; ++j64) {
    const uint8_t* q = qs + 32 * j64;
    float sc1, m1, sc2, m2;
    q4k_scale_min(2 * j64, scales, &sc1, &m1);
    q4k_scale_min(2 * j64 + 1, scales, &sc2, &m2);
    float d1 = d * sc1, min1 = dmin * m1;
    float d2 = d * sc2, min2 = dmin * m2;
    for (int l = 0; l < 32; ++l) {
      out[64 * j64 + l] = d1 * (float)(q[l] & 0x0F) - min1;
      out[64 * j64 + 32 + l] = d2 * (float)(q[l] >> 4) - min2;
    }
  }
}

/* quant.rs:114-133 dequant_block_q6_k */
void orc_dequant_block_q6_k(const uint8_t* b, float* out) {
  float d = f16le(b + 208);
  for (int half = 0; half < 2; ++half) {
    const uint8_t* ql = b + 64 * half;
    const uint8_t* qh = b + 128 + 32 * half;
    const uint8_t* sc = b + 192 + 8 * half;
    float* y = out + 128 * half;
    for (int l = 0; l < 32; ++l) {
      int is = l / 16;
      int32_t q1 = ((int32_t)(ql[l] & 0x0F) | (((int32_t)qh[l] & 3) << 4)) - 32;
      int32_t q2 = ((int32_t)(ql[l + 32] & 0x0F) | ((((int32_t)qh[l] >> 2) & 3) << 4)) - 32;
      int32_t q3 = ((int32_t)(ql[l] >> 4) | ((((int32_t)qh[l] >> 4) & 3) << 4)) - 32;
      int32_t q4 = ((int32_t)(ql[l + 32] >> 4) | ((((int32_t)qh[l] >> 6) & 3) << 4)) - 32;
      y[l] = d * (float)(int8_t)sc[is] * (float)q1;
      y[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
      y[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
      y[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
    }
  }
}

/* quant.rs:17-42 dequantize_q8_0 (per-block body) */
static void dequant_block_q8_0(const uint8_t* b, float* out) {
  float d = f16le(b);
  for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)b[2 + i];
}

typedef void (*block_fn)(const uint8_t*, float*);
static block_fn block_dequant(uint32_t type) { /* quant.rs:137-144 (+ Q8_0) */
  switch (type) {
    case ORC_Q5_0: return orc_dequant_block_q5_0;
    case ORC_Q4_K: return orc_dequant_block_q4_k;
    case ORC_Q6_K: return orc_dequant_block_q6_k;
    case ORC_Q8_0: return dequant_block_q8_0;
    default: return NULL;
  }
}

/* F16 is not a format the reference loads: its dequantize has no F16 arm
 * (quant.rs:279).  With the extension switched on (the tests of the
 * engine's F16 support), F16 data widens exactly to f32 through
 * orc_f16_to_f32; off, it is the reference's error. */
static int f16_extension = 0;
void orc_set_f16_extension(int on) { f16_extension = on != 0; }

/* quant.rs:261-281 dequantize (with the length checks of :17-32, :147-161) */
int orc_dequantize(uint32_t type, const uint8_t* raw, size_t raw_len, size_t n, float* out) {
  if (type == ORC_F16 && f16_extension) {
    if (raw_len != n * 2) {
      orc_set_error("F16 data is %zu bytes, expected %zu", raw_len, n * 2);
      return -1;
    }
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32((uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8)));
    return 0;
  }
  if (type == ORC_F32) {
    if (raw_len != n * 4) {
      orc_set_error("F32 data is %zu bytes, expected %zu", raw_len, n * 4);
      return -1;
    }
    memcpy(out, raw, n * 4);
    return 0;
  }
  block_fn f = block_dequant(type);
  if (!f) {
    orc_set_error("dequantization for type %u is not implemented", type);
    return -1;
  }
  size_t be, bb;
  orc_block_layout(type, &be, &bb);
  if (n % be != 0) {
    orc_set_error("element count %zu is not a multiple of %zu", n, be);
    return -1;
  }
  size_t nb = n / be;
  if (raw_len != nb * bb) {
    orc_set_error("data is %zu bytes, expected %zu (%zu blocks of %zu)", raw_len, nb * bb, nb, bb);
    return -1;
  }
  for (size_t i = 0; i < nb; ++i) f(raw + i * bb, out + i * be);
  return 0;
}

/* quant.rs:234-258 matmul_q8_0, one output element */
static float row_dot_q8_0(const uint8_t* row, size_t n_blocks, const float* a_row) {
  float acc = 0.0f;
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t* blk = row + b * 34;
    float scale = f16le(blk);
    const uint8_t* qs = blk + 2;
    const float* ab = a_row + b * 32;
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < 4; ++j)
      for (int l = 0; l < 8; ++l) lanes[l] += ab[j * 8 + l] * (float)(int8_t)qs[j * 8 + l];
    float s = -0.0f; /* Sum for f32 folds from -0.0 */
    for (int l = 0; l < 8; ++l) s += lanes[l];
    acc += scale * s;
  }
  return acc;
}

/* quant.rs:198-227 matmul_blocks, one output element */
static float row_dot_blocks(const uint8_t* row, size_t n_blocks, size_t be, size_t bb, block_fn f,
                            const float* a_row) {
  float buf[256];
  float acc = 0.0f;
  for (size_t b = 0; b < n_blocks; ++b) {
    f(row + b * bb, buf);
    acc += orc_dot(a_row + b * be, buf, be);
  }
  return acc;
}

/* quant.rs:170-193 matmul_quant over tensor.rs:86-137 matmul_with.  Decode
 * (seq == 1) parallelises 64-row chunks; prefill keeps the weight-row outer
 * loop that re-dequantises each row per activation row, as the reference
 * does.  Each output element is computed by exactly one thread, so the
 * result does not depend on the thread count. */
int orc_matmul_quant(const float* a, size_t seq, const uint8_t* raw, size_t raw_len, size_t d_out,
                     size_t d_in, uint32_t type, float* out) {
  size_t be, bb;
  if (type != ORC_Q8_0 && type != ORC_Q5_0 && type != ORC_Q4_K && type != ORC_Q6_K) {
    orc_set_error("no fused matmul kernel for type %u", type);
    return -1;
  }
  orc_block_layout(type, &be, &bb);
  if (d_in % be != 0) {
    orc_set_error("matmul: in dim %zu not a multiple of %zu", d_in, be);
    return -1;
  }
  size_t nbk = d_in / be, row_bytes = nbk * bb;
  if (raw_len != d_out * row_bytes) {
    orc_set_error("matmul: bad weight byte count %zu, expected %zu", raw_len, d_out * row_bytes);
    return -1;
  }
  block_fn f = block_dequant(type);
  long n_chunks = (long)((d_out + 63) / 64);
#pragma omp parallel for schedule(dynamic, 1)
  for (long c = 0; c < n_chunks; ++c) {
    size_t o_end = (size_t)(c + 1) * 64 < d_out ? (size_t)(c + 1) * 64 : d_out;
    for (size_t o = (size_t)c * 64; o < o_end; ++o) {
      const uint8_t* row = raw + o * row_bytes;
      for (size_t s = 0; s < seq; ++s) {
        const float* a_row = a + s * d_in;
        out[s * d_out + o] = type == ORC_Q8_0 ? row_dot_q8_0(row, nbk, a_row)
                                              : row_dot_blocks(row, nbk, be, bb, f, a_row);
      }
    }
  }
  return 0;
}
