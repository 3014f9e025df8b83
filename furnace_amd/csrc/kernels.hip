// gfx950 kernels of the token loop: dequant, fused dequant-GEMV, embedding,
// RoPE + KV-cache write, split-sequence GQA decode attention, argmax.
#include "formats.hpp"
#include "kernels.hpp"

namespace frn {

constexpr int ATT_CHUNK = 256;  // positions per attention block

// ---- reductions -----------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// Sum over a 256-thread block; every thread gets the result.
__device__ __forceinline__ float block_sum256(float v, float* red4) {
  v = wave_sum(v);
  int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red4[w] = v;
  __syncthreads();
  float r = red4[0] + red4[1] + red4[2] + red4[3];
  __syncthreads();
  return r;
}

// ---- dequant (quant.rs:261-281), bit-exact -------------------------------
__global__ void k_dequant(uint32_t type, const uint8_t* __restrict__ raw, size_t n, float* __restrict__ out) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  int be = blk_elems(type), bb = blk_bytes(type);
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += stride) {
    if (type == T_F32) {
      out[i] = ((const float*)raw)[i];
    } else {
      size_t b = i / (size_t)be;
      out[i] = decode_elem(type, raw + b * (size_t)bb, (int)(i - b * (size_t)be));
    }
  }
}

hipError_t launch_dequant(uint32_t type, const uint8_t* raw, size_t n, float* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)blocks), dim3(256), 0, s, type, raw, n, out);
  return hipGetLastError();
}

// ---- fused dequant-GEMV ---------------------------------------------------
__host__ __device__ inline int items_per_row(uint32_t t, uint32_t in, bool pairs) {
  if (t == T_Q4_K || t == T_Q6_K) return (int)(in / 256) * 8;
  if (t == T_Q8_0 || t == T_Q5_0) return (int)(pairs ? in / 64 : in / 32);
  return (int)(in / 16);  // F32: 16 floats per item
}

template <uint32_t T>
__device__ __forceinline__ float item_dot(const uint8_t* row, int it, const float* xs, const float* xsum, bool pairs) {
  if constexpr (T == T_Q4_K) {
    return q4k_item(row, it, xs, xsum);
  } else if constexpr (T == T_Q6_K) {
    return q6k_item(row, it, xs);
  } else if constexpr (T == T_Q8_0) {
    return pairs ? q8_0_pair_item(row, it, xs) : small_block_item(T_Q8_0, row, it, xs);
  } else if constexpr (T == T_Q5_0) {
    return pairs ? q5_0_pair_item(row, it, xs) : small_block_item(T_Q5_0, row, it, xs);
  } else {
    const float4* w = (const float4*)row + it * 4;
    const float4* X = (const float4*)xs + it * 4;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 a = w[i], b = X[i];
      s += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
    }
    return s;
  }
}

// Stage x (optionally rmsnorm'd, tensor.rs:164-185) into LDS; for Q4_K also
// the 16-value chunk sums used by q4k_item.
template <bool XSUM>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, uint32_t in, const float* __restrict__ norm_w,
                                        float eps, float* xs, float* xsum, float* red4) {
  float ss = 0.f;
  for (uint32_t i = threadIdx.x * 4; i < in; i += 1024) {
    float4 v = *(const float4*)(x + i);
    *(float4*)(xs + i) = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (norm_w) {
    ss = block_sum256(ss, red4);
    float inv = 1.0f / sqrtf(ss / (float)in + eps);
    for (uint32_t i = threadIdx.x * 4; i < in; i += 1024) {
      float4 v = *(float4*)(xs + i), w = *(const float4*)(norm_w + i);
      v.x = v.x * inv * w.x;
      v.y = v.y * inv * w.y;
      v.z = v.z * inv * w.z;
      v.w = v.w * inv * w.w;
      *(float4*)(xs + i) = v;
    }
  }
  __syncthreads();
  if (XSUM) {
    for (uint32_t c = threadIdx.x; c < in / 16; c += 256) {
      const float4* p = (const float4*)(xs + 16 * c);
      float4 a = p[0], b = p[1], cc = p[2], d = p[3];
      xsum[c] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) + ((cc.x + cc.y) + (cc.z + cc.w)) +
                ((d.x + d.y) + (d.z + d.w));
    }
    __syncthreads();
  }
}

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal in the reference
  uint32_t u = __float_as_uint(v);
  uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

// One group of LPR lanes per output row; 256 / LPR rows per block.
template <uint32_t T, int LPR, int MODE>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a, int pairs) {
  extern __shared__ float4 smem4[];
  __shared__ float red4[4];
  __shared__ uint64_t best_s[256 / LPR];
  float* xs = (float*)smem4;
  float* xsum = xs + a.in;
  stage_x<T == T_Q4_K>(a.x, a.in, a.norm_w, a.eps, xs, xsum, red4);
  constexpr int G = 256 / LPR;
  const int g = threadIdx.x / LPR, gl = threadIdx.x % LPR;
  const uint32_t row = blockIdx.x * G + g;
  const int n_items = items_per_row(T, a.in, pairs != 0);
  float acc = 0.f, acc2 = 0.f;
  if (row < a.rows) {
    const uint8_t* wr = a.w + (size_t)row * a.row_bytes;
    for (int it = gl; it < n_items; it += LPR) acc += item_dot<T>(wr, it, xs, xsum, pairs != 0);
    if (MODE == GEMV_SWIGLU) {
      const uint8_t* wr2 = a.w2 + (size_t)row * a.row_bytes;
      for (int it = gl; it < n_items; it += LPR) acc2 += item_dot<T>(wr2, it, xs, xsum, pairs != 0);
    }
  }
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) {
    acc += __shfl_xor(acc, o, LPR);
    if (MODE == GEMV_SWIGLU) acc2 += __shfl_xor(acc2, o, LPR);
  }
  if (MODE == GEMV_ARGMAX) {
    if (gl == 0) {
      if (row < a.rows) {
        a.out[row] = acc;
        best_s[g] = argmax_key(acc, row);
      } else {
        best_s[g] = 0;
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint64_t b = 0;
      for (int i = 0; i < G; ++i) b = best_s[i] > b ? best_s[i] : b;
      atomicMax((unsigned long long*)&a.state->best, (unsigned long long)b);
    }
  } else if (gl == 0 && row < a.rows) {
    if (MODE == GEMV_STORE) a.out[row] = a.bias ? acc + a.bias[row] : acc;
    if (MODE == GEMV_RESID) a.out[row] = a.out[row] + acc;
    if (MODE == GEMV_SWIGLU) a.out[row] = acc / (1.0f + expf(-acc)) * acc2;  // tensor.rs:224
  }
}

size_t gemv_lds_bytes(uint32_t type, uint32_t in) {
  return (size_t)in * 4 + (type == T_Q4_K ? (size_t)(in / 16) * 4 : 0);
}

template <uint32_t T, int LPR, int MODE>
static hipError_t go(const GemvArgs& a, hipStream_t s) {
  int pairs = ((a.in / 32) % 2) == 0;
  unsigned blocks = (a.rows + (256 / LPR) - 1) / (256 / LPR);
  hipLaunchKernelGGL((k_gemv<T, LPR, MODE>), dim3(blocks), dim3(256), gemv_lds_bytes(T, a.in), s, a, pairs);
  return hipGetLastError();
}

template <uint32_t T, int MODE>
static hipError_t pick_lpr(const GemvArgs& a, hipStream_t s) {
  // 16 lanes per row when that already gives >= 256 blocks; otherwise 64
  // lanes per row so small-row matrices still spread over the 256 CUs.
  if ((size_t)a.rows * 16 / 256 >= 256) return go<T, 16, MODE>(a, s);
  return go<T, 64, MODE>(a, s);
}

template <int MODE>
static hipError_t pick_type(const GemvArgs& a, hipStream_t s) {
  switch (a.type) {
    case T_Q4_K: return pick_lpr<T_Q4_K, MODE>(a, s);
    case T_Q6_K: return pick_lpr<T_Q6_K, MODE>(a, s);
    case T_Q8_0: return pick_lpr<T_Q8_0, MODE>(a, s);
    case T_Q5_0: return pick_lpr<T_Q5_0, MODE>(a, s);
    case T_F32: return pick_lpr<T_F32, MODE>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv(const GemvArgs& a, GemvMode mode, hipStream_t s) {
  switch (mode) {
    case GEMV_STORE: return pick_type<GEMV_STORE>(a, s);
    case GEMV_RESID: return pick_type<GEMV_RESID>(a, s);
    case GEMV_SWIGLU: return pick_type<GEMV_SWIGLU>(a, s);
    case GEMV_ARGMAX: return pick_type<GEMV_ARGMAX>(a, s);
  }
  return hipErrorInvalidValue;
}

template <uint32_t T, int LPR>
static hipError_t prep_one(size_t bytes) {
  hipError_t e;
  if ((e = hipFuncSetAttribute((const void*)k_gemv<T, LPR, GEMV_STORE>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes))) return e;
  if ((e = hipFuncSetAttribute((const void*)k_gemv<T, LPR, GEMV_RESID>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes))) return e;
  if ((e = hipFuncSetAttribute((const void*)k_gemv<T, LPR, GEMV_SWIGLU>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes))) return e;
  return hipFuncSetAttribute((const void*)k_gemv<T, LPR, GEMV_ARGMAX>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

hipError_t gemv_prepare(uint32_t max_in) {
  size_t bytes = gemv_lds_bytes(T_Q4_K, max_in);
  if (bytes < 65536) bytes = 65536;
  hipError_t e;
  if ((e = prep_one<T_Q4_K, 16>(bytes)) || (e = prep_one<T_Q4_K, 64>(bytes))) return e;
  if ((e = prep_one<T_Q6_K, 16>(bytes)) || (e = prep_one<T_Q6_K, 64>(bytes))) return e;
  if ((e = prep_one<T_Q8_0, 16>(bytes)) || (e = prep_one<T_Q8_0, 64>(bytes))) return e;
  if ((e = prep_one<T_Q5_0, 16>(bytes)) || (e = prep_one<T_Q5_0, 64>(bytes))) return e;
  if ((e = prep_one<T_F32, 16>(bytes)) || (e = prep_one<T_F32, 64>(bytes))) return e;
  return hipSuccess;
}

// ---- embedding row (model.rs:482-506) --------------------------------------
__global__ void k_embed(const uint8_t* __restrict__ table, uint32_t type, uint32_t hidden, uint32_t row_bytes,
                        StepState* st, float* __restrict__ x) {
  uint32_t tok = st->tok;
  if (blockIdx.x == 0 && threadIdx.x == 0) st->best = 0;
  const uint8_t* row = table + (size_t)tok * row_bytes;
  int be = blk_elems(type), bb = blk_bytes(type);
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
    x[i] = type == T_F32 ? ((const float*)row)[i] : decode_elem(type, row + (size_t)(i / be) * bb, (int)(i % be));
}

hipError_t launch_embed(const uint8_t* table, uint32_t type, uint32_t hidden, uint32_t row_bytes, StepState* st,
                        float* x, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3((hidden + 255) / 256), dim3(256), 0, s, table, type, hidden, row_bytes, st, x);
  return hipGetLastError();
}

// ---- RoPE at the absolute position + KV append (model.rs:193-217, 346-356)
// rope_cs holds, per position, cos[hd/2] | sin[hd/2] computed on the host
// with the same powf/sinf/cosf calls as the CPU path; the rotation itself is
// evaluated without FMA contraction, so q/k match the CPU bit for bit given
// equal inputs.
__global__ void k_rope_kv(float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                          const float* __restrict__ cs, uint32_t nh, uint32_t nkv, uint32_t hd,
                          float* __restrict__ kc, float* __restrict__ vc, const StepState* st) {
  uint32_t pos = st->pos, half = hd / 2;
  const float* cr = cs + (size_t)pos * hd;
  const float* sr = cr + half;
  uint32_t nq = nh * half, nk = nkv * half, kvd = nkv * hd;
  float* kdst = kc + (size_t)pos * kvd;
  float* vdst = vc + (size_t)pos * kvd;
  for (uint32_t i = threadIdx.x; i < nq + nk + kvd; i += blockDim.x) {
    if (i < nq + nk) {
      bool isq = i < nq;
      uint32_t ii = isq ? i : i - nq, h = ii / half, j = ii % half;
      const float* src = isq ? q : k;
      float a = src[h * hd + j], b = src[h * hd + j + half], c = cr[j], sn = sr[j];
      float r0 = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, sn));
      float r1 = __fadd_rn(__fmul_rn(a, sn), __fmul_rn(b, c));
      float* dst = isq ? q : kdst;
      dst[h * hd + j] = r0;
      dst[h * hd + j + half] = r1;
    } else {
      uint32_t ii = i - nq - nk;
      vdst[ii] = v[ii];
    }
  }
}

hipError_t launch_rope_kv(float* q, const float* k, const float* v, const float* rope_cs, uint32_t nh, uint32_t nkv,
                          uint32_t hd, float* kc, float* vc, const StepState* st, hipStream_t s) {
  hipLaunchKernelGGL(k_rope_kv, dim3(1), dim3(256), 0, s, q, k, v, rope_cs, nh, nkv, hd, kc, vc, st);
  return hipGetLastError();
}

// ---- GQA decode attention over the cache (model.rs:371-438) -----------------
// Block (kv head g, split s) scores positions [256 s, 256 s + 256) for all
// GQ query heads sharing g, so each cached K/V row is read once per block.
// Partial (o, m, l) per (head, split) is merged by k_attn_combine.
template <int HD, int GQM>
__global__ __launch_bounds__(256) void k_attn_split(const float* __restrict__ q, const float* __restrict__ kc,
                                                    const float* __restrict__ vc, uint32_t nh, uint32_t nkv,
                                                    uint32_t max_splits, float scale, float* __restrict__ part,
                                                    const StepState* st) {
  constexpr int DPL = HD / 16, PARTS = 256 / HD;
  __shared__ float qs[GQM * HD];
  __shared__ float sc[GQM * ATT_CHUNK];
  __shared__ float ml[GQM * 2];
  __shared__ float osum[PARTS * GQM * HD];
  const int GQ = (int)(nh / nkv);
  const uint32_t T = st->pos + 1, g = blockIdx.x, split = blockIdx.y, t0 = split * ATT_CHUNK;
  if (t0 >= T) return;
  const uint32_t n = min((uint32_t)ATT_CHUNK, T - t0);
  const size_t kvd = (size_t)nkv * HD;
  for (int i = threadIdx.x; i < GQ * HD; i += 256) qs[i] = q[(size_t)g * GQ * HD + i];
  __syncthreads();
  const int l16 = threadIdx.x & 15, slot = threadIdx.x >> 4;
  for (uint32_t tb = 0; tb < n; tb += 16) {
    uint32_t t = tb + slot;
    float kr[DPL];
    if (t < n) {
      const float4* kp = (const float4*)(kc + (size_t)(t0 + t) * kvd + (size_t)g * HD + l16 * DPL);
#pragma unroll
      for (int i = 0; i < DPL / 4; ++i) {
        float4 f = kp[i];
        kr[4 * i] = f.x; kr[4 * i + 1] = f.y; kr[4 * i + 2] = f.z; kr[4 * i + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < DPL; ++i) kr[i] = 0.f;
    }
#pragma unroll
    for (int h = 0; h < GQM; ++h) {
      if (h < GQ) {
        float p = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) p += kr[i] * qs[h * HD + l16 * DPL + i];
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) p += __shfl_xor(p, o, 16);
        if (l16 == 0 && t < n) sc[h * ATT_CHUNK + t] = p * scale;
      }
    }
  }
  __syncthreads();
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int h = wv; h < GQ; h += 4) {
    float m = -INFINITY;
    for (uint32_t t = lane; t < n; t += 64) m = fmaxf(m, sc[h * ATT_CHUNK + t]);
    m = wave_max(m);
    float l = 0.f;
    for (uint32_t t = lane; t < n; t += 64) {
      float p = expf(sc[h * ATT_CHUNK + t] - m);
      sc[h * ATT_CHUNK + t] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      ml[2 * h] = m;
      ml[2 * h + 1] = l;
    }
  }
  __syncthreads();
  const int d = threadIdx.x % HD, prt = threadIdx.x / HD;
  float acc[GQM];
#pragma unroll
  for (int h = 0; h < GQM; ++h) acc[h] = 0.f;
  for (uint32_t t = prt; t < n; t += PARTS) {
    float vv = vc[(size_t)(t0 + t) * kvd + (size_t)g * HD + d];
#pragma unroll
    for (int h = 0; h < GQM; ++h)
      if (h < GQ) acc[h] += sc[h * ATT_CHUNK + t] * vv;
  }
#pragma unroll
  for (int h = 0; h < GQM; ++h)
    if (h < GQ) osum[(prt * GQM + h) * HD + d] = acc[h];
  __syncthreads();
  for (int i = threadIdx.x; i < GQ * HD; i += 256) {
    int h = i / HD, dd = i % HD;
    float o = 0.f;
    for (int pp = 0; pp < PARTS; ++pp) o += osum[(pp * GQM + h) * HD + dd];
    float* dst = part + ((size_t)(g * GQ + h) * max_splits + split) * (HD + 2);
    dst[dd] = o;
    if (dd == 0) {
      dst[HD] = ml[2 * h];
      dst[HD + 1] = ml[2 * h + 1];
    }
  }
}

__global__ void k_attn_combine(const float* __restrict__ part, uint32_t hd, uint32_t max_splits,
                               float* __restrict__ att, const StepState* st) {
  const uint32_t h = blockIdx.x, T = st->pos + 1, ns = (T + ATT_CHUNK - 1) / ATT_CHUNK;
  const float* P = part + (size_t)h * max_splits * (hd + 2);
  float M = -INFINITY;
  for (uint32_t s = 0; s < ns; ++s) M = fmaxf(M, P[s * (hd + 2) + hd]);
  float L = 0.f;
  for (uint32_t s = 0; s < ns; ++s) L += P[s * (hd + 2) + hd + 1] * expf(P[s * (hd + 2) + hd] - M);
  for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
    float o = 0.f;
    for (uint32_t s = 0; s < ns; ++s) o += P[s * (hd + 2) + d] * expf(P[s * (hd + 2) + hd] - M);
    att[h * hd + d] = o / L;
  }
}

size_t attention_part_floats(uint32_t nh, uint32_t hd, uint32_t max_ctx) {
  uint32_t ms = (max_ctx + ATT_CHUNK - 1) / ATT_CHUNK;
  return (size_t)nh * ms * (hd + 2);
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc, uint32_t nh, uint32_t nkv, uint32_t hd,
                            uint32_t max_ctx, float scale, float* part, float* att, const StepState* st,
                            hipStream_t s) {
  uint32_t ms = (max_ctx + ATT_CHUNK - 1) / ATT_CHUNK, gq = nh / nkv;
  dim3 grid(nkv, ms);
  if (hd == 128 && gq <= 8)
    hipLaunchKernelGGL((k_attn_split<128, 8>), grid, dim3(256), 0, s, q, kc, vc, nh, nkv, ms, scale, part, st);
  else if (hd == 64 && gq <= 8)
    hipLaunchKernelGGL((k_attn_split<64, 8>), grid, dim3(256), 0, s, q, kc, vc, nh, nkv, ms, scale, part, st);
  else if (hd == 64 && gq <= 16)
    hipLaunchKernelGGL((k_attn_split<64, 16>), grid, dim3(256), 0, s, q, kc, vc, nh, nkv, ms, scale, part, st);
  else
    return hipErrorInvalidValue;
  hipError_t e = hipGetLastError();
  if (e) return e;
  hipLaunchKernelGGL(k_attn_combine, dim3(nh), dim3(128), 0, s, part, hd, ms, att, st);
  return hipGetLastError();
}

// ---- step bookkeeping and argmax (generate.rs:69-77) ------------------------
__global__ void k_step_end(StepState* st, int has_logits) {
  if (has_logits) {
    uint32_t idx = 0xFFFFFFFFu - (uint32_t)(st->best & 0xFFFFFFFFull);
    st->next_tok = idx;
    st->tok = idx;
  }
  st->pos += 1;
}

hipError_t launch_step_end(StepState* st, int has_logits, hipStream_t s) {
  hipLaunchKernelGGL(k_step_end, dim3(1), dim3(1), 0, s, st, has_logits);
  return hipGetLastError();
}

__global__ void k_argmax_init(uint64_t* best) { *best = 0; }
__global__ void k_argmax_blocks(const float* __restrict__ x, size_t n, uint64_t* best) {
  __shared__ uint64_t wb[4];
  uint64_t b = 0;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint64_t k = argmax_key(x[i], (uint32_t)i);
    b = k > b ? k : b;
  }
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t other = __shfl_xor(b, o, 64);
    b = other > b ? other : b;
  }
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; ++i) b = wb[i] > wb[0] ? (wb[0] = wb[i]) : wb[0];
    atomicMax((unsigned long long*)best, (unsigned long long)wb[0]);
  }
}
__global__ void k_argmax_final(const uint64_t* best, uint32_t* out) {
  *out = 0xFFFFFFFFu - (uint32_t)(*best & 0xFFFFFFFFull);
}

hipError_t launch_argmax(const float* x, size_t n, uint64_t* scratch, uint32_t* out, hipStream_t s) {
  hipLaunchKernelGGL(k_argmax_init, dim3(1), dim3(1), 0, s, scratch);
  size_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  if (blocks == 0) blocks = 1;
  hipLaunchKernelGGL(k_argmax_blocks, dim3((unsigned)blocks), dim3(256), 0, s, x, n, scratch);
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1), 0, s, scratch, out);
  return hipGetLastError();
}

}  // namespace frn
