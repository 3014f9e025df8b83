// gfx950 kernels of the token loop: dequant, fused dequant-GEMV, embedding,
// RoPE + KV-cache write, split-sequence GQA decode attention, argmax.
#include "formats.hpp"
#include "kernels.hpp"

namespace frn {

constexpr int ATT_CHUNK = 64;  // positions per attention block (one wave per softmax row)

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

// Per-format raw-register type and prefetch depth (items in flight per lane).
template <uint32_t T>
struct Fmt;
template <>
struct Fmt<T_Q4_K> {
  using Raw = Q4KRaw;
  static constexpr int B = 8;
  static __device__ __forceinline__ Raw load(const uint8_t* row, int it, bool) { return q4k_load(row, it); }
  static __device__ __forceinline__ float dot(const Raw& r, const uint8_t*, int it, const XLds& X, bool) {
    return q4k_dot(r, it, X);
  }
};
template <>
struct Fmt<T_Q6_K> {
  using Raw = Q6KRaw;
  static constexpr int B = 6;
  static __device__ __forceinline__ Raw load(const uint8_t* row, int it, bool) { return q6k_load(row, it); }
  static __device__ __forceinline__ float dot(const Raw& r, const uint8_t*, int it, const XLds& X, bool) {
    return q6k_dot(r, it, X);
  }
};
template <>
struct Fmt<T_Q8_0> {
  using Raw = Q8PairRaw;
  static constexpr int B = 4;
  static __device__ __forceinline__ Raw load(const uint8_t* row, int it, bool pairs) {
    Raw r;
    if (pairs) r = q8_0_pair_load(row, it);
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw& r, const uint8_t* row, int it, const XLds& X, bool pairs) {
    return pairs ? q8_0_pair_dot(r, it, X) : small_block_item(T_Q8_0, row, it, X.xf);
  }
};
template <>
struct Fmt<T_Q5_0> {
  using Raw = Q5PairRaw;
  static constexpr int B = 4;
  static __device__ __forceinline__ Raw load(const uint8_t* row, int it, bool pairs) {
    Raw r;
    if (pairs) r = q5_0_pair_load(row, it);
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw& r, const uint8_t* row, int it, const XLds& X, bool pairs) {
    return pairs ? q5_0_pair_dot(r, it, X.xf) : small_block_item(T_Q5_0, row, it, X.xf);
  }
};
struct F32Raw {
  float4 w[4];
};
template <>
struct Fmt<T_F32> {  // 16 floats per item
  using Raw = F32Raw;
  static constexpr int B = 4;
  static __device__ __forceinline__ Raw load(const uint8_t* row, int it, bool) {
    Raw r;
    const float4* w = (const float4*)row + it * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.w[i] = w[i];
    return r;
  }
  static __device__ __forceinline__ float dot(const Raw& r, const uint8_t*, int it, const XLds& X, bool) {
    const float4* Xp = (const float4*)X.xf + it * 4;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 b = Xp[i];
      s += r.w[i].x * b.x + r.w[i].y * b.y + r.w[i].z * b.z + r.w[i].w * b.w;
    }
    return s;
  }
};

// ---- activation staging ------------------------------------------------------
// Async global -> LDS copy of n floats (n % 4 == 0): each wave instruction
// moves 64 x 16 B with global_load_lds_dwordx4, so staging costs one memory
// latency however long the vector is, and no VGPRs.  Caller waits + syncs.
__device__ __forceinline__ void lds_copy_issue(const float* __restrict__ src, float* dst, uint32_t n) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n16 = n / 4;
  for (uint32_t base = wave * 64; base < n16; base += 256)
    if (base + lane < n16)
      __builtin_amdgcn_global_load_lds((const void*)(src + 4 * (base + lane)),
                                       (__attribute__((address_space(3))) void*)(dst + 4 * base), 16, 0, 0);
}

// After the copies of x (and the rmsnorm gain) have landed: apply rmsnorm
// (tensor.rs:164-185: x * (1 / sqrt(mean(x^2) + eps)) * w) in place, then
// split every 32-value chunk into the int8 digit planes + metadata that the
// quantized items read (see XLds in formats.hpp).  Each thread handles 8
// consecutive values; the 4 threads of a chunk are adjacent lanes.
__device__ __forceinline__ void stage_finish(uint32_t K, bool norm, float eps, float* xf, const float* nw,
                                             uint8_t* pl, float* red4) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  float inv = 1.0f;
  if (norm) {
    float ss = 0.f;
    for (uint32_t i = threadIdx.x * 4; i < K; i += 1024) {
      float4 v = *(const float4*)(xf + i);
      ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = block_sum256(ss, red4);
    inv = 1.0f / sqrtf(ss / (float)K + eps);
  }
  const uint32_t n16 = K / 16;
  for (uint32_t u0 = 0; u0 < K / 8; u0 += 256) {  // uniform trip count: the shuffles need whole groups
    const uint32_t u = u0 + threadIdx.x;
    const bool live = u < K / 8;
    float v[8];
    float4* p = (float4*)(xf + 8 * (live ? u : 0));
    float4 a = p[0], b = p[1];
    if (norm && live) {
      const float4* w = (const float4*)(nw + 8 * u);
      float4 wa = w[0], wb = w[1];
      a.x = a.x * inv * wa.x; a.y = a.y * inv * wa.y; a.z = a.z * inv * wa.z; a.w = a.w * inv * wa.w;
      b.x = b.x * inv * wb.x; b.y = b.y * inv * wb.y; b.z = b.z * inv * wb.z; b.w = b.w * inv * wb.w;
      p[0] = a;
      p[1] = b;
    }
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    float amax = 0.f, xsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      amax = fmaxf(amax, fabsf(v[i]));
      xsum += v[i];
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 4));  // over the 32-value chunk
    const float inv_s = amax > 0.f ? 127.0f / amax : 0.f;
    const float cs = amax > 0.f ? (1.0f / inv_s) * (1.0f / 16384.0f) : 0.f;
    uint32_t w0[2] = {0, 0}, w1[2] = {0, 0}, w2[2] = {0, 0};
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float t = v[i] * inv_s;
      float r0 = rintf(t), e0 = (t - r0) * 128.0f;
      float r1 = rintf(e0), e1 = (e0 - r1) * 128.0f;
      float r2 = rintf(e1);
      int d0 = (int)r0, d1 = (int)r1, d2 = (int)r2;
      w0[i >> 2] |= (uint32_t)(d0 & 0xFF) << (8 * (i & 3));
      w1[i >> 2] |= (uint32_t)(d1 & 0xFF) << (8 * (i & 3));
      w2[i >> 2] |= (uint32_t)(d2 & 0xFF) << (8 * (i & 3));
      s0 += d0;
      s1 += d1;
      s2 += d2;
    }
    // per 16-value record: the two threads u, u^1
    xsum += __shfl_xor(xsum, 1, 2);
    s0 += __shfl_xor(s0, 1, 2);
    s1 += __shfl_xor(s1, 1, 2);
    s2 += __shfl_xor(s2, 1, 2);
    if (live) {
      const uint32_t c = u >> 1, off = 16u * swz(c, n16) + 8u * (u & 1);
      *(uint2*)(pl + off) = make_uint2(w0[0], w0[1]);
      *(uint2*)(pl + K + off) = make_uint2(w1[0], w1[1]);
      *(uint2*)(pl + 2 * K + off) = make_uint2(w2[0], w2[1]);
      if ((u & 1) == 0)
        *(float4*)(pl + 3 * K + 16u * swz(c, n16)) =
            make_float4(cs, xsum, __int_as_float(s0), __int_as_float(128 * s1 + s2));
    }
  }
  __syncthreads();
}

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal in the reference
  uint32_t u = __float_as_uint(v);
  uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

// ---- fused dequant-GEMV -----------------------------------------------------------
// A block stages x (and applies the rmsnorm) once; then each of its 4 waves
// works alone through "units" of 64 / LPR rows, one group of LPR lanes per
// row (SWIGLU: per gate/up row pair).  Wave w of block b takes units
// 4b + w, 4b + w + 4 * nblk, ...  Lane gl owns items gl, gl + LPR, ... of
// its row; the loads of the next unit are issued before the current one is
// computed (double buffer), and the first unit's loads before the staging.
template <uint32_t T, int LPR, int MODE>
struct Gemv {
  using F = Fmt<T>;
  using Raw = typename F::Raw;
  static constexpr int B = F::B;
  static constexpr int R = MODE == GEMV_SWIGLU ? 2 : 1;
  static constexpr int G = 64 / LPR;  // rows per unit
  static_assert(B % R == 0, "batch must hold whole row groups");

  const GemvArgs& a;
  const GemvSeg& sg;
  const XLds& X;
  int gl, g;
  bool pr;
  int n_items;

  __device__ __forceinline__ uint32_t row_of(uint32_t unit) const { return unit * G + g; }
  __device__ __forceinline__ int work(uint32_t row) const {
    return (row < sg.rows && gl < n_items) ? (n_items - gl + LPR - 1) / LPR * R : 0;
  }
  __device__ __forceinline__ const uint8_t* wrow(uint32_t row, int r) const {
    return (r == 0 ? sg.w : sg.w2) + (size_t)row * sg.row_bytes;
  }
  __device__ __forceinline__ int issue(uint32_t unit, Raw (&raw)[B]) const {
    const uint32_t row = row_of(unit);
    const int n = work(row), nb = n < B ? n : B;
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (b < nb) raw[b] = F::load(wrow(row, b % R), gl + (b / R) * LPR, pr);
    return nb;
  }
  // consume a unit whose first batch is in raw; returns the row's results
  __device__ __forceinline__ void compute(uint32_t unit, Raw (&raw)[B], int nb, uint64_t& best) const {
    const uint32_t row = row_of(unit);
    const int n_work = work(row);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    int k0 = 0;
    while (nb > 0) {
#pragma unroll
      for (int b = 0; b < B; ++b)
        if (b < nb) acc[b % R] += F::dot(raw[b], wrow(row, b % R), gl + ((k0 + b) / R) * LPR, X, pr);
      k0 += nb;
      nb = n_work - k0 < B ? n_work - k0 : B;
#pragma unroll
      for (int b = 0; b < B; ++b)  // rows longer than one batch: further batches, not prefetched
        if (b < nb) raw[b] = F::load(wrow(row, b % R), gl + ((k0 + b) / R) * LPR, pr);
    }
    float acc0 = acc[0], acc1 = acc[R - 1];
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) {
      acc0 += __shfl_xor(acc0, o, LPR);
      if (MODE == GEMV_SWIGLU) acc1 += __shfl_xor(acc1, o, LPR);
    }
    if (gl == 0 && row < sg.rows) {
      if (MODE == GEMV_STORE) sg.out[row] = sg.bias ? acc0 + sg.bias[row] : acc0;  // model.rs:179-183
      if (MODE == GEMV_RESID) {
        float v = sg.resid[row] + acc0;  // tensor.rs:232
        sg.out[row] = v;
        if (sg.out2) sg.out2[row] = v;
      }
      if (MODE == GEMV_SWIGLU) sg.out[row] = acc0 / (1.0f + expf(-acc0)) * acc1;  // tensor.rs:224
      if (MODE == GEMV_ARGMAX) {
        sg.out[row] = acc0;
        uint64_t kk = argmax_key(acc0, row);
        best = kk > best ? kk : best;
      }
    }
  }
};

template <uint32_t T, int LPR, int MODE>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, const GemvSeg& sg, uint32_t blk, uint32_t nblk, float* xs,
                                          float* nw, uint8_t* pl, float* red4, uint64_t* best_s) {
  using W = Gemv<T, LPR, MODE>;
  const XLds X{xs, pl, a.in};
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool pr = ((a.in / 32) % 2) == 0;
  const W w{a, sg, X, lane % LPR, lane / LPR, pr, items_per_row(T, a.in, pr)};
  const uint32_t n_units = (sg.rows + W::G - 1) / W::G, stride = 4 * nblk;
  uint32_t unit = 4 * blk + wave;
  typename W::Raw ra[W::B], rb[W::B];
  int na = unit < n_units ? w.issue(unit, ra) : 0, nb = 0;
  lds_copy_issue(a.x, xs, a.in);
  if (a.norm_w) lds_copy_issue(a.norm_w, nw, a.in);
  stage_finish(a.in, a.norm_w != nullptr, a.eps, xs, nw, pl, red4);
  uint64_t best = 0;
  while (unit < n_units) {  // per-wave loop, unrolled by two for the double buffer
    uint32_t next = unit + stride;
    if (next < n_units) nb = w.issue(next, rb);
    w.compute(unit, ra, na, best);
    unit = next;
    if (unit >= n_units) break;
    next = unit + stride;
    if (next < n_units) na = w.issue(next, ra);
    w.compute(unit, rb, nb, best);
    unit = next;
  }
  if (MODE == GEMV_ARGMAX) {
    for (int o = 32; o > 0; o >>= 1) {
      uint64_t other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    if (lane == 0) best_s[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
      uint64_t b = best_s[0];
      for (int i = 1; i < 4; ++i) b = best_s[i] > b ? best_s[i] : b;
      a.best[blockIdx.x] = b;
    }
  }
}

// T0 serves every segment whose type is T0, T1 the others (T1 == T0 for
// single-format launches), so each kernel carries one or two format paths.
template <uint32_t T0, uint32_t T1, int LPR, int MODE>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  extern __shared__ float4 smem4[];
  __shared__ float red4[4];
  __shared__ uint64_t best_s[4];
  // LDS: x[in] f32 | 4 byte planes of in bytes (digits, metadata) | norm gain[in] (only with a norm)
  float* xs = (float*)smem4;
  uint8_t* pl = (uint8_t*)(xs + a.in);
  float* nw = (float*)(pl + 4 * (size_t)a.in);
  int si = 0;
  while (si + 1 < a.n_seg && blockIdx.x >= a.seg[si + 1].block0) ++si;
  const GemvSeg& sg = a.seg[si];
  const uint32_t blk = blockIdx.x - sg.block0;
  const uint32_t nblk = (si + 1 < a.n_seg ? a.seg[si + 1].block0 : gridDim.x) - sg.block0;
  if (T0 == T1 || sg.type == T0)
    gemv_body<T0, LPR, MODE>(a, sg, blk, nblk, xs, nw, pl, red4, best_s);
  else
    gemv_body<T1, LPR, MODE>(a, sg, blk, nblk, xs, nw, pl, red4, best_s);
}

size_t gemv_lds_bytes(uint32_t in, bool norm) { return (size_t)in * (4 + 4 + (norm ? 4 : 0)); }

// Lanes per row: 16 when the launch has enough rows to fill the GPU with
// groups of 16 rows, else 32 or 64 so small matrices still spread over the
// 256 CUs -- but never so many that most lanes of a group sit idle.
static int lanes_per_row(uint32_t total_rows, int n_items) {
  int lpr = total_rows >= 8192 ? 16 : total_rows >= 4096 ? 32 : 64;
  while (lpr > 16 && n_items <= lpr / 2) lpr /= 2;
  return lpr;
}

constexpr uint32_t GEMV_MAX_BLOCKS = 512;  // 2 resident blocks (8 waves) per CU

// Blocks per segment in proportion to its units of 64 / LPR rows; each
// block runs 4 wave workers.
static uint32_t plan_blocks(GemvArgs& a, uint32_t rows_per_unit) {
  uint32_t want[3], total = 0;
  for (int i = 0; i < a.n_seg; ++i) {
    uint32_t units = (a.seg[i].rows + rows_per_unit - 1) / rows_per_unit;
    want[i] = (units + 3) / 4;
    total += want[i];
  }
  uint32_t grid = total < GEMV_MAX_BLOCKS ? total : GEMV_MAX_BLOCKS, used = 0;
  for (int i = 0; i < a.n_seg; ++i) {
    uint32_t b = i + 1 == a.n_seg ? grid - used : (uint32_t)(((uint64_t)grid * want[i] + total / 2) / total);
    if (b < 1) b = 1;
    if (b > want[i]) b = want[i];
    a.seg[i].block0 = used;
    used += b;
  }
  return used;
}

uint32_t gemv_blocks(uint32_t type, uint32_t rows, uint32_t in) {
  int lpr = lanes_per_row(rows, items_per_row(type, in, ((in / 32) % 2) == 0));
  uint32_t units = (rows + 64 / lpr - 1) / (64 / lpr), want = (units + 3) / 4;
  return want < GEMV_MAX_BLOCKS ? want : GEMV_MAX_BLOCKS;
}

template <uint32_t T0, uint32_t T1, int LPR, int MODE>
static hipError_t go(GemvArgs a, hipStream_t s, uint32_t* nblocks) {
  uint32_t total = plan_blocks(a, 64 / LPR);
  if (nblocks) *nblocks = total;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL((k_gemv<T0, T1, LPR, MODE>), dim3(total), dim3(256), gemv_lds_bytes(a.in, a.norm_w != nullptr),
                     s, a);
  return hipGetLastError();
}

template <uint32_t T0, uint32_t T1, int MODE>
static hipError_t pick_lpr(const GemvArgs& a, hipStream_t s, uint32_t* nb) {
  uint32_t rows = 0;
  for (int i = 0; i < a.n_seg; ++i) rows += a.seg[i].rows;
  int lpr = lanes_per_row(rows, items_per_row(a.seg[0].type, a.in, ((a.in / 32) % 2) == 0));
  if (lpr == 16) return go<T0, T1, 16, MODE>(a, s, nb);
  if (lpr == 32) return go<T0, T1, 32, MODE>(a, s, nb);
  return go<T0, T1, 64, MODE>(a, s, nb);
}

template <int MODE>
static hipError_t pick_types(const GemvArgs& a, hipStream_t s, uint32_t* nb) {
  uint32_t t0 = a.seg[0].type, t1 = t0;
  for (int i = 1; i < a.n_seg; ++i)
    if (a.seg[i].type != t0) {
      if (t1 != t0 && a.seg[i].type != t1) return hipErrorNotSupported;
      t1 = a.seg[i].type;
    }
  if (t0 == t1) {
    switch (t0) {
      case T_Q4_K: return pick_lpr<T_Q4_K, T_Q4_K, MODE>(a, s, nb);
      case T_Q6_K: return pick_lpr<T_Q6_K, T_Q6_K, MODE>(a, s, nb);
      case T_Q8_0: return pick_lpr<T_Q8_0, T_Q8_0, MODE>(a, s, nb);
      case T_Q5_0: return pick_lpr<T_Q5_0, T_Q5_0, MODE>(a, s, nb);
      case T_F32: return pick_lpr<T_F32, T_F32, MODE>(a, s, nb);
    }
    return hipErrorInvalidValue;
  }
  if (t0 == T_Q4_K && t1 == T_Q6_K) return pick_lpr<T_Q4_K, T_Q6_K, MODE>(a, s, nb);
  if (t0 == T_Q6_K && t1 == T_Q4_K) return pick_lpr<T_Q6_K, T_Q4_K, MODE>(a, s, nb);
  return hipErrorNotSupported;
}

// Mixed formats without a two-format kernel: one launch per segment.
template <int MODE>
static hipError_t launch_split(const GemvArgs& a, hipStream_t s, uint32_t* nb) {
  hipError_t e = pick_types<MODE>(a, s, nb);
  if (e != hipErrorNotSupported) return e;
  for (int i = 0; i < a.n_seg; ++i) {
    GemvArgs one = a;
    one.n_seg = 1;
    one.seg[0] = a.seg[i];
    if ((e = pick_types<MODE>(one, s, nb))) return e;
  }
  return hipSuccess;
}

hipError_t launch_gemv(GemvArgs a, GemvMode mode, hipStream_t s, uint32_t* nb) {
  switch (mode) {
    case GEMV_STORE: return launch_split<GEMV_STORE>(a, s, nb);
    case GEMV_RESID: return launch_split<GEMV_RESID>(a, s, nb);
    case GEMV_SWIGLU: return launch_split<GEMV_SWIGLU>(a, s, nb);
    case GEMV_ARGMAX: return launch_split<GEMV_ARGMAX>(a, s, nb);
  }
  return hipErrorInvalidValue;
}

template <uint32_t T0, uint32_t T1, int LPR>
static hipError_t prep_one(int bytes) {
  hipError_t e;
  if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_STORE>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes))) return e;
  if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_RESID>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes))) return e;
  if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_SWIGLU>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes))) return e;
  return hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_ARGMAX>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <uint32_t T0, uint32_t T1>
static hipError_t prep_types(int bytes) {
  hipError_t e;
  if ((e = prep_one<T0, T1, 16>(bytes)) || (e = prep_one<T0, T1, 32>(bytes))) return e;
  return prep_one<T0, T1, 64>(bytes);
}

hipError_t gemv_prepare(size_t bytes) {
  if (bytes < 65536) bytes = 65536;
  int b = (int)bytes;
  hipError_t e;
  if ((e = prep_types<T_Q4_K, T_Q4_K>(b)) || (e = prep_types<T_Q6_K, T_Q6_K>(b)) ||
      (e = prep_types<T_Q8_0, T_Q8_0>(b)) || (e = prep_types<T_Q5_0, T_Q5_0>(b)) ||
      (e = prep_types<T_F32, T_F32>(b)) || (e = prep_types<T_Q4_K, T_Q6_K>(b)) || (e = prep_types<T_Q6_K, T_Q4_K>(b)))
    return e;
  return hipSuccess;
}

// ---- embedding row (model.rs:482-506) --------------------------------------
__global__ void k_embed(const uint8_t* __restrict__ table, uint32_t type, uint32_t hidden, uint32_t row_bytes,
                        StepState* st, float* __restrict__ x) {
  uint32_t tok = st->tok;
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

// ---- decode attention (model.rs:193-217, 346-356, 371-438) ---------------------
// One launch per layer.  Block (kv head g, split s) covers positions
// [64 s, 64 s + 64) for the GQ query heads sharing g:
//  - rotates those query heads and head g's new key at the step position
//    (rope_cs holds cos[hd/2] | sin[hd/2] per position, computed on the host
//    with the CPU path's powf/sinf/cosf; the rotation is evaluated without
//    FMA contraction, so q/k match the CPU bit for bit given equal inputs);
//  - the block holding the step position appends head g's k/v to the cache;
//  - scores, chunk softmax and P.V from K rows in registers and V rows in
//    LDS, all loads issued up front; partial (o, m, l) per head to `part`;
//  - the last block of kv head g to finish (atomic counter) merges the
//    splits into att and re-zeroes the counter.
template <int HD, int GQM>
__global__ __launch_bounds__(256) void k_attention(const float* __restrict__ q, const float* __restrict__ kn,
                                                   const float* __restrict__ vn, const float* __restrict__ cs,
                                                   float* __restrict__ kc, float* __restrict__ vc, uint32_t nh,
                                                   uint32_t nkv, uint32_t max_splits, float scale,
                                                   float* __restrict__ part, uint32_t* counters,
                                                   float* __restrict__ att, const StepState* st) {
  constexpr int C = ATT_CHUNK, TPP = 256 / C, DPT = HD / TPP, PARTS = 256 / HD, HALF = HD / 2;
  __shared__ float qs[GQM * HD];
  __shared__ float kcur[HD], vcur[HD];
  __shared__ float vs[C * HD];
  __shared__ float ps[GQM * C];
  __shared__ float ml[GQM * 2];
  __shared__ float osum[PARTS * GQM * HD];
  __shared__ uint32_t last_flag;
  const int GQ = (int)(nh / nkv);
  const uint32_t pos = st->pos, T = pos + 1, g = blockIdx.x, split = blockIdx.y, t0 = split * C;
  if (t0 >= T) return;
  const uint32_t n = min((uint32_t)C, T - t0), ns = (T + C - 1) / C;
  const size_t kvd = (size_t)nkv * HD;
  const int p = threadIdx.x / TPP, sub = threadIdx.x % TPP;
  const uint32_t tp = t0 + p;
  const bool valid = (uint32_t)p < n, cur = valid && tp == pos;
  // cached rows (positions < pos); the step's own row comes from kcur/vcur
  const size_t off = (size_t)((valid && !cur) ? tp : 0) * kvd + (size_t)g * HD + sub * DPT;
  float4 kr[DPT / 4], vr[DPT / 4];
#pragma unroll
  for (int i = 0; i < DPT / 4; ++i) {
    kr[i] = ((const float4*)(kc + off))[i];
    vr[i] = ((const float4*)(vc + off))[i];
  }
  const float* cr = cs + (size_t)pos * HD;
  for (int i = threadIdx.x; i < GQ * HALF + HALF; i += 256) {
    int h = i / HALF, j = i % HALF;
    const float* src = h < GQ ? q + (size_t)(g * GQ + h) * HD : kn + (size_t)g * HD;
    float a0 = src[j], b0 = src[j + HALF], c0 = cr[j], s0 = cr[HALF + j];
    float r0 = __fsub_rn(__fmul_rn(a0, c0), __fmul_rn(b0, s0));
    float r1 = __fadd_rn(__fmul_rn(a0, s0), __fmul_rn(b0, c0));
    float* dst = h < GQ ? qs + h * HD : kcur;
    dst[j] = r0;
    dst[j + HALF] = r1;
  }
  for (int d = threadIdx.x; d < HD; d += 256) vcur[d] = vn[(size_t)g * HD + d];
  __syncthreads();
  if (split == ns - 1)  // KvCache::append of head g at pos
    for (int d = threadIdx.x; d < HD; d += 256) {
      kc[(size_t)pos * kvd + (size_t)g * HD + d] = kcur[d];
      vc[(size_t)pos * kvd + (size_t)g * HD + d] = vcur[d];
    }
  if (cur) {
#pragma unroll
    for (int i = 0; i < DPT / 4; ++i) {
      kr[i] = ((const float4*)(kcur + sub * DPT))[i];
      vr[i] = ((const float4*)(vcur + sub * DPT))[i];
    }
  }
#pragma unroll
  for (int i = 0; i < DPT / 4; ++i)
    ((float4*)(vs + p * HD + sub * DPT))[i] = valid ? vr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int h = 0; h < GQM; ++h) {
    if (h < GQ) {
      const float4* qh = (const float4*)(qs + h * HD + sub * DPT);
      float sdot = 0.f;
#pragma unroll
      for (int i = 0; i < DPT / 4; ++i) {
        float4 a = kr[i], b = qh[i];
        sdot += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
      }
#pragma unroll
      for (int o = TPP / 2; o > 0; o >>= 1) sdot += __shfl_xor(sdot, o, TPP);
      if (sub == 0) ps[h * C + p] = valid ? sdot * scale : -INFINITY;  // model.rs:397
    }
  }
  __syncthreads();
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int h = wv; h < GQ; h += 4) {  // C == 64: one wave per softmax row
    float v = ps[h * C + lane];
    float m = wave_max(v);
    float e = expf(v - m);
    ps[h * C + lane] = e;
    float l = wave_sum(e);
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
    float vv = vs[t * HD + d];
#pragma unroll
    for (int h = 0; h < GQM; ++h)
      if (h < GQ) acc[h] += ps[h * C + t] * vv;
  }
#pragma unroll
  for (int h = 0; h < GQM; ++h)
    if (h < GQ) osum[(prt * GQM + h) * HD + d] = acc[h];
  __syncthreads();
  for (int i = threadIdx.x; i < GQ * HD; i += 256) {
    int h = i / HD, dd = i % HD;
    float o = 0.f;
#pragma unroll
    for (int pp = 0; pp < PARTS; ++pp) o += osum[(pp * GQM + h) * HD + dd];
    float* dst = part + ((size_t)(g * GQ + h) * max_splits + split) * (HD + 2);
    dst[dd] = o;
    if (dd == 0) {
      dst[HD] = ml[2 * h];
      dst[HD + 1] = ml[2 * h + 1];
    }
  }
  // publish the partial, count finished splits of kv head g
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last_flag = atomicAdd(&counters[g], 1u) == ns - 1;
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  if (threadIdx.x == 0) counters[g] = 0;
  for (int i = threadIdx.x; i < GQ * HD; i += 256) {
    int h = i / HD, dd = i % HD;
    const float* P = part + (size_t)(g * GQ + h) * max_splits * (HD + 2);
    float M = -INFINITY;
    for (uint32_t sp = 0; sp < ns; ++sp) M = fmaxf(M, P[sp * (HD + 2) + HD]);
    float L = 0.f, o = 0.f;
    for (uint32_t sp = 0; sp < ns; ++sp) {
      float w = expf(P[sp * (HD + 2) + HD] - M);
      L += P[sp * (HD + 2) + HD + 1] * w;
      o += P[sp * (HD + 2) + dd] * w;
    }
    att[(size_t)(g * GQ + h) * HD + dd] = o / L;
  }
}

size_t attention_part_floats(uint32_t nh, uint32_t hd, uint32_t max_ctx) {
  uint32_t ms = (max_ctx + ATT_CHUNK - 1) / ATT_CHUNK;
  return (size_t)nh * ms * (hd + 2);
}

hipError_t launch_attention(const float* q, const float* k, const float* v, const float* cs, float* kc, float* vc,
                            uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_ctx, float scale, float* part,
                            uint32_t* counters, float* att, const StepState* st, hipStream_t s) {
  uint32_t ms = (max_ctx + ATT_CHUNK - 1) / ATT_CHUNK, gq = nh / nkv;
  dim3 grid(nkv, ms);
  if (hd == 128 && gq <= 8)
    hipLaunchKernelGGL((k_attention<128, 8>), grid, dim3(256), 0, s, q, k, v, cs, kc, vc, nh, nkv, ms, scale, part,
                       counters, att, st);
  else if (hd == 64 && gq <= 16)
    hipLaunchKernelGGL((k_attention<64, 16>), grid, dim3(256), 0, s, q, k, v, cs, kc, vc, nh, nkv, ms, scale, part,
                       counters, att, st);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---- step bookkeeping and argmax (generate.rs:69-77) ------------------------
// 1024 threads: max over the lm_head blocks' packed candidates (largest
// logit, then smallest row), then advance the position.
__global__ __launch_bounds__(1024) void k_step_end(StepState* st, const uint64_t* __restrict__ best,
                                                   uint32_t n_best) {
  __shared__ uint64_t wb[16];
  if (best) {
    uint64_t b = 0;
    for (uint32_t i = threadIdx.x; i < n_best; i += 1024) b = best[i] > b ? best[i] : b;
    for (int o = 32; o > 0; o >>= 1) {
      uint64_t other = __shfl_xor(b, o, 64);
      b = other > b ? other : b;
    }
    if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int i = 1; i < 16; ++i) b = wb[i] > b ? wb[i] : b;
      uint32_t idx = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull);
      st->next_tok = idx;
      st->tok = idx;
    }
  }
  if (threadIdx.x == 0) st->pos += 1;
}

hipError_t launch_step_end(StepState* st, const uint64_t* best, uint32_t n_best, hipStream_t s) {
  hipLaunchKernelGGL(k_step_end, dim3(1), dim3(1024), 0, s, st, best, n_best);
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
