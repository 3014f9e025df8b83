// GEMV items of each weight format (loads and dots over the staged
// activation vector) and the packed argmax key, shared by the per-launch
// GEMV kernels and the resident decode kernel.
#pragma once
#include "formats.hpp"
#include "kernels.hpp"

namespace frn {

// ---- fused dequant-GEMV ---------------------------------------------------
__host__ __device__ inline int items_per_row(uint32_t t, uint32_t in, bool pairs) {
  if (t == T_Q4_K || t == T_Q6_K) return (int)(in / 256) * 8;
  if (t == T_Q8_0 || t == T_Q5_0) return (int)(pairs ? in / 64 : in / 32);
  return (int)(in / 16);  // F32, F16: 16 values per item
}

// Items of one row a lane loads per pipeline step: 3 for the K-quants (also
// for SWIGLU's two rows per lane: 248 VGPRs, still 2 blocks per CU; 16
// lanes x 3 items cover a 1536-value row exactly, where 32 x 2 left a
// quarter of the slots masked), 2 for the others, one less for SWIGLU.
__host__ __device__ constexpr int gemv_bi(uint32_t t, int mode) {
  return t == T_Q4_K || t == T_Q6_K ? 3 : 2 - (mode == GEMV_SWIGLU ? 1 : 0);
}

// Per-format raw-register type, the NC staged chunks an item reads
// (chunk(it, i)), and dot(), which gets the row's byte offset (alignment of
// the 2-byte aligned formats), its pointer (nullptr for a masked item; only
// the odd-block fallback reads through it) and the item's chunks.  NC == 0:
// the item reads the f32 copy of x in LDS instead.
template <uint32_t T>
struct Fmt;
template <>
struct Fmt<T_Q4_K> {
  using Raw = Q4KRaw;
  static constexpr int NC = 2;
  static __device__ __forceinline__ uint32_t chunk(int it, int i, bool) { return q4k_chunk(it, i); }
  static __device__ __forceinline__ Raw load(rsrc_t r, uint32_t row, int it, bool) { return q4k_load(r, row, it); }
  template <class XT>
  static __device__ __forceinline__ float dot(const Raw& w, uint32_t, const uint8_t*, int it, const XT* x,
                                              const XLds&, bool) {
    return q4k_dot(w, it, x[0], x[1]);
  }
};
template <>
struct Fmt<T_Q6_K> {
  using Raw = Q6KRaw;
  static constexpr int NC = 2;
  static __device__ __forceinline__ uint32_t chunk(int it, int i, bool) { return q6k_chunk(it, i); }
  static __device__ __forceinline__ Raw load(rsrc_t r, uint32_t row, int it, bool) { return q6k_load(r, row, it); }
  template <class XT>
  static __device__ __forceinline__ float dot(const Raw& w, uint32_t row, const uint8_t*, int it, const XT* x,
                                              const XLds&, bool) {
    return q6k_dot(w, row, it, x[0], x[1]);
  }
};
template <>
struct Fmt<T_Q8_0> {
  using Raw = Q8PairRaw;
  static constexpr int NC = 4;
  static __device__ __forceinline__ uint32_t chunk(int it, int i, bool pairs) {
    return pairs ? q8_0_pair_chunk(it, i) : 0u;
  }
  static __device__ __forceinline__ Raw load(rsrc_t r, uint32_t row, int it, bool pairs) {
    return q8_0_pair_load(r, pairs ? row : BUF_INVALID, it);
  }
  template <class XT>
  static __device__ __forceinline__ float dot(const Raw& w, uint32_t, const uint8_t* rowp, int it, const XT* x,
                                              const XLds& X, bool pairs) {
    if (pairs) return q8_0_pair_dot(w, {x[0], x[1], x[2], x[3]});
    return rowp ? small_block_item(T_Q8_0, rowp, it, X.xf) : 0.f;
  }
};
template <>
struct Fmt<T_Q5_0> {
  using Raw = Q5PairRaw;
  static constexpr int NC = 0;
  static __device__ __forceinline__ uint32_t chunk(int, int, bool) { return 0u; }
  static __device__ __forceinline__ Raw load(rsrc_t r, uint32_t row, int it, bool pairs) {
    return q5_0_pair_load(r, pairs ? row : BUF_INVALID, it);
  }
  template <class XT>
  static __device__ __forceinline__ float dot(const Raw& w, uint32_t, const uint8_t* rowp, int it, const XT*,
                                              const XLds& X, bool pairs) {
    if (pairs) return q5_0_pair_dot(w, it, X.xf);
    return rowp ? small_block_item(T_Q5_0, rowp, it, X.xf) : 0.f;
  }
};
struct F32Raw {
  uint4 w[4];
};
template <>
struct Fmt<T_F32> {  // 16 floats per item
  using Raw = F32Raw;
  static constexpr int NC = 0;
  static __device__ __forceinline__ uint32_t chunk(int, int, bool) { return 0u; }
  static __device__ __forceinline__ Raw load(rsrc_t r, uint32_t row, int it, bool) {
    Raw o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o.w[i] = bl128(r, row + 64u * (uint32_t)it + 16u * i);
    return o;
  }
  template <class XT>
  static __device__ __forceinline__ float dot(const Raw& w, uint32_t, const uint8_t*, int it, const XT*,
                                              const XLds& X, bool) {
    const float4* Xp = (const float4*)X.xf + it * 4;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4 b = Xp[i];
      s += __uint_as_float(w.w[i].x) * b.x + __uint_as_float(w.w[i].y) * b.y + __uint_as_float(w.w[i].z) * b.z +
           __uint_as_float(w.w[i].w) * b.w;
    }
    return s;
  }
};

struct F16Raw {
  uint4 w[2];
};
template <>
struct Fmt<T_F16> {  // 16 halves per item (a format the reference does not load)
  using Raw = F16Raw;
  static constexpr int NC = 0;
  static __device__ __forceinline__ uint32_t chunk(int, int, bool) { return 0u; }
  static __device__ __forceinline__ Raw load(rsrc_t r, uint32_t row, int it, bool) {
    Raw o;
    o.w[0] = bl128(r, row + 32u * (uint32_t)it);
    o.w[1] = bl128(r, row + 32u * (uint32_t)it + 16u);
    return o;
  }
  template <class XT>
  static __device__ __forceinline__ float dot(const Raw& w, uint32_t, const uint8_t*, int it, const XT*,
                                              const XLds& X, bool) {
    const float4* Xp = (const float4*)X.xf + it * 4;
    const uint32_t h[8] = {w.w[0].x, w.w[0].y, w.w[0].z, w.w[0].w, w.w[1].x, w.w[1].y, w.w[1].z, w.w[1].w};
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 b = Xp[i];
      s += f16_bits_to_f32(h[2 * i] & 0xFFFFu) * b.x + f16_bits_to_f32(h[2 * i] >> 16) * b.y +
           f16_bits_to_f32(h[2 * i + 1] & 0xFFFFu) * b.z + f16_bits_to_f32(h[2 * i + 1] >> 16) * b.w;
    }
    return s;
  }
};

// Packed argmax key: larger key = larger logit, then smaller index (the
// first maximum wins, generate.rs:69-77).  The reference scans with a
// strict `>` from index 0, so a NaN logit is never taken after index 0
// (every comparison with it is false), and a NaN at index 0 is never
// replaced: NaN ranks below every value elsewhere and above every value at
// index 0.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  if (v != v) return idx == 0 ? ~0ull : (uint64_t)(0xFFFFFFFFu - idx);
  if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal in the reference
  uint32_t u = __float_as_uint(v);
  uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

}  // namespace frn
