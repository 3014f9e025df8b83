// Device-side decoding of GGUF quantized blocks (gfx950).
//
// Block layouts follow furnace src/quant.rs:3-133:
//   Q8_0 34 B / 32 values  : f16 d | 32 x i8              y = d*q
//   Q5_0 22 B / 32 values  : f16 d | u32 qh | 16 B nibbles y = d*(q5 - 16)
//   Q4_K 144 B / 256 values: f16 d | f16 dmin | 12 B 6-bit (sc,m) | 128 B nibbles
//                            y = (d*sc)*q - dmin*m per 32-value sub-block
//   Q6_K 210 B / 256 values: 128 B low nibbles | 64 B 2-bit highs | 16 x i8 sc | f16 d
//                            y = (d*sc)*(q6 - 32) per 16-value sub-block
// Every dequantized value is an exactly representable product of small
// integers and f16 scales, so the element decoders below are bit-exact with
// the CPU path regardless of FMA contraction.
//
// GEMV "items": each lane handles fixed 32- or 64-value slices of a weight
// row whose bytes it loads with 16-byte (or dword-aligned) loads, so that a
// group of lanes reads one contiguous stretch of the row.  Q4_K superblocks
// (144 B) keep 16-byte alignment; Q6_K (210 B), Q8_0 (34 B) and Q5_0 (22 B)
// blocks only keep 2-byte alignment, which load16_at() repairs with
// v_alignbyte_b32 without reading outside the block.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frn {

enum : uint32_t { T_F32 = 0, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

__host__ __device__ constexpr int blk_elems(uint32_t t) {
  return t == T_Q4_K || t == T_Q6_K ? 256 : (t == T_F32 ? 1 : 32);
}
__host__ __device__ constexpr int blk_bytes(uint32_t t) {
  return t == T_Q4_K ? 144 : t == T_Q6_K ? 210 : t == T_Q8_0 ? 34 : t == T_Q5_0 ? 22 : 4;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }
__device__ __forceinline__ uint32_t ld_u8(const uint8_t* p) { return *p; }

// 16 bytes starting at a 2-byte aligned address p, realigned in registers.
// Reads only [p & ~3, p + 18) when p % 4 == 2 and [p, p + 16) otherwise, so
// it never touches bytes outside the 2 bytes before and after the field.
__device__ __forceinline__ uint4 load16_at(const uint8_t* p) {
  uint32_t sh = (uint32_t)((uintptr_t)p & 3u);
  const uint32_t* base = (const uint32_t*)(p - sh);  // pointer arithmetic keeps the global address space
  uint32_t w0 = base[0], w1 = base[1], w2 = base[2], w3 = base[3];
  uint32_t w4 = base[sh ? 4 : 3];
  uint4 r;
  r.x = __builtin_amdgcn_alignbyte(w1, w0, sh);
  r.y = __builtin_amdgcn_alignbyte(w2, w1, sh);
  r.z = __builtin_amdgcn_alignbyte(w3, w2, sh);
  r.w = __builtin_amdgcn_alignbyte(w4, w3, sh);
  return r;
}

// Byte k of w as float; the backend selects v_cvt_f32_ubyte{k}.
__device__ __forceinline__ float byte_f(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }

// ---- bit-exact element decoders (dequant kernels, embedding rows) --------

// quant.rs:78-88 q4k_scale_min
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t* s, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = s[j] & 63u;
    m = s[j + 4] & 63u;
  } else {
    sc = (s[j + 4] & 0x0Fu) | ((uint32_t)(s[j - 4] >> 6) << 4);
    m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
  }
}

// q4k_scale_min on the 12 scale bytes held as three dwords s0..3 | s4..7 |
// s8..11 (no byte addressing of registers).
__device__ __forceinline__ void q4k_scale_min_regs(uint32_t a, uint32_t b, uint32_t c, int j, uint32_t& sc,
                                                   uint32_t& m) {
  if (j < 4) {
    sc = (a >> (8 * j)) & 63u;
    m = (b >> (8 * j)) & 63u;
  } else {
    int jj = 8 * (j - 4);
    sc = ((c >> jj) & 0x0Fu) | (((a >> (jj + 6)) & 3u) << 4);
    m = ((c >> (jj + 4)) & 0x0Fu) | (((b >> (jj + 6)) & 3u) << 4);
  }
}

// Value i of one block (quant.rs:17-42, 53-63, 93-109, 114-133).
__device__ __forceinline__ float decode_elem(uint32_t t, const uint8_t* b, int i) {
  if (t == T_Q8_0) {
    return f16_bits_to_f32(ld_u16(b)) * (float)(int8_t)b[2 + i];
  } else if (t == T_Q5_0) {
    float d = f16_bits_to_f32(ld_u16(b));
    uint32_t qh = b[2] | (b[3] << 8) | (b[4] << 16) | ((uint32_t)b[5] << 24);
    int j = i & 15;
    uint32_t nib = i < 16 ? (b[6 + j] & 0x0Fu) : (uint32_t)(b[6 + j] >> 4);
    uint32_t hi = ((qh >> i) & 1u) << 4;
    return d * (float)((int32_t)(nib | hi) - 16);
  } else if (t == T_Q4_K) {
    float d = f16_bits_to_f32(ld_u16(b)), dmin = f16_bits_to_f32(ld_u16(b + 2));
    int j64 = i >> 6, l = i & 31, hi = (i >> 5) & 1;
    uint32_t sc, m;
    q4k_scale_min(2 * j64 + hi, b + 4, sc, m);
    uint8_t q = b[16 + 32 * j64 + l];
    uint32_t nib = hi ? (uint32_t)(q >> 4) : (uint32_t)(q & 0x0F);
    float dd = d * (float)sc, mm = dmin * (float)m;
    return dd * (float)nib - mm;
  } else if (t == T_Q6_K) {
    float d = f16_bits_to_f32(ld_u16(b + 208));
    int half = i >> 7, r = i & 127, k = r >> 5, l = r & 31;
    const uint8_t* ql = b + 64 * half;
    uint32_t qh = b[128 + 32 * half + l];
    uint32_t lo = (k & 1) ? ql[l + 32] : ql[l];
    lo = (k & 2) ? (lo >> 4) : (lo & 0x0Fu);
    int32_t q = (int32_t)(lo | (((qh >> (2 * k)) & 3u) << 4)) - 32;
    int8_t sc = (int8_t)b[192 + 8 * half + (l >> 4) + 2 * k];
    return d * (float)sc * (float)q;
  }
  return 0.f;
}

// ---- activation vector in LDS ----------------------------------------------
// A GEMV block stages its input vector once:
//   xf[K]     f32 values (rmsnorm applied), used by the f32 items;
//   4 planes of K/16 records of 16 bytes, one record per 16-value chunk c:
//     plane 0..2: the chunk's digits d0, d1, d2 (signed bytes) with
//                 x ~= s * (d0 + d1/128 + d2/16384) per 32-value chunk
//                 (|error| <= max|x| * 2^-22 -- f32-level);
//     plane 3:    {s / 16384, sum(x), sum(d0), 128*sum(d1) + sum(d2)}.
// Records sit at chunk index swz(c), a permutation that spreads the chunks
// a 16-lane group reads in one instruction over the LDS banks.
// (Only whole groups of 8 chunks are permuted, so the map stays inside the
// first n = K/16 records.)
__device__ __forceinline__ uint32_t swz(uint32_t c, uint32_t n) {
  return c < (n & ~7u) ? c ^ (((c >> 3) & 1u) * 6u) : c;
}

struct XLds {
  const float* xf;     // [K]
  const uint8_t* pl;   // 4 planes of K bytes
  uint32_t K;
  __device__ __forceinline__ uint4 digits(uint32_t plane, uint32_t c) const {
    return *(const uint4*)(pl + (size_t)plane * K + 16u * swz(c, K / 16));
  }
  __device__ __forceinline__ float4 meta(uint32_t c) const {
    return *(const float4*)(pl + 3u * (size_t)K + 16u * swz(c, K / 16));
  }
};

// sum over 16 bytes of q * digit, for one digit plane
__device__ __forceinline__ int dot16(const uint32_t* q, uint4 d, int acc) {
  acc = __builtin_amdgcn_sdot4((int)q[0], (int)d.x, acc, false);
  acc = __builtin_amdgcn_sdot4((int)q[1], (int)d.y, acc, false);
  acc = __builtin_amdgcn_sdot4((int)q[2], (int)d.z, acc, false);
  acc = __builtin_amdgcn_sdot4((int)q[3], (int)d.w, acc, false);
  return acc;
}
// sum(q * x) over one 16-value chunk for small non-negative q (Q4_K: q < 16,
// so 16 * 15 * 127 * 2^14 fits int32): one chain, scaled by the chunk scale.
__device__ __forceinline__ float qx16_small(const uint32_t* q, const XLds& X, uint32_t c, float4& m) {
  uint4 a = X.digits(0, c), b = X.digits(1, c), d = X.digits(2, c);
  m = X.meta(c);
  int acc = dot16(q, a, 0);
  acc = dot16(q, b, acc << 7);
  acc = dot16(q, d, acc << 7);
  return (float)acc * m.x;
}
// sum((q - bias) * x) over one chunk for 8-bit q: the d0 part and the
// d1/d2 part are accumulated separately so neither overflows int32.
__device__ __forceinline__ float qx16_wide(const uint32_t* q, const XLds& X, uint32_t c, int bias) {
  uint4 a = X.digits(0, c), b = X.digits(1, c), d = X.digits(2, c);
  float4 m = X.meta(c);
  int hi = dot16(q, a, 0) - bias * __float_as_int(m.z);
  int lo = dot16(q, d, dot16(q, b, 0) << 7) - bias * __float_as_int(m.w);
  return ((float)hi * 16384.0f + (float)lo) * m.x;
}

// ---- GEMV items ---------------------------------------------------------
// Each item is split into load() -- the raw bytes of one 32- or 64-value
// slice of a weight row, fetched into registers -- and dot() -- decode and
// multiply with the staged activation vector -- so a lane can issue the
// loads of several items before waiting on any of them.

// Q4_K: 8 items per superblock.  Item (k, j), j = 2*j64 + hh, covers the 16
// quant bytes qs[32*j64 + 16*hh .. +16]: low nibbles are values
// 64*j64 + 16*hh + [0,16) of sub-block 2*j64, high nibbles values
// 64*j64 + 32 + 16*hh + [0,16) of sub-block 2*j64+1.  Factorised as
// (d*sc)*sum(q*x) - (dmin*m)*sum(x).
struct Q4KRaw {
  uint4 hdr, q;
};
__device__ __forceinline__ Q4KRaw q4k_load(const uint8_t* row, int item) {
  const uint8_t* sb = row + (size_t)(item >> 3) * 144;
  Q4KRaw r;
  r.hdr = *(const uint4*)sb;
  r.q = *(const uint4*)(sb + 16 + 16 * (item & 7));
  return r;
}
__device__ __forceinline__ float q4k_dot(const Q4KRaw& r, int item, const XLds& X) {
  int k = item >> 3, j = item & 7, j64 = j >> 1, hh = j & 1;
  float d = f16_bits_to_f32(r.hdr.x & 0xFFFFu), dmin = f16_bits_to_f32(r.hdr.x >> 16);
  uint32_t scA, mA, scB, mB;  // scales[12] live in hdr.y..hdr.w
  q4k_scale_min_regs(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j64, scA, mA);
  q4k_scale_min_regs(r.hdr.y, r.hdr.z, r.hdr.w, 2 * j64 + 1, scB, mB);
  uint32_t lo[4] = {r.q.x & 0x0F0F0F0Fu, r.q.y & 0x0F0F0F0Fu, r.q.z & 0x0F0F0F0Fu, r.q.w & 0x0F0F0F0Fu};
  uint32_t hi[4] = {(r.q.x >> 4) & 0x0F0F0F0Fu, (r.q.y >> 4) & 0x0F0F0F0Fu, (r.q.z >> 4) & 0x0F0F0F0Fu,
                    (r.q.w >> 4) & 0x0F0F0F0Fu};
  uint32_t cA = 16 * k + 4 * j64 + hh, cB = cA + 2;
  float4 mtA, mtB;
  float fA = qx16_small(lo, X, cA, mtA), fB = qx16_small(hi, X, cB, mtB);
  return (d * (float)scA) * fA - (dmin * (float)mA) * mtA.y + (d * (float)scB) * fB - (dmin * (float)mB) * mtB.y;
}

// Q6_K: 8 items per superblock.  Item (k, h, lq, p): half h, value lanes
// l = 16*lq + [0,16), quarter pair p selects k6 in {p, p+2}:
//   k6 = p   -> low nibbles of ql[64h + 32p + l]  with qh bits 2p..2p+1
//   k6 = p+2 -> high nibbles of the same bytes     with qh bits 2p+4..2p+5
// values 128h + 32*k6 + l, sub-scales sc[8h + 2*k6 + lq].
struct Q6KRaw {
  uint4 ql, qh;
  uint32_t d, s0, s1;
};
__device__ __forceinline__ Q6KRaw q6k_load(const uint8_t* row, int item) {
  int k = item >> 3, r = item & 7, h = r >> 2, lq = (r >> 1) & 1, p = r & 1;
  const uint8_t* sb = row + (size_t)k * 210;
  Q6KRaw o;
  o.ql = load16_at(sb + 64 * h + 32 * p + 16 * lq);
  o.qh = load16_at(sb + 128 + 32 * h + 16 * lq);
  o.d = ld_u16(sb + 208);
  o.s0 = ld_u8(sb + 192 + 8 * h + 2 * p + lq);
  o.s1 = ld_u8(sb + 192 + 8 * h + 2 * (p + 2) + lq);
  return o;
}
__device__ __forceinline__ float q6k_dot(const Q6KRaw& o, int item, const XLds& X) {
  int k = item >> 3, r = item & 7, h = r >> 2, lq = (r >> 1) & 1, p = r & 1;
  float d = f16_bits_to_f32(o.d);
  float s0 = (float)(int8_t)o.s0, s1 = (float)(int8_t)o.s1;
  uint32_t lw[4] = {o.ql.x, o.ql.y, o.ql.z, o.ql.w}, hw[4] = {o.qh.x, o.qh.y, o.qh.z, o.qh.w};
  uint32_t v0[4], v1[4];
  const uint32_t sh0 = 2 * p, sh1 = 2 * p + 4;
#pragma unroll
  for (int w = 0; w < 4; ++w) {  // 6-bit values as bytes: nibble | 2 high bits << 4
    v0[w] = (lw[w] & 0x0F0F0F0Fu) | (((hw[w] >> sh0) & 0x03030303u) << 4);
    v1[w] = ((lw[w] >> 4) & 0x0F0F0F0Fu) | (((hw[w] >> sh1) & 0x03030303u) << 4);
  }
  uint32_t c0 = 16 * k + 8 * h + 2 * p + lq, c1 = c0 + 4;
  return (d * s0) * qx16_wide(v0, X, c0, 32) + (d * s1) * qx16_wide(v1, X, c1, 32);
}

// Q8_0, rows with an even number of blocks: item = block pair (68 B,
// dword aligned): d0 | 32 q | d1 | 32 q.
struct Q8PairRaw {
  uint32_t v[17];
};
__device__ __forceinline__ Q8PairRaw q8_0_pair_load(const uint8_t* row, int item) {
  const uint32_t* w = (const uint32_t*)(row + (size_t)item * 68);
  Q8PairRaw r;
#pragma unroll
  for (int i = 0; i < 17; ++i) r.v[i] = w[i];
  return r;
}
__device__ __forceinline__ float q8_0_pair_dot(const Q8PairRaw& r, int item, const XLds& X) {
  const uint32_t* v = r.v;
  float d0 = f16_bits_to_f32(v[0] & 0xFFFFu), d1 = f16_bits_to_f32(v[8] >> 16);
  uint32_t q0[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q0[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);  // bytes 2..34
  uint32_t c = 4 * item;
  float b0 = qx16_wide(q0, X, c, 0) + qx16_wide(q0 + 4, X, c + 1, 0);
  float b1 = qx16_wide(v + 9, X, c + 2, 0) + qx16_wide(v + 13, X, c + 3, 0);  // bytes 36..68
  return d0 * b0 + d1 * b1;
}

// Q5_0, rows with an even number of blocks: item = block pair (44 B), on
// the f32 vector.
struct Q5PairRaw {
  uint32_t v[11];
};
__device__ __forceinline__ Q5PairRaw q5_0_pair_load(const uint8_t* row, int item) {
  const uint32_t* w = (const uint32_t*)(row + (size_t)item * 44);
  Q5PairRaw r;
#pragma unroll
  for (int i = 0; i < 11; ++i) r.v[i] = w[i];
  return r;
}
__device__ __forceinline__ float q5_0_pair_dot(const Q5PairRaw& r, int item, const float* xs) {
  const uint32_t* v = r.v;
  // block 0: d0 = bytes 0..2, qh0 = bytes 2..6, qs0 = bytes 6..22
  // block 1: d1 = bytes 22..24, qh1 = bytes 24..28, qs1 = bytes 28..44
  float d0 = f16_bits_to_f32(v[0] & 0xFFFFu), d1 = f16_bits_to_f32(v[5] >> 16);
  uint32_t qh0 = __builtin_amdgcn_alignbyte(v[1], v[0], 2), qh1 = v[6];
  uint32_t qs0[4], qs1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qs0[i] = __builtin_amdgcn_alignbyte(v[2 + i], v[1 + i], 2);
    qs1[i] = v[7 + i];
  }
  const float* Xp = xs + 64 * item;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    uint32_t b0 = (qs0[j >> 2] >> (8 * (j & 3))) & 0xFFu, b1 = (qs1[j >> 2] >> (8 * (j & 3))) & 0xFFu;
    float a0 = (float)((int32_t)((b0 & 0x0Fu) | (((qh0 >> j) & 1u) << 4)) - 16);
    float a1 = (float)((int32_t)((b0 >> 4) | (((qh0 >> (j + 16)) & 1u) << 4)) - 16);
    float c0 = (float)((int32_t)((b1 & 0x0Fu) | (((qh1 >> j) & 1u) << 4)) - 16);
    float c1 = (float)((int32_t)((b1 >> 4) | (((qh1 >> (j + 16)) & 1u) << 4)) - 16);
    s0 += a0 * Xp[j] + a1 * Xp[16 + j];
    s1 += c0 * Xp[32 + j] + c1 * Xp[48 + j];
  }
  return d0 * s0 + d1 * s1;
}

// Odd block counts (Q8_0/Q5_0 rows of 32*odd values): one block per item,
// byte loads.  Correct for any 2-byte alignment; only used off the hot path.
__device__ __forceinline__ float small_block_item(uint32_t t, const uint8_t* row, int item, const float* xs) {
  const uint8_t* b = row + (size_t)item * blk_bytes(t);
  float d = f16_bits_to_f32(ld_u16(b));
  const float* X = xs + 32 * item;
  float s = 0.f;
  if (t == T_Q8_0) {
    for (int i = 0; i < 32; ++i) s += (float)(int8_t)b[2 + i] * X[i];
  } else {
    uint32_t qh = b[2] | (b[3] << 8) | (b[4] << 16) | ((uint32_t)b[5] << 24);
    for (int j = 0; j < 16; ++j) {
      s += (float)((int32_t)((b[6 + j] & 0x0Fu) | (((qh >> j) & 1u) << 4)) - 16) * X[j];
      s += (float)((int32_t)((uint32_t)(b[6 + j] >> 4) | (((qh >> (j + 16)) & 1u) << 4)) - 16) * X[16 + j];
    }
  }
  return d * s;
}

}  // namespace frn
