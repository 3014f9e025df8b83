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
// blocks only keep 2-byte alignment, which the items repair in registers
// with v_alignbyte_b32, never reading outside the block.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frn {

enum : uint32_t { T_F32 = 0, T_F16 = 1, T_Q5_0 = 6, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };

// ---- cross-lane all-reduce ----------------------------------------------------
// All-reduce over aligned groups of W lanes (W a power of two up to 64):
// DPP moves inside each 16-lane row (quad xor 1, quad xor 2, half-row
// mirror, row mirror -- every lane ends with its group's result, paired as
// in an xor butterfly) and v_readlane across rows.  __shfl_xor compiles to
// ds_bpermute, a round trip through the LDS crossbar per step; a DPP move
// is an operand modifier of the VALU instruction.  Every lane of the wave
// must be active.
template <int CTRL, class T>
__device__ __forceinline__ T dpp_mov(T v) {
  return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <class T>
__device__ __forceinline__ T lane_read(T v, int lane) {
  return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
struct OpAdd {
  template <class T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
template <int W, class T, class Op = OpAdd>
__device__ __forceinline__ T group_reduce(T v, Op op = Op()) {
  static_assert(sizeof(T) == 4 && W >= 1 && W <= 64 && (W & (W - 1)) == 0, "32-bit values, W = 2^k <= 64");
  if constexpr (W >= 2) v = op(v, dpp_mov<0xB1>(v));    // quad_perm [1,0,3,2]
  if constexpr (W >= 4) v = op(v, dpp_mov<0x4E>(v));    // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v = op(v, dpp_mov<0x141>(v));   // row_half_mirror
  if constexpr (W >= 16) v = op(v, dpp_mov<0x140>(v));  // row_mirror
  if constexpr (W >= 32) {
    const T r0 = lane_read(v, 0), r1 = lane_read(v, 16), r2 = lane_read(v, 32), r3 = lane_read(v, 48);
    if constexpr (W == 64)
      v = op(op(r0, r1), op(r2, r3));
    else
      v = (__lane_id() & 32) ? op(r2, r3) : op(r0, r1);
  }
  return v;
}

__host__ __device__ constexpr int blk_elems(uint32_t t) {
  return t == T_Q4_K || t == T_Q6_K ? 256 : (t == T_F32 || t == T_F16 ? 1 : 32);
}
__host__ __device__ constexpr int blk_bytes(uint32_t t) {
  return t == T_Q4_K ? 144 : t == T_Q6_K ? 210 : t == T_Q8_0 ? 34 : t == T_Q5_0 ? 22 : t == T_F16 ? 2 : 4;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }

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
// s8..11 (no byte addressing of registers).  Both forms are computed and
// selected, so a lane-dependent j costs no branch.
__device__ __forceinline__ void q4k_scale_min_regs(uint32_t a, uint32_t b, uint32_t c, int j, uint32_t& sc,
                                                   uint32_t& m) {
  const uint32_t lo = 8u * (j & 3);
  const uint32_t sc_lo = (a >> lo) & 63u, m_lo = (b >> lo) & 63u;
  const uint32_t sc_hi = ((c >> lo) & 0x0Fu) | (((a >> (lo + 6)) & 3u) << 4);
  const uint32_t m_hi = ((c >> (lo + 4)) & 0x0Fu) | (((b >> (lo + 6)) & 3u) << 4);
  sc = j < 4 ? sc_lo : sc_hi;
  m = j < 4 ? m_lo : m_hi;
}
// The scale and min of sub-blocks 2*j64 and 2*j64 + 1 (one Q4_K item's
// pair, both below 4 or both from 4 on) packed as bytes 0 and 1 of sc and
// m: bytes t, t+1 (t = 2*(j64 & 1)) of the 6-bit fields, or of the 4-bit
// fields of s8..11 with the top 2 bits of s0..7 above them.  Every mask
// and shift depends on the lane's j64 only.
__device__ __forceinline__ void q4k_scale_min_pair(uint32_t a, uint32_t b, uint32_t c, int j64, uint32_t& sc,
                                                   uint32_t& m) {
  const uint32_t s = 16u * (uint32_t)(j64 & 1);
  const bool hi = j64 >= 2;
  const uint32_t mask1 = hi ? 0x0F0Fu : 0x3F3Fu, mask2 = hi ? 0xC0C0u : 0u, msh = hi ? 4u : 0u;
  sc = (((hi ? c : a) >> s) & mask1) | (((a >> s) & mask2) >> 2);
  m = (((hi ? c : b) >> (s + msh)) & mask1) | (((b >> s) & mask2) >> 2);
}

// Value i of one block (quant.rs:17-42, 53-63, 93-109, 114-133).
__device__ __forceinline__ float decode_elem(uint32_t t, const uint8_t* b, int i) {
  if (t == T_F16) {  // IEEE half -> single, exact (a format the reference does not load)
    return f16_bits_to_f32(ld_u16(b));
  } else if (t == T_Q8_0) {
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
//   xf[K]     f32 values (rmsnorm applied), used by the f32 items (not
//             written where only K-quant items read the int8 form);
//   4 planes of K/16 records of 16 bytes, one record per 16-value chunk c:
//     plane 0..2: the chunk's digits d0, d1, d2 (signed bytes) with
//                 x ~= s * (d0 + d1/128 + d2/16384) per 32-value chunk,
//                 s = 1/(127/max|x|) through hardware reciprocals
//                 (|error| <= max|x| * 2^-21 -- f32-level);
//     plane 3:    {s / 16384, sum(x), -32*sum(d0), -32*(128*sum(d1) + sum(d2))}
//                 (the digit sums pre-multiplied by Q6_K's -32 offset; 0
//                 where only Q4_K or Q8_0 items read the record).
// Records sit at chunk index swz(c), a permutation that spreads the chunks
// a 16-lane group reads in one instruction over the LDS banks.
// (Only whole groups of 8 chunks are permuted, so the map stays inside the
// first n = K/16 records.)
__device__ __forceinline__ uint32_t swz(uint32_t c, uint32_t n) {
  return c < (n & ~7u) ? c ^ (((c >> 3) & 1u) * 6u) : c;
}

// One staged 16-value chunk as the items use it: digit planes 0..2 and
// the metadata record.
struct XC {
  uint4 a, b, d;
  float4 m;
};

// The f32 form (every launch but the lm_head's): x itself and the sum of
// each 16-value chunk, for the terms that multiply sum(x) (Q4_K's min,
// Q6_K's -32 offset).  One chunk as the items use it:
struct XF {
  float4 v[4];
  float s;
};

// Padded f32 layout (the f32 form, Q4_K/Q6_K items): float4 f of x sits at
// f + f/16 + 4 (f/64), one spare slot after every 4 chunks of 16 values and
// four more after every 16.  The lanes of one LDS cycle read chunks 16b +
// 4j + h (Q4_K: j < 4, h < 2, two consecutive b) or 16k + 8h + 2p + l
// (Q6_K): unpadded, those sit at 4 (resp. 4) distinct 16-byte slots of a
// 256-byte bank row, 8-way (4-way) conflicts; padded, at 16 distinct slots
// (Q4_K) and 2-way at most (Q6_K).  A chunk's 4 float4 stay contiguous.
__host__ __device__ constexpr uint32_t xf_pad4(uint32_t f) { return f + (f >> 4) + 4u * (f >> 6); }
// floats the padded layout of K values occupies (K a multiple of 4)
__host__ __device__ constexpr uint32_t xf_padded_floats(uint32_t K) { return K + K / 8; }

struct XLds {
  const float* xf;     // [K] (PAD: padded as xf_pad4)
  const uint8_t* pl;   // int8 form: 4 planes of K bytes; f32 form: K/16 chunk sums
  uint32_t K;
  template <bool PAD = false>
  __device__ __forceinline__ XF fchunk(uint32_t c) const {
    XF x;
    const uint32_t b = PAD ? xf_pad4(4u * c) : 4u * c;
#pragma unroll
    for (int i = 0; i < 4; ++i) x.v[i] = ((const float4*)xf)[b + i];
    x.s = ((const float*)pl)[c];
    return x;
  }
  __device__ __forceinline__ XC chunk(uint32_t c) const {
    const uint32_t o = 16u * swz(c, K / 16);
    XC x;
    x.a = *(const uint4*)(pl + o);
    x.b = *(const uint4*)(pl + K + o);
    x.d = *(const uint4*)(pl + 2u * K + o);
    x.m = *(const float4*)(pl + 3u * K + o);
    return x;
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
__device__ __forceinline__ float qx16_small(const uint32_t* q, const XC& x) {
  int acc = dot16(q, x.a, 0);
  acc = dot16(q, x.b, acc << 7);
  acc = dot16(q, x.d, acc << 7);
  return (float)acc * x.m.x;
}
// sum((q - 32) * x) over one chunk for Q6_K's 6-bit q (the offset enters
// as the chunk's pre-multiplied digit sums, the accumulators' start
// values); the d0 part and the d1/d2 part are accumulated separately so
// neither overflows int32.
__device__ __forceinline__ float qx16_q6(const uint32_t* q, const XC& x) {
  int hi = dot16(q, x.a, __float_as_int(x.m.z));
  int lo = dot16(q, x.d, (dot16(q, x.b, 0) << 7) + __float_as_int(x.m.w));
  return ((float)hi * 16384.0f + (float)lo) * x.m.x;
}
// sum(q * x) over one chunk for signed 8-bit q (Q8_0).
__device__ __forceinline__ float qx16_s8(const uint32_t* q, const XC& x) {
  int hi = dot16(q, x.a, 0);
  int lo = dot16(q, x.d, dot16(q, x.b, 0) << 7);
  return ((float)hi * 16384.0f + (float)lo) * x.m.x;
}

// ---- GEMV items ---------------------------------------------------------
// Each item is split into load() -- the raw bytes of one 32- or 64-value
// slice of a weight row, fetched with raw buffer loads -- and dot() --
// realign, decode and multiply with the staged activation vector.  Loads
// go through a buffer resource whose range is the weight matrix: an item
// of a row past the end, or past the row's last block, is given an offset
// >= BUF_INVALID, which the hardware range check turns into zeros without
// a memory access.  So every lane issues the same load sequence with no
// branches, and the compiler can keep a whole batch in flight (a predicated
// load, or one whose data is realigned right away, makes it wait on the
// spot).  All zero bytes decode to zero weights (every scale is zero), and
// the chunk index of such an item is clamped, so its dot is exactly 0.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr uint32_t BUF_INVALID = 0x80000000u;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // dword3 0x00020000: raw (untyped, unswizzled) 32-bit data format on gfx9
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bl128(rsrc_t r, uint32_t off) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 bl64(rsrc_t r, uint32_t off) {
  u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t bl32(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t bl16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
// 16 bytes at a 2-byte aligned offset, from the 20 bytes loaded at the
// dword below it: w = dwords [off & ~3, +16), x = the dword after.
__device__ __forceinline__ void realign16(const uint4& w, uint32_t x, uint32_t sh, uint32_t (&o)[4]) {
  o[0] = __builtin_amdgcn_alignbyte(w.y, w.x, sh);
  o[1] = __builtin_amdgcn_alignbyte(w.z, w.y, sh);
  o[2] = __builtin_amdgcn_alignbyte(w.w, w.z, sh);
  o[3] = __builtin_amdgcn_alignbyte(x, w.w, sh);
}

// Q4_K: 8 items per superblock.  Item (k, j), j = 2*j64 + hh, covers the 16
// quant bytes qs[32*j64 + 16*hh .. +16]: low nibbles are values
// 64*j64 + 16*hh + [0,16) of sub-block 2*j64, high nibbles values
// 64*j64 + 32 + 16*hh + [0,16) of sub-block 2*j64+1.  Factorised as
// (d*sc)*sum(q*x) - (dmin*m)*sum(x).  Superblocks are 16-byte aligned.
struct Q4KRaw {
  uint4 hdr, q;
};
__device__ __forceinline__ Q4KRaw q4k_load(rsrc_t r, uint32_t row, int item) {
  const uint32_t sb = row + (uint32_t)(item >> 3) * 144u;
  Q4KRaw o;
  o.hdr = bl128(r, sb);
  o.q = bl128(r, sb + 16u + 16u * (item & 7));
  return o;
}
// staged chunks item `item` reads: low nibbles, high nibbles
__device__ __forceinline__ uint32_t q4k_chunk(int item, int i) {
  const int k = item >> 3, j = item & 7;
  return 16u * k + 4u * (j >> 1) + (j & 1) + 2u * i;
}
__device__ __forceinline__ float q4k_dot(const Q4KRaw& r, int item, const XC& xA, const XC& xB) {
  int j = item & 7, j64 = j >> 1;
  float d = f16_bits_to_f32(r.hdr.x & 0xFFFFu), dmin = f16_bits_to_f32(r.hdr.x >> 16);
  uint32_t sc, m;  // scales[12] live in hdr.y..hdr.w
  q4k_scale_min_pair(r.hdr.y, r.hdr.z, r.hdr.w, j64, sc, m);
  const uint32_t scA = sc & 0xFFu, scB = (sc >> 8) & 0xFFu, mA = m & 0xFFu, mB = (m >> 8) & 0xFFu;
  uint32_t lo[4] = {r.q.x & 0x0F0F0F0Fu, r.q.y & 0x0F0F0F0Fu, r.q.z & 0x0F0F0F0Fu, r.q.w & 0x0F0F0F0Fu};
  uint32_t hi[4] = {(r.q.x >> 4) & 0x0F0F0F0Fu, (r.q.y >> 4) & 0x0F0F0F0Fu, (r.q.z >> 4) & 0x0F0F0F0Fu,
                    (r.q.w >> 4) & 0x0F0F0F0Fu};
  float fA = qx16_small(lo, xA), fB = qx16_small(hi, xB);
  return (d * (float)scA) * fA - (dmin * (float)mA) * xA.m.y + (d * (float)scB) * fB - (dmin * (float)mB) * xB.m.y;
}

// sum over 16 bytes w (4 dwords, byte i of w[k] is value 4k + i) of
// byte * x (v_cvt_f32_ubyte{i} + FMA)
__device__ __forceinline__ float bx16(const uint32_t* w, const XF& x) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    s = fmaf(byte_f(w[k], 0), x.v[k].x, s);
    s = fmaf(byte_f(w[k], 1), x.v[k].y, s);
    s = fmaf(byte_f(w[k], 2), x.v[k].z, s);
    s = fmaf(byte_f(w[k], 3), x.v[k].w, s);
  }
  return s;
}
// the same for signed bytes (exact int8 -> f32)
__device__ __forceinline__ float sx16(const uint32_t* w, const XF& x) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    s = fmaf((float)(int8_t)(w[k] & 0xFFu), x.v[k].x, s);
    s = fmaf((float)(int8_t)((w[k] >> 8) & 0xFFu), x.v[k].y, s);
    s = fmaf((float)(int8_t)((w[k] >> 16) & 0xFFu), x.v[k].z, s);
    s = fmaf((float)(int8_t)(w[k] >> 24), x.v[k].w, s);
  }
  return s;
}
__device__ __forceinline__ float q4k_dot(const Q4KRaw& r, int item, const XF& xA, const XF& xB) {
  int j = item & 7, j64 = j >> 1;
  float d = f16_bits_to_f32(r.hdr.x & 0xFFFFu), dmin = f16_bits_to_f32(r.hdr.x >> 16);
  uint32_t sc, m;
  q4k_scale_min_pair(r.hdr.y, r.hdr.z, r.hdr.w, j64, sc, m);
  const uint32_t scA = sc & 0xFFu, scB = (sc >> 8) & 0xFFu, mA = m & 0xFFu, mB = (m >> 8) & 0xFFu;
  uint32_t lo[4] = {r.q.x & 0x0F0F0F0Fu, r.q.y & 0x0F0F0F0Fu, r.q.z & 0x0F0F0F0Fu, r.q.w & 0x0F0F0F0Fu};
  uint32_t hi[4] = {(r.q.x >> 4) & 0x0F0F0F0Fu, (r.q.y >> 4) & 0x0F0F0F0Fu, (r.q.z >> 4) & 0x0F0F0F0Fu,
                    (r.q.w >> 4) & 0x0F0F0F0Fu};
  const float fA = bx16(lo, xA), fB = bx16(hi, xB);
  return (d * (float)scA) * fA - (dmin * (float)mA) * xA.s + (d * (float)scB) * fB - (dmin * (float)mB) * xB.s;
}

// Q6_K: 8 items per superblock.  Item (k, h, lq, p): half h, value lanes
// l = 16*lq + [0,16), quarter pair p selects k6 in {p, p+2}:
//   k6 = p   -> low nibbles of ql[64h + 32p + l]  with qh bits 2p..2p+1
//   k6 = p+2 -> high nibbles of the same bytes     with qh bits 2p+4..2p+5
// values 128h + 32*k6 + l, sub-scales sc[8h + 2*k6 + lq].  Superblocks
// (210 B) are only 2-byte aligned: ql and qh come as 20 bytes from the
// dword below and are realigned in dot(); the two scale bytes (4 apart)
// come in one 8-byte load from the dword below the first; d by itself.
struct Q6KRaw {
  uint4 ql, qh;
  uint32_t qlx, qhx;
  uint2 sc;
  uint32_t d;
};
__device__ __forceinline__ Q6KRaw q6k_load(rsrc_t r, uint32_t row, int item) {
  int k = item >> 3, rr = item & 7, h = rr >> 2, lq = (rr >> 1) & 1, p = rr & 1;
  const uint32_t sb = row + (uint32_t)k * 210u;
  const uint32_t a = (sb + 64u * h + 32u * p + 16u * lq) & ~3u, b = (sb + 128u + 32u * h + 16u * lq) & ~3u;
  Q6KRaw o;
  o.ql = bl128(r, a);
  o.qlx = bl32(r, a + 16u);
  o.qh = bl128(r, b);
  o.qhx = bl32(r, b + 16u);
  o.sc = bl64(r, (sb + 192u + 8u * h + 2u * p + lq) & ~3u);
  o.d = bl16(r, sb + 208u);
  return o;
}
// staged chunks item `item` reads: quarter p, quarter p + 2
__device__ __forceinline__ uint32_t q6k_chunk(int item, int i) {
  const int k = item >> 3, rr = item & 7, h = rr >> 2, lq = (rr >> 1) & 1, p = rr & 1;
  return 16u * k + 8u * h + 2u * p + lq + 4u * i;
}
// The item's 32 6-bit values as bytes (quarter p in v0, p + 2 in v1) and
// its scale factors d*sc.
__device__ __forceinline__ void q6k_unpack(const Q6KRaw& o, uint32_t row, int item, uint32_t (&v0)[4],
                                           uint32_t (&v1)[4], float& ds0, float& ds1) {
  int k = item >> 3, rr = item & 7, h = rr >> 2, lq = (rr >> 1) & 1, p = rr & 1;
  const uint32_t sb = row + (uint32_t)k * 210u, sh = sb & 3u;
  const uint32_t ss = 8u * ((sb + 192u + 8u * h + 2u * p + lq) & 3u);
  float d = f16_bits_to_f32(o.d & 0xFFFFu);
  ds0 = d * (float)(int8_t)((o.sc.x >> ss) & 0xFFu);
  ds1 = d * (float)(int8_t)((o.sc.y >> ss) & 0xFFu);
  uint32_t lw[4], hw[4];
  realign16(o.ql, o.qlx, sh, lw);
  realign16(o.qh, o.qhx, sh, hw);
  // nibble | 2 high bits << 4: a bit-field insert of the nibbles into the
  // shifted high bits, then the top 2 bits cleared
  const uint32_t sh0 = 2 * p;
  constexpr uint32_t NIB = 0x0F0F0F0Fu;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    v0[w] = ((lw[w] & NIB) | ((hw[w] << (4 - sh0)) & ~NIB)) & 0x3F3F3F3Fu;
    v1[w] = (((lw[w] >> 4) & NIB) | ((hw[w] >> sh0) & ~NIB)) & 0x3F3F3F3Fu;
  }
}
__device__ __forceinline__ float q6k_dot(const Q6KRaw& o, uint32_t row, int item, const XC& x0, const XC& x1) {
  uint32_t v0[4], v1[4];
  float ds0, ds1;
  q6k_unpack(o, row, item, v0, v1, ds0, ds1);
  return ds0 * qx16_q6(v0, x0) + ds1 * qx16_q6(v1, x1);
}
__device__ __forceinline__ float q6k_dot(const Q6KRaw& o, uint32_t row, int item, const XF& x0, const XF& x1) {
  uint32_t v0[4], v1[4];
  float ds0, ds1;
  q6k_unpack(o, row, item, v0, v1, ds0, ds1);
  return ds0 * fmaf(-32.0f, x0.s, bx16(v0, x0)) + ds1 * fmaf(-32.0f, x1.s, bx16(v1, x1));  // (q - 32) . x
}

// Q8_0, rows with an even number of blocks: item = block pair (68 B,
// dword aligned): d0 | 32 q | d1 | 32 q.
struct Q8PairRaw {
  uint4 a, b, c, e;
  uint32_t f;
};
__device__ __forceinline__ Q8PairRaw q8_0_pair_load(rsrc_t r, uint32_t row, int item) {
  const uint32_t o = row + 68u * (uint32_t)item;
  Q8PairRaw v;
  v.a = bl128(r, o);
  v.b = bl128(r, o + 16u);
  v.c = bl128(r, o + 32u);
  v.e = bl128(r, o + 48u);
  v.f = bl32(r, o + 64u);
  return v;
}
__device__ __forceinline__ uint32_t q8_0_pair_chunk(int item, int i) { return 4u * item + i; }
__device__ __forceinline__ float q8_0_pair_dot(const Q8PairRaw& r, const XC (&x)[4]) {
  const uint32_t v[17] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c.x,
                          r.c.y, r.c.z, r.c.w, r.e.x, r.e.y, r.e.z, r.e.w, r.f};
  float d0 = f16_bits_to_f32(v[0] & 0xFFFFu), d1 = f16_bits_to_f32(v[8] >> 16);
  uint32_t q0[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q0[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);  // bytes 2..34
  float b0 = qx16_s8(q0, x[0]) + qx16_s8(q0 + 4, x[1]);
  float b1 = qx16_s8(v + 9, x[2]) + qx16_s8(v + 13, x[3]);  // bytes 36..68
  return d0 * b0 + d1 * b1;
}
__device__ __forceinline__ float q8_0_pair_dot(const Q8PairRaw& r, const XF (&x)[4]) {
  const uint32_t v[17] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c.x,
                          r.c.y, r.c.z, r.c.w, r.e.x, r.e.y, r.e.z, r.e.w, r.f};
  float d0 = f16_bits_to_f32(v[0] & 0xFFFFu), d1 = f16_bits_to_f32(v[8] >> 16);
  uint32_t q0[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q0[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);
  float b0 = sx16(q0, x[0]) + sx16(q0 + 4, x[1]);
  float b1 = sx16(v + 9, x[2]) + sx16(v + 13, x[3]);
  return d0 * b0 + d1 * b1;
}

// Q5_0, rows with an even number of blocks: item = block pair (44 B), on
// the f32 vector.
struct Q5PairRaw {
  uint4 a, b;
  uint2 c;
  uint32_t e;
};
__device__ __forceinline__ Q5PairRaw q5_0_pair_load(rsrc_t r, uint32_t row, int item) {
  const uint32_t o = row + 44u * (uint32_t)item;
  Q5PairRaw v;
  v.a = bl128(r, o);
  v.b = bl128(r, o + 16u);
  v.c = bl64(r, o + 32u);
  v.e = bl32(r, o + 40u);
  return v;
}
__device__ __forceinline__ float q5_0_pair_dot(const Q5PairRaw& r, int item, const float* xs) {
  const uint32_t v[11] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c.x, r.c.y, r.e};
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
// byte loads from the row pointer at dot time.  Correct for any 2-byte
// alignment; only used off the hot path.
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
