// gfx950 kernels of the prefill: the prompt's tokens processed as a block
// of rows per layer (Model::forward_cached with seq > 1, model.rs:579-592,
// layer_forward_cached model.rs:444-478).
//
//  - k_embed_rows     embedding rows of the block's token ids
//  - k_rows_split     rows of x, rmsnorm'd when a gain is given, split into
//                     the bf16 planes x = hi + lo the GEMMs read
//  - k_group_sums     sums of the 32-value groups of split rows (the Q4_K
//                     GEMMs' offset term)
//  - k_gemm_b3        C = A . W^T with W in its raw GGUF blocks: each wave
//                     decodes its weight rows straight into MFMA operands.
//                     Q4_K: the exact quants as bf16, two
//                     v_mfma_f32_32x32x16_bf16 per operand pair (q.x_hi,
//                     q.x_lo) into a per-group product scaled by d sc, and
//                     the groups' -dmin m offsets applied per 16 groups with
//                     the group sums; the other formats: the dequantized
//                     weight (f32, the dequant kernel's formulas with fused
//                     products) split into bf16 hi + lo, three MFMAs per
//                     pair (hi.hi, hi.lo, lo.hi).  Epilogues: store + bias,
//                     residual add, SwiGLU of two weights into split planes
//  - k_rope_kv_rows   RoPE of q and k rows at their positions, KV append
//  - k_kv_split       a layer's K and V as bf16 hi + lo planes (V transposed)
//  - k_attn_rows_mfma causal GQA attention of 128 query rows of one head per
//                     block (one wave per 32 rows) over the cache, key tiles
//                     shared through LDS, on split-operand
//                     v_mfma_f32_32x32x16_bf16 (S^T = K Q^T, then
//                     O^T += V^T P^T), online softmax over 32-key tiles
//
// The split products carry 16+ significant bits per operand into f32
// accumulators (Q4_K quants exactly): the GEMM differs from the CPU path by
// the order of its sums and a relative error below ~2^-15 per product.
#include <stdlib.h>

#include <algorithm>

#include <type_traits>

#include "formats.hpp"
#include "kernels.hpp"

namespace frn {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---- embedding rows (model.rs:482-506) ----------------------------------------------
__global__ void k_embed_rows(const uint8_t* __restrict__ table, uint32_t type, uint32_t hidden, uint32_t row_bytes,
                             const uint32_t* __restrict__ ids, float* __restrict__ x) {
  const uint32_t r = blockIdx.y;
  const uint8_t* row = table + (size_t)ids[r] * row_bytes;
  const int be = blk_elems(type), bb = blk_bytes(type);
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
    x[(size_t)r * hidden + i] =
        type == T_F32 ? ((const float*)row)[i] : decode_elem(type, row + (size_t)(i / be) * bb, (int)(i % be));
}

hipError_t launch_embed_rows(const uint8_t* table, uint32_t type, uint32_t hidden, uint32_t row_bytes,
                             const uint32_t* ids, uint32_t n, float* x, hipStream_t s) {
  hipLaunchKernelGGL(k_embed_rows, dim3((hidden + 255) / 256, n), dim3(256), 0, s, table, type, hidden, row_bytes, ids,
                     x);
  return hipGetLastError();
}

// ---- bf16 split of operands ---------------------------------------------------------
// x = hi + lo + e with hi = bf16(x) (to nearest even), lo = bf16(x - hi),
// |e| <= 2^-16 |x| (bf16 keeps 8 significant bits).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// two values to a bf16 pair (value a in the low half), one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}
// a pair of values -> the pair of their bf16 hi and the pair of their lo
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pk_bf16(a, b);
  lo = pk_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}
// 8 values -> 8 bf16 hi and 8 bf16 lo, value i in half i%2 of dword i/2
// (the order of the MFMA operands)
__device__ __forceinline__ void split8(const float (&y)[8], uint4& hi, uint4& lo) {
  split2(y[0], y[1], hi.x, lo.x);
  split2(y[2], y[3], hi.y, lo.y);
  split2(y[4], y[5], hi.z, lo.z);
  split2(y[6], y[7], hi.w, lo.w);
}
__device__ __forceinline__ void split1(float y, uint16_t& hi, uint16_t& lo) {
  uint32_t h, l;
  split2(y, 0.0f, h, l);
  hi = (uint16_t)h;
  lo = (uint16_t)l;
}

// One block per row: the rmsnorm factor 1/sqrt(mean(x^2) + eps) when nw is
// given (tensor.rs:164-185: (x * inv) * w), then the split.  cols % 8 == 0.
// With xh given (cols % 32 == 0), also the sums of the row's 32-value
// groups of hi + lo, as launch_group_sums writes them (the four threads of
// a group add their 8 values in order, then pairwise).
__global__ __launch_bounds__(256) void k_rows_split(const float* __restrict__ x, uint32_t cols,
                                                    const float* __restrict__ nw, float eps, uint16_t* __restrict__ hi,
                                                    uint16_t* __restrict__ lo, uint16_t* __restrict__ xh,
                                                    uint16_t* __restrict__ xl) {
  __shared__ float red[4];
  const float* row = x + (size_t)blockIdx.x * cols;
  float inv = 1.0f;
  if (nw) {
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < cols; i += 256) ss += row[i] * row[i];
    ss = group_reduce<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)cols + eps);
  }
  for (uint32_t i = 8 * threadIdx.x; i < cols; i += 8 * 256) {
    const float4 a = *(const float4*)(row + i), b = *(const float4*)(row + i + 4);
    float y[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (nw) {
      const float4 wa = *(const float4*)(nw + i), wb = *(const float4*)(nw + i + 4);
      const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = y[j] * inv * w[j];
    }
    uint4 h, l;
    split8(y, h, l);
    *(uint4*)(hi + (size_t)blockIdx.x * cols + i) = h;
    *(uint4*)(lo + (size_t)blockIdx.x * cols + i) = l;
    if (xh) {  // cols % 32 == 0: the four threads of a group are in this pass together
      const uint32_t wh[4] = {h.x, h.y, h.z, h.w}, wl[4] = {l.x, l.y, l.z, l.w};
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        part += __uint_as_float(wh[e] << 16) + __uint_as_float(wl[e] << 16);
        part += __uint_as_float(wh[e] & 0xFFFF0000u) + __uint_as_float(wl[e] & 0xFFFF0000u);
      }
      part = group_reduce<4>(part);
      if ((threadIdx.x & 3) == 0) {
        const size_t gi = (size_t)blockIdx.x * (cols / 32) + i / 32;
        split1(part, xh[gi], xl[gi]);
      }
    }
  }
}

hipError_t launch_rows_split(const float* x, uint32_t rows, uint32_t cols, const float* nw, float eps, uint16_t* hi,
                             uint16_t* lo, uint16_t* xh, uint16_t* xl, hipStream_t s) {
  if (cols % 8 || (xh && (cols % 32 || !xl))) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rows_split, dim3(rows), dim3(256), 0, s, x, cols, nw, eps, hi, lo, xh, xl);
  return hipGetLastError();
}

// One thread per 32-value group of a row: the sum of its values hi + lo in
// index order (each hi + lo is exact in f32), split into bf16 hi + lo.
__global__ __launch_bounds__(256) void k_group_sums(const uint16_t* __restrict__ hi, const uint16_t* __restrict__ lo,
                                                    uint32_t cols, uint16_t* __restrict__ xh,
                                                    uint16_t* __restrict__ xl) {
  const uint32_t r = blockIdx.y, ng = cols / 32, gi = blockIdx.x * 256 + threadIdx.x;
  if (gi >= ng) return;
  const uint4* ph = (const uint4*)(hi + (size_t)r * cols + 32 * gi);
  const uint4* pl = (const uint4*)(lo + (size_t)r * cols + 32 * gi);
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint4 a = ph[c], b = pl[c];
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {  // value 2e in the low half, 2e + 1 in the high half
      sum += __uint_as_float(wa[e] << 16) + __uint_as_float(wb[e] << 16);
      sum += __uint_as_float(wa[e] & 0xFFFF0000u) + __uint_as_float(wb[e] & 0xFFFF0000u);
    }
  }
  split1(sum, xh[(size_t)r * ng + gi], xl[(size_t)r * ng + gi]);
}

hipError_t launch_group_sums(const uint16_t* hi, const uint16_t* lo, uint32_t rows, uint32_t cols, uint16_t* xh,
                             uint16_t* xl, hipStream_t s) {
  if (cols % 32 || rows == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_group_sums, dim3((cols / 32 + 255) / 256, rows), dim3(256), 0, s, hi, lo, cols, xh, xl);
  return hipGetLastError();
}

// ---- weight tiles of the GEMM -------------------------------------------------------
// Eight consecutive weights w[n][k .. k + 8) (k % 8 == 0, inside one 32-value
// group) of a row at byte offset `row` (BUF_INVALID: zeros): decode_elem's
// formulas, the scale products fused (d*sc*q - dmin*m as one FMA; within
// 2^-24 of the unfused value, far below the bf16 split that follows).
// Raw bytes are fetched by load(), decoded by decode().
template <uint32_t T>
struct Deq8;

template <>
struct Deq8<T_Q4_K> {  // quant.rs:93-109
  uint4 hdr;
  uint2 q;
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row, uint32_t k) {
    const uint32_t sb = row + (k / 256) * 144, j = (k % 256) / 32, l = k % 32;
    hdr = bl128(r, sb);
    q = bl64(r, sb + 16 + 32 * (j / 2) + l);
  }
  __device__ __forceinline__ void decode(uint32_t k, float (&y)[8]) const {
    const uint32_t j = (k % 256) / 32;
    const float d = f16_bits_to_f32(hdr.x & 0xFFFFu), dmin = f16_bits_to_f32(hdr.x >> 16);
    uint32_t sc, m;
    q4k_scale_min_regs(hdr.y, hdr.z, hdr.w, (int)j, sc, m);
    const float dd = d * (float)sc, mm = dmin * (float)m;
    const uint32_t sh = (j & 1) ? 4 : 0;
    // the 8 nibbles as bytes, then byte -> f32 conversions
    const uint32_t n0 = (q.x >> sh) & 0x0F0F0F0Fu, n1 = (q.y >> sh) & 0x0F0F0F0Fu;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      y[i] = fmaf(dd, byte_f(n0, i), -mm);
      y[4 + i] = fmaf(dd, byte_f(n1, i), -mm);
    }
  }
};

// 8 bytes at a 2-byte aligned offset: 12 bytes from the dword below
__device__ __forceinline__ uint2 load8_at(rsrc_t r, uint32_t off, uint32_t& sh) {
  const uint32_t a = off & ~3u;
  sh = off & 3u;
  const uint2 w = bl64(r, a);
  const uint32_t x = bl32(r, a + 8);
  return make_uint2(__builtin_amdgcn_alignbyte(w.y, w.x, sh), __builtin_amdgcn_alignbyte(x, w.y, sh));
}

template <>
struct Deq8<T_Q6_K> {  // quant.rs:114-133
  uint2 ql, qh;
  uint32_t sc, d;
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row, uint32_t k) {
    const uint32_t sb = row + (k / 256) * 210, idx = k % 256, h = idx / 128, rr = idx % 128, k6 = rr / 32, l = rr % 32;
    uint32_t s1, s2;
    ql = load8_at(r, sb + 64 * h + 32 * (k6 & 1) + l, s1);
    qh = load8_at(r, sb + 128 + 32 * h + l, s2);
    const uint32_t so = sb + 192 + 8 * h + l / 16 + 2 * k6;
    sc = bl32(r, so & ~3u) >> (8 * (so & 3u));
    d = bl16(r, sb + 208);
  }
  __device__ __forceinline__ void decode(uint32_t k, float (&y)[8]) const {
    const uint32_t idx = k % 256, k6 = (idx % 128) / 32;
    const float dsc = f16_bits_to_f32(d & 0xFFFFu) * (float)(int8_t)(sc & 0xFFu);
    const uint32_t lsh = (k6 & 2) ? 4 : 0, hsh = 2 * k6;
    // the 8 6-bit values as bytes (low nibble | 2 high bits << 4), then
    // byte -> f32 and (v - 32) * d*sc as one FMA
    const uint32_t v0 = ((ql.x >> lsh) & 0x0F0F0F0Fu) | (((qh.x >> hsh) & 0x03030303u) << 4);
    const uint32_t v1 = ((ql.y >> lsh) & 0x0F0F0F0Fu) | (((qh.y >> hsh) & 0x03030303u) << 4);
    const float off = -32.0f * dsc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      y[i] = fmaf(dsc, byte_f(v0, i), off);
      y[4 + i] = fmaf(dsc, byte_f(v1, i), off);
    }
  }
};

template <>
struct Deq8<T_Q8_0> {  // quant.rs:17-42
  uint2 q;
  uint32_t d;
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row, uint32_t k) {
    const uint32_t b = row + (k / 32) * 34;
    uint32_t s;
    q = load8_at(r, b + 2 + k % 32, s);
    d = bl16(r, b);
  }
  __device__ __forceinline__ void decode(uint32_t, float (&y)[8]) const {
    const float dd = f16_bits_to_f32(d & 0xFFFFu);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = dd * (float)(int8_t)(((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu);
  }
};

template <>
struct Deq8<T_Q5_0> {  // quant.rs:53-63: the whole 22-byte block, from the dword below
  uint4 a;
  uint2 b;
  uint32_t sh;
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row, uint32_t k) {
    const uint32_t off = row + (k / 32) * 22;
    const uint32_t al = off & ~3u;
    sh = off & 3u;
    a = bl128(r, al);
    b = bl64(r, al + 16);
  }
  __device__ __forceinline__ void decode(uint32_t k, float (&y)[8]) const {
    const uint32_t w[6] = {a.x, a.y, a.z, a.w, b.x, b.y};
    uint32_t v[6];  // the block's bytes 0..23 realigned
#pragma unroll
    for (int i = 0; i < 5; ++i) v[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
    v[5] = __builtin_amdgcn_alignbyte(0u, w[5], sh);
    const float d = f16_bits_to_f32(v[0] & 0xFFFFu);
    const uint32_t qh = __builtin_amdgcn_alignbyte(v[1], v[0], 2);
    const uint32_t j0 = k % 32;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t j = j0 + i, jj = j & 15, byte_i = 6 + jj;  // qs[jj] is block byte 6 + jj
      const uint32_t byte = (v[byte_i / 4] >> (8 * (byte_i % 4))) & 0xFFu;
      const uint32_t nib = j < 16 ? (byte & 0x0Fu) : (byte >> 4);
      const uint32_t hi = ((qh >> j) & 1u) << 4;
      y[i] = d * (float)((int32_t)(nib | hi) - 16);
    }
  }
};

template <>
struct Deq8<T_F16> {  // a format the reference does not load
  uint4 a;
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row, uint32_t k) { a = bl128(r, row + 2 * k); }
  __device__ __forceinline__ void decode(uint32_t, float (&y)[8]) const {
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      y[2 * i] = f16_bits_to_f32(w[i] & 0xFFFFu);
      y[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
};

template <>
struct Deq8<T_F32> {
  uint4 a, b;
  __device__ __forceinline__ void load(rsrc_t r, uint32_t row, uint32_t k) {
    a = bl128(r, row + 4 * k);
    b = bl128(r, row + 4 * k + 16);
  }
  __device__ __forceinline__ void decode(uint32_t, float (&y)[8]) const {
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = __uint_as_float(w[i]);
  }
};

// ---- the GEMM ---------------------------------------------------------------------
// Block tile: (32 MT tokens) x (4 waves x 32 NJ weight rows) per weight
// matrix, k-steps of 32.  The A planes of a k-step go through LDS (shared
// by the 4 waves; double buffer, one barrier per k-step); each wave loads,
// decodes and splits its own weight rows straight into MFMA operands, so
// no weight value is decoded twice and the LDS carries only A (and, for
// Q4_K, each wave's window of group offsets).  Per k-step a wave runs
// 2 x MT x NW x NJ x 3 v_mfma_f32_32x32x16_bf16 (hi.hi, hi.lo, lo.hi; the
// lo.lo term is below 2^-14 of the product), Q4_K 2 x MT x NW x NJ x 2
// (+ 3 per 16 k-steps for the offsets).  Lane l supplies
// A[l%32][8(l/32) .. +8] and B[8(l/32) .. +8][l%32]; register v of lane l
// is C[8(v/4) + 4(l/32) + v%4][l%32] (layouts checked on gfx950).  The raw
// weight bytes of k-step t + 2 and the A planes of k-step t + 1 are in
// flight while k-step t computes.  LDS rows of 32 bf16 are padded to 40
// (80 bytes: the 16-byte reads of 16 consecutive rows hit distinct banks).
constexpr int BKP = 56;
template <int MT>
__host__ __device__ constexpr uint32_t gemm_lds_bytes() {
  return 2u * 2u * 32u * MT * BKP * 2u;  // 2 buffers x 2 planes x rows x padded row
}
// Q4_K: + each wave's window of group offsets, [32 rows][16 groups] f32
// per weight tile
template <uint32_t T, int MODE, int MT, int NJ>
__host__ __device__ constexpr uint32_t gemm_lds_bytes_t() {
  return gemm_lds_bytes<MT>() + (T == T_Q4_K ? 4u * (MODE == GEMM_SWIGLU ? 2u : 1u) * NJ * 512u * 4u : 0u);
}

// the output columns of a launch: segment 0's and the more[] segments'
__host__ __device__ inline uint32_t gemm_cols(const GemmArgs& g) {
  uint32_t n = g.N;
  for (uint32_t i = 0; i < g.n_more; ++i) n += g.more[i].N;
  return n;
}

template <uint32_t T, int MODE, int MT, int NJ>
__global__ __launch_bounds__(256, 2) void k_gemm_b3(GemmArgs g) {
  constexpr int NW = MODE == GEMM_SWIGLU ? 2 : 1, TM = 32 * MT, TN = 4 * 32 * NJ;
  // A loaders: TM rows x 32 values x 2 planes per k-step = TM * 8 uint4;
  // thread t takes rows t / 4 + 64 i (i < (TM + 63) / 64), 16-byte chunk t % 4
  constexpr int AI = (TM + 63) / 64;
  extern __shared__ __attribute__((aligned(16))) uint16_t lds16[];
  constexpr uint32_t A_PL = TM * BKP;
  auto A = [&](int b, int p) { return lds16 + (2 * b + p) * A_PL; };
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, col = lane & 31, kh = 8 * (lane >> 5);
  // the block's weight matrix (segment) and its tile within it
  const uint8_t* sw = g.w;
  const float* sbias = g.bias;
  float* sout = g.out;
  uint32_t sN = g.N, sldo = g.ldo, tile = blockIdx.x, coff = 0;  // coff: the segment's first column of all
  if (MODE == GEMM_STORE) {
    for (uint32_t i = 0; i < g.n_more; ++i) {
      const uint32_t tiles = (sN + TN - 1) / TN;
      if (tile < tiles) break;
      tile -= tiles;
      coff += sN;
      sw = g.more[i].w;
      sbias = g.more[i].bias;
      sout = g.more[i].out;
      sN = g.more[i].N;
      sldo = g.more[i].ldo;
    }
  }
  const uint32_t r0 = blockIdx.y * TM, n0 = tile * TN + wave * 32 * NJ;
  const uint32_t a_bytes = g.P * g.K * 2;
  const rsrc_t rah = make_rsrc(g.a_hi, a_bytes), ral = make_rsrc(g.a_lo, a_bytes);
  const rsrc_t rw[2] = {make_rsrc(sw, sN * g.row_bytes), make_rsrc(NW == 2 ? g.w2 : sw, sN * g.row_bytes)};
  // the block's k-steps: all of K, or chunk z of a split K (a multiple of 8
  // k-steps, so superblocks stay whole; the offsets' windows start at k0)
  const uint32_t nk_all = g.K / 32, k0 = g.ksplit > 1 ? blockIdx.z * g.kchunk : 0;
  const uint32_t nk = g.ksplit > 1 ? min(g.kchunk, nk_all - k0) : nk_all;
  uint32_t a_off[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const uint32_t r = t / 4 + 64 * i;
    a_off[i] = r < TM && r0 + r < g.P ? 2 * ((r0 + r) * g.K + 32 * k0 + 8 * (t % 4)) : BUF_INVALID;
  }
  // this lane's weight rows: n0 + 32 j + col
  uint32_t w_off[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    w_off[j] = n0 + 32 * j + col < sN
                   ? (n0 + 32 * j + col) * g.row_bytes + (32 * k0 / (uint32_t)blk_elems(T)) * (uint32_t)blk_bytes(T)
                   : BUF_INVALID;

  // raw data of two k-steps in flight: A planes [set][i], weights [set][w][j][ks]
  uint4 pah[2][AI], pal[2][AI];  // (one set used when ASETS == 1)
  Deq8<T> pw[2][NW][NJ][2];
  f32x16 acc[MT][NW][NJ];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][w][j][v] = 0.f;

  // Q4_K: per pair of k-steps (one 32-byte group of quants, sub-blocks 2G
  // and 2G + 1 in its low and high nibbles) lane (row, half h) loads the
  // group's bytes 16h .. 16h + 16 and the superblock header: two 16-byte
  // loads per two k-steps instead of four 8- and 16-byte loads per k-step
  // (the memory pipeline, not the matrix cores, bounds this GEMM).  The
  // k order inside a k-step is permuted to match (MFMA half ks of lane
  // half h takes values 16h + 8ks .. +8, in A as in W).
  constexpr bool QK = T == T_Q4_K;
  uint4 qhdr[2][NW][NJ], qraw[2][NW][NJ];
  // Q4_K splits each 32-value group's dot product as quant.rs:100-106's
  // terms: (d sc) * sum(q x) - (dmin m) * sum(x).  The quants q (0..15)
  // are exact in bf16, so sum(q x) takes two MFMAs per operand pair
  // (q.x_hi, q.x_lo) into a per-group product that is scaled by d sc into
  // the accumulator.  The offsets -dmin m of 16 consecutive groups collect
  // in LDS (the wave's [32 rows][16 groups] f32 window) and are applied as
  // one more k = 16 product with the groups' sums of x (x_hi + x_lo, from
  // launch_group_sums or the row split), split three ways like the other
  // operands.
  float* const mwin0 = (float*)(lds16 + 4 * A_PL);
  auto mwin = [&](int w, int j) { return mwin0 + ((wave * NW + w) * NJ + j) * 512; };
  const rsrc_t rxh = make_rsrc(QK ? g.x_hi : nullptr, QK ? g.P * nk_all * 2 : 0);
  const rsrc_t rxl = make_rsrc(QK ? g.x_lo : nullptr, QK ? g.P * nk_all * 2 : 0);
  // the offsets of window wi (groups 16 wi .. +16; `half`: only the first
  // 8 exist) times the group sums, into the accumulators
  auto offsets = [&](uint32_t wi, bool half) {
    const int h = lane >> 5;
    const bool live = !half || h == 0;
    bf16x8 mh[NW][NJ], ml[NW][NJ];
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float* mp = mwin(w, j) + 16 * col + 8 * h;
        const float4 u = *(const float4*)mp, v = *(const float4*)(mp + 4);
        float y[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = live ? y[e] : 0.f;
        uint4 hi, lo;
        split8(y, hi, lo);
        mh[w][j] = __builtin_bit_cast(bf16x8, hi);
        ml[w][j] = __builtin_bit_cast(bf16x8, lo);
      }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const uint32_t r = r0 + 32 * i + col;
      const uint32_t o = live && r < g.P ? 2 * (r * nk_all + k0 + 16 * wi + 8 * h) : BUF_INVALID;
      const bf16x8 xh = __builtin_bit_cast(bf16x8, bl128(rxh, o)), xl = __builtin_bit_cast(bf16x8, bl128(rxl, o));
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          acc[i][w][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, mh[w][j], acc[i][w][j], 0, 0, 0);
          acc[i][w][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, ml[w][j], acc[i][w][j], 0, 0, 0);
          acc[i][w][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl, mh[w][j], acc[i][w][j], 0, 0, 0);
        }
    }
  };
  auto fetch_wq = [&](int s, uint32_t grp) {
    const uint32_t sb = (grp / 4) * 144u, qo = sb + 16u + 32u * (grp % 4) + (uint32_t)(2 * kh);
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const bool ok = 2 * grp < nk && w_off[j] != BUF_INVALID;
        qhdr[s][w][j] = bl128(rw[w], ok ? w_off[j] + sb : BUF_INVALID);
        qraw[s][w][j] = bl128(rw[w], ok ? w_off[j] + qo : BUF_INVALID);
      }
  };
  // Q6_K: per half superblock (four k-steps, quarters k6 of 32 values) lane
  // (row, half h) loads ql bytes 32p + 16h .. +16 (p = k6 & 1: low
  // nibbles for k6 < 2, high above), qh bytes 16h .. +16 (2 bits per k6),
  // the half's 8 scale bytes and d; 20-byte loads from the dword below,
  // realigned on use (superblocks are 2-byte aligned).  Same permuted k
  // order as Q4_K.
  constexpr bool Q6 = T == T_Q6_K;
  struct Raw20 {
    uint4 a;
    uint32_t x;
  };
  Raw20 q6l[Q6 ? 2 : 1][NW][NJ][2], q6h[Q6 ? 2 : 1][NW][NJ];
  uint4 q6s[Q6 ? 2 : 1][NW][NJ];
  uint32_t q6d[Q6 ? 2 : 1][NW][NJ];
  auto fetch_w6 = [&](int s, uint32_t half) {
    const uint32_t sbo = (half / 2) * 210u, hh = half % 2;
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const bool ok = 4 * half < nk && w_off[j] != BUF_INVALID;
        const uint32_t base = ok ? w_off[j] + sbo : BUF_INVALID, al = base & ~3u;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const uint32_t o = al + 64u * hh + 32u * p + (uint32_t)(2 * kh);
          q6l[s][w][j][p].a = bl128(rw[w], o);
          q6l[s][w][j][p].x = bl32(rw[w], o + 16u);
        }
        const uint32_t oh = al + 128u + 32u * hh + (uint32_t)(2 * kh);
        q6h[s][w][j].a = bl128(rw[w], oh);
        q6h[s][w][j].x = bl32(rw[w], oh + 16u);
        q6s[s][w][j] = bl128(rw[w], al + 192u + 8u * hh);
        q6d[s][w][j] = bl32(rw[w], al + 208u);
      }
  };
  auto fetch_a = [&](int s, uint32_t kt) {
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const uint32_t o = a_off[i] == BUF_INVALID || kt >= nk ? BUF_INVALID : a_off[i] + 64 * kt;
      pah[s][i] = bl128(rah, o);
      pal[s][i] = bl128(ral, o);
    }
  };
  auto put_a = [&](int s, int b) {
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const uint32_t r = t / 4 + 64 * i;
      if (r < TM) {
        *(uint4*)(A(b, 0) + r * BKP + 8 * (t % 4)) = pah[s][i];
        *(uint4*)(A(b, 1) + r * BKP + 8 * (t % 4)) = pal[s][i];
      }
    }
  };
  auto fetch_w = [&](int s, uint32_t kt) {
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          pw[s][w][j][ks].load(rw[w], kt >= nk ? BUF_INVALID : w_off[j], 32 * kt + 16 * ks + kh);
  };

  // k-step kt: LDS buffer kt & 1, weight register set kt & 1.  Two k-steps
  // per trip keep every buffer and set index a constant (a register array
  // indexed at run time would live in scratch memory).
  // One k-step kt (LDS buffer and register sets b = kt & 1): all of its A
  // operands are read from LDS up front (a read just before its MFMA would
  // stall the matrix pipe on the LDS latency), the weight operands of the
  // first half are decoded, then the MFMAs run with the accumulators
  // alternating (independent MFMAs back to back) while the second half's
  // weights are decoded.  Then: weights of k-step kt + 2 into set b, the A
  // planes of k-step kt + 1 (fetched a step earlier) into LDS buffer b ^ 1,
  // and A of k-step kt + 3 into the set they came from, so every load has
  // two k-steps of compute to arrive.
  // SwiGLU's MT 4 tile keeps one set of A registers (fetched a k-step
  // ahead) so that two waves per SIMD still fit; the others keep two
  constexpr int ASETS = NW == 2 && MT == 4 ? 1 : 2;
  // pc: the k-step's position in the loop trip (a constant): LDS buffer
  // pc % 2; Q4_K register set pc / 2 and nibble half pc % 2; Q6_K register
  // set pc / 4 and quarter pc % 4
  auto step = [&](auto pcc, uint32_t kt) {
    constexpr int pc = decltype(pcc)::value, b = pc % 2, S = Q6 ? pc / 4 : pc / 2, H = pc % 2, K6 = pc % 4;
    if constexpr (ASETS == 1) {
      if (kt + 1 < nk) fetch_a(0, kt + 1);
    }
    bf16x8 ah[2][MT], al[2][MT], bh[2][NW][NJ], bl[2][NW][NJ];
    auto read_a = [&](int ks) {
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const uint32_t ko = (QK || Q6) ? 2 * kh + 8 * ks : 16 * ks + kh;
        ah[ks][i] = *(const bf16x8*)(A(b, 0) + (32 * i + col) * BKP + ko);
        al[ks][i] = *(const bf16x8*)(A(b, 1) + (32 * i + col) * BKP + ko);
      }
    };
    // both halves' A operands up front when the registers allow (one
    // weight matrix); with two (SwiGLU) the second half's are read once
    // the first half's MFMAs are issued, so they reuse its registers
    constexpr bool A_EARLY = NW == 1 || MT <= 2;
    if constexpr (!QK) {
      read_a(0);
      if constexpr (A_EARLY) read_a(1);
    }
    auto decode = [&](int ks) {
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          float y[8];
          if constexpr (Q6) {  // quant.rs:114-133, quarter K6 of half (kt / 4) % 2
            const uint32_t sh = (w_off[j] + (kt / 8) * 210u) & 3u;
            uint32_t lo4[4], hi4[4];
            realign16(q6l[S][w][j][K6 & 1].a, q6l[S][w][j][K6 & 1].x, sh, lo4);
            realign16(q6h[S][w][j].a, q6h[S][w][j].x, sh, hi4);
            const uint4 sw = q6s[S][w][j];
            const uint32_t sb = sh + 2 * K6 + (kh >> 3), sd = sb >> 2;  // scale byte of this half lane
            const uint32_t sword = sd == 0 ? sw.x : sd == 1 ? sw.y : sd == 2 ? sw.z : sw.w;
            const float dsc = f16_bits_to_f32(q6d[S][w][j] >> (8 * sh) & 0xFFFFu) *
                              (float)(int8_t)((sword >> (8 * (sb & 3))) & 0xFFu);
            const float off = -32.0f * dsc;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const uint32_t nib = ((K6 & 2) ? lo4[2 * ks + e] >> 4 : lo4[2 * ks + e]) & 0x0F0F0F0Fu;
              const uint32_t v = nib | (((hi4[2 * ks + e] >> (2 * K6)) & 0x03030303u) << 4);
#pragma unroll
              for (int i = 0; i < 4; ++i) y[4 * e + i] = fmaf(dsc, byte_f(v, i), off);
            }
          } else {
            pw[b][w][j][ks].decode(32 * kt + 16 * ks + kh, y);
          }
          uint4 hi, lo;
          split8(y, hi, lo);
          bh[ks][w][j] = __builtin_bit_cast(bf16x8, hi);
          bl[ks][w][j] = __builtin_bit_cast(bf16x8, lo);
        }
    };
    auto mma = [&](int ks) {
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
          for (int i = 0; i < MT; ++i)
            acc[i][w][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[ks][i], bh[ks][w][j], acc[i][w][j], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < MT; ++i)
            acc[i][w][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[ks][i], bl[ks][w][j], acc[i][w][j], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < MT; ++i)
            acc[i][w][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[ks][i], bh[ks][w][j], acc[i][w][j], 0, 0, 0);
        }
    };
    if constexpr (QK) {  // quant.rs:93-109, group kt % 8 of superblock kt / 8
      bf16x8 bq[2][NW][NJ];
      float dsc[NW][NJ];
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const uint4 hd = qhdr[S][w][j], q = qraw[S][w][j];
          uint32_t sc, m;
          q4k_scale_min_regs(hd.y, hd.z, hd.w, (int)(kt % 8), sc, m);
          dsc[w][j] = f16_bits_to_f32(hd.x & 0xFFFFu) * (float)sc;
          mwin(w, j)[16 * col + (kt & 15)] = -(f16_bits_to_f32(hd.x >> 16) * (float)m);
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const uint32_t n0 = ((ks ? q.z : q.x) >> (4 * H)) & 0x0F0F0F0Fu;
            const uint32_t n1 = ((ks ? q.w : q.y) >> (4 * H)) & 0x0F0F0F0Fu;
            const uint4 u = make_uint4(pk_bf16(byte_f(n0, 0), byte_f(n0, 1)), pk_bf16(byte_f(n0, 2), byte_f(n0, 3)),
                                       pk_bf16(byte_f(n1, 0), byte_f(n1, 1)), pk_bf16(byte_f(n1, 2), byte_f(n1, 3)));
            bq[ks][w][j] = __builtin_bit_cast(bf16x8, u);
          }
        }
      // per IC token tiles: the group's products in fresh accumulators
      // (four MFMAs each, the IC x NW x NJ chains interleaved), then scaled
      // into the tiles' accumulators.  The empty asm pins each scaling
      // here, so that only this group's products are live.
      constexpr int IC = NW * NJ == 1 && MT % 2 == 0 ? 2 : 1;
#pragma unroll
      for (int i0 = 0; i0 < MT; i0 += IC) {
        bf16x8 a0h[IC], a0l[IC], a1h[IC], a1l[IC];
#pragma unroll
        for (int c = 0; c < IC; ++c) {
          const uint16_t* ar = A(b, 0) + (32 * (i0 + c) + col) * BKP + 2 * kh;
          const uint16_t* al_ = A(b, 1) + (32 * (i0 + c) + col) * BKP + 2 * kh;
          a0h[c] = *(const bf16x8*)ar;
          a0l[c] = *(const bf16x8*)al_;
          a1h[c] = *(const bf16x8*)(ar + 8);
          a1l[c] = *(const bf16x8*)(al_ + 8);
        }
#pragma unroll
        for (int c = 0; c < IC; ++c)
#pragma unroll
          for (int w = 0; w < NW; ++w)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              f32x16 t = {};
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0h[c], bq[0][w][j], t, 0, 0, 0);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0l[c], bq[0][w][j], t, 0, 0, 0);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1h[c], bq[1][w][j], t, 0, 0, 0);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1l[c], bq[1][w][j], t, 0, 0, 0);
#pragma unroll
              for (int v = 0; v < 16; ++v) acc[i0 + c][w][j][v] = fmaf(dsc[w][j], t[v], acc[i0 + c][w][j][v]);
              asm volatile("" : "+v"(acc[i0 + c][w][j]));
            }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      decode(0);
      __builtin_amdgcn_sched_barrier(0);
      mma(0);
      if constexpr (!A_EARLY) {
        __builtin_amdgcn_sched_barrier(0);
        read_a(1);
      }
      decode(1);
      mma(1);
    }
    // weights two k-steps (Q4_K: two groups) ahead; past the end: no memory access
    if constexpr (QK) {
      if (H == 1) fetch_wq(S, (kt + 3) / 2);
    } else if constexpr (Q6) {
      if (K6 == 3) fetch_w6(S, kt / 4 + 2);
    } else {
      fetch_w(b, kt + 2);
    }
    if (kt + 1 < nk) {
      if constexpr (ASETS == 1) {
        put_a(0, b ^ 1);
      } else {
        put_a(b ^ 1, b ^ 1);
        fetch_a(b ^ 1, kt + 3);
      }
    }
    __syncthreads();
    // a full window of offsets (written before the barrier above)
    if constexpr (QK && pc == 3) {
      if ((kt & 15) == 15) offsets(kt / 16, false);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  fetch_a(0, 0);
  if constexpr (ASETS == 2) fetch_a(1, 1);
  if constexpr (QK) {
    fetch_wq(0, 0);
    fetch_wq(1, 1);
  } else if constexpr (Q6) {
    fetch_w6(0, 0);
    fetch_w6(1, 1);
  } else {
    fetch_w(0, 0);
    fetch_w(1, 1);
  }
  put_a(0, 0);
  if constexpr (ASETS == 2) fetch_a(0, 2);
  __syncthreads();
  if constexpr (QK) {
    // four k-steps (two groups) per trip; K-quant rows hold a multiple of
    // 256 values, so nk % 8 == 0
    for (uint32_t kt = 0; kt < nk; kt += 4) {
      step(I0{}, kt);
      step(I1{}, kt + 1);
      step(std::integral_constant<int, 2>{}, kt + 2);
      step(std::integral_constant<int, 3>{}, kt + 3);
    }
    if (nk & 15) offsets(nk / 16, true);  // a row of 16 w + 8 groups
  } else if constexpr (Q6) {
    // eight k-steps (a superblock: its two halves) per trip
    for (uint32_t kt = 0; kt < nk; kt += 8) {
      step(std::integral_constant<int, 0>{}, kt);
      step(std::integral_constant<int, 1>{}, kt + 1);
      step(std::integral_constant<int, 2>{}, kt + 2);
      step(std::integral_constant<int, 3>{}, kt + 3);
      step(std::integral_constant<int, 4>{}, kt + 4);
      step(std::integral_constant<int, 5>{}, kt + 5);
      step(std::integral_constant<int, 6>{}, kt + 6);
      step(std::integral_constant<int, 7>{}, kt + 7);
    }
  } else {
    for (uint32_t kt = 0; kt < nk; kt += 2) {
      step(I0{}, kt);
      if (kt + 1 < nk) step(I1{}, kt + 1);
    }
  }
  // epilogue: register v of lane l is C[8(v/4) + 4(l/32) + v%4][l%32]
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t n = n0 + 32 * j + col;
    if (n >= sN) continue;
    const float bias = (MODE == GEMM_STORE && sbias) ? sbias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t r = r0 + 32 * i + 8 * (v / 4) + 4 * (lane >> 5) + (v & 3);
        if (r >= g.P) continue;
        const size_t o = (size_t)r * sldo + n;
        if (MODE == GEMM_STORE) {
          if (g.ksplit > 1)  // [z][P][all segments' columns]
            g.partial[((size_t)blockIdx.z * g.P + r) * gemm_cols(g) + coff + n] = acc[i][0][j][v];
          else
            sout[o] = sbias ? acc[i][0][j][v] + bias : acc[i][0][j][v];  // model.rs:179-183
        }
        if (MODE == GEMM_RESID) {
          if (g.ksplit > 1)
            g.partial[((size_t)blockIdx.z * g.P + r) * sN + n] = acc[i][0][j][v];
          else
            sout[o] = sout[o] + acc[i][0][j][v];  // tensor.rs:232
        }
        if (MODE == GEMM_SWIGLU) {
          if (g.ksplit > 1) {  // the two products' partials, [z][2][P][N]
            float* pz = g.partial + (size_t)blockIdx.z * 2 * g.P * sN + (size_t)r * sN + n;
            pz[0] = acc[i][0][j][v];
            pz[(size_t)g.P * sN] = acc[i][NW - 1][j][v];
          } else {  // tensor.rs:224
            const float gg = acc[i][0][j][v];
            split1(gg / (1.0f + expf(-gg)) * acc[i][NW - 1][j][v], g.o_hi[o], g.o_lo[o]);
          }
        }
      }
  }
}

template <int MODE, int MT, int NJ>
static hipError_t gemm_go_types(const GemmArgs& g, dim3 grid, uint32_t lds, hipStream_t s);

template <int MODE, int MT, int NJ>
static hipError_t gemm_go_b3(const GemmArgs& g, hipStream_t s) {
  uint32_t tiles = (g.N + 128 * NJ - 1) / (128 * NJ);
  for (uint32_t i = 0; MODE == GEMM_STORE && i < g.n_more; ++i) tiles += (g.more[i].N + 128 * NJ - 1) / (128 * NJ);
  dim3 grid(tiles, (g.P + 32 * MT - 1) / (32 * MT), g.ksplit > 1 ? g.ksplit : 1);
  constexpr uint32_t lds = gemm_lds_bytes<MT>();
  if constexpr (MODE == GEMM_SWIGLU && MT == 4) {  // Q4_K only (gemm_go)
    if (g.type != T_Q4_K) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_gemm_b3<T_Q4_K, MODE, MT, NJ>), grid, dim3(256), (gemm_lds_bytes_t<T_Q4_K, MODE, MT, NJ>()),
                       s, g);
    return hipGetLastError();
  } else {
    return gemm_go_types<MODE, MT, NJ>(g, grid, lds, s);
  }
}

template <int MODE, int MT, int NJ>
static hipError_t gemm_go_types(const GemmArgs& g, dim3 grid, uint32_t lds, hipStream_t s) {
  switch (g.type) {
    case T_Q4_K:
      hipLaunchKernelGGL((k_gemm_b3<T_Q4_K, MODE, MT, NJ>), grid, dim3(256), (gemm_lds_bytes_t<T_Q4_K, MODE, MT, NJ>()),
                         s, g);
      break;
    case T_Q6_K: hipLaunchKernelGGL((k_gemm_b3<T_Q6_K, MODE, MT, NJ>), grid, dim3(256), lds, s, g); break;
    case T_Q8_0: hipLaunchKernelGGL((k_gemm_b3<T_Q8_0, MODE, MT, NJ>), grid, dim3(256), lds, s, g); break;
    case T_Q5_0: hipLaunchKernelGGL((k_gemm_b3<T_Q5_0, MODE, MT, NJ>), grid, dim3(256), lds, s, g); break;
    case T_F32: hipLaunchKernelGGL((k_gemm_b3<T_F32, MODE, MT, NJ>), grid, dim3(256), lds, s, g); break;
    case T_F16: hipLaunchKernelGGL((k_gemm_b3<T_F16, MODE, MT, NJ>), grid, dim3(256), lds, s, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Tiles of 128 weight rows per matrix by 32 MT tokens: MT 4 (128 tokens)
// above 64 rows, MT 2 above 32, MT 1 below.  SwiGLU's two matrices take MT
// 4 only in Q4_K, whose weight registers leave room for it at two waves
// per SIMD (the other formats' would spill).
template <int MODE>
static hipError_t gemm_go(const GemmArgs& g, hipStream_t s) {
  if (g.P > 64 && (MODE != GEMM_SWIGLU || g.type == T_Q4_K)) return gemm_go_b3<MODE, 4, 1>(g, s);
  if (g.P > 32) return gemm_go_b3<MODE, 2, 1>(g, s);
  return gemm_go_b3<MODE, 1, 1>(g, s);
}

// The Q4_K kernels' LDS (A planes + offset windows) passes the default 64
// KiB limit at 128-token tiles.
template <int MODE>
static hipError_t gemm_prepare_mode() {
  const auto attr = hipFuncAttributeMaxDynamicSharedMemorySize;
  hipError_t e;
  if ((e = hipFuncSetAttribute((const void*)k_gemm_b3<T_Q4_K, MODE, 4, 1>, attr,
                               (int)gemm_lds_bytes_t<T_Q4_K, MODE, 4, 1>())) ||
      (e = hipFuncSetAttribute((const void*)k_gemm_b3<T_Q4_K, MODE, 2, 1>, attr,
                               (int)gemm_lds_bytes_t<T_Q4_K, MODE, 2, 1>())))
    return e;
  return hipFuncSetAttribute((const void*)k_gemm_b3<T_Q4_K, MODE, 1, 1>, attr,
                             (int)gemm_lds_bytes_t<T_Q4_K, MODE, 1, 1>());
}

hipError_t gemm_prepare() {
  hipError_t e;
  if ((e = gemm_prepare_mode<GEMM_STORE>()) || (e = gemm_prepare_mode<GEMM_RESID>())) return e;
  return gemm_prepare_mode<GEMM_SWIGLU>();
}

// out[r][n] (row stride ldo) += the ksplit partial products in z order
__global__ __launch_bounds__(256) void k_split_sum(const float* __restrict__ partial, uint32_t ksplit, uint32_t P,
                                                   uint32_t N, float* __restrict__ out, uint32_t ldo) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= P * N) return;
  const uint32_t r = i / N, n = i % N;
  float sum = out[(size_t)r * ldo + n];
  for (uint32_t z = 0; z < ksplit; ++z) sum += partial[(size_t)z * P * N + i];
  out[(size_t)r * ldo + n] = sum;
}

// SwiGLU of split products: the gate and up sums over z, then silu(g) * u
// (tensor.rs:224) into the split planes
__global__ __launch_bounds__(256) void k_split_swiglu(const float* __restrict__ partial, uint32_t ksplit, uint32_t P,
                                                      uint32_t N, uint16_t* __restrict__ o_hi,
                                                      uint16_t* __restrict__ o_lo, uint32_t ldo) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= P * N) return;
  const uint32_t r = i / N, n = i % N;
  float gs = 0.f, us = 0.f;
  for (uint32_t z = 0; z < ksplit; ++z) {
    gs += partial[(size_t)(2 * z) * P * N + i];
    us += partial[(size_t)(2 * z + 1) * P * N + i];
  }
  split1(gs / (1.0f + expf(-gs)) * us, o_hi[(size_t)r * ldo + n], o_lo[(size_t)r * ldo + n]);
}

// Store of split products: the sums over z, + the segment's bias
// (model.rs:179-183), into the segment's output
__global__ __launch_bounds__(256) void k_split_store(const float* __restrict__ partial, uint32_t ksplit, GemmArgs g) {
  const uint32_t cols = gemm_cols(g), i = blockIdx.x * 256 + threadIdx.x;
  if (i >= g.P * cols) return;
  const uint32_t r = i / cols;
  uint32_t n = i % cols, ldo = g.ldo;
  const float* bias = g.bias;
  float* out = g.out;
  if (n >= g.N) {
    n -= g.N;
    uint32_t k = 0;
    while (k + 1 < g.n_more && n >= g.more[k].N) n -= g.more[k++].N;
    bias = g.more[k].bias;
    out = g.more[k].out;
    ldo = g.more[k].ldo;
  }
  float sum = 0.f;
  for (uint32_t z = 0; z < ksplit; ++z) sum += partial[(size_t)z * g.P * cols + i];
  out[(size_t)r * ldo + n] = bias ? sum + bias[n] : sum;
}

// Split K for a launch of fewer than 256 blocks (most CUs idle): chunks of
// a multiple of 8 or 16 k-steps, enough of them for ~256 blocks, within
// the partial buffer.
static void plan_ksplit(GemmArgs& g, GemmMode mode) {
  g.ksplit = 1;
  g.kchunk = 0;
  if (!g.partial) return;
  const size_t per = mode == GEMM_SWIGLU ? 2 : 1;  // partial products per output
  const uint32_t mt = g.P > 64 && (mode != GEMM_SWIGLU || g.type == T_Q4_K) ? 4 : g.P > 32 ? 2 : 1;
  uint32_t tiles = (g.N + 127) / 128;
  for (uint32_t i = 0; i < g.n_more; ++i) tiles += (g.more[i].N + 127) / 128;
  const uint32_t ttiles = (g.P + 32 * mt - 1) / (32 * mt), blocks = tiles * ttiles, nk = g.K / 32;
  // chunks of 8 k-steps (whole superblocks; a Q4_K chunk of 8 applies half
  // an offset window) below 64 k-steps, of 16 above: more chunks of a long K
  // cost more in partial traffic than they gain (7B: 11.8 -> 11.9 ms at 128
  // tokens with 8; 1.5B 5.3 -> 5.0 ms, 0.5B 3.1 -> 1.9 ms)
  const uint32_t minc = nk < 64 ? 8 : 16;
  if (blocks >= 256 || nk < 2 * minc) return;  // (below 128: 7B 512-token prefill 26.9 ms, 256: 25.6)
  const uint32_t want = (256 + blocks - 1) / blocks;
  uint32_t chunk = std::max<uint32_t>(minc, nk / want / minc * minc);
  while ((size_t)((nk + chunk - 1) / chunk) * per * g.P * gemm_cols(g) > g.partial_floats) chunk += minc;
  const uint32_t ks = (nk + chunk - 1) / chunk;
  if (ks < 2) return;
  g.ksplit = ks;
  g.kchunk = chunk;
}

hipError_t launch_gemm(const GemmArgs& g0, GemmMode mode, hipStream_t s) {
  GemmArgs g = g0;
  plan_ksplit(g, mode);
  if (g.K % 32 || g.P == 0 || g.N == 0) return hipErrorInvalidValue;
  if ((uint64_t)g.N * g.row_bytes >= BUF_INVALID || (uint64_t)g.P * g.K * 2 >= BUF_INVALID) return hipErrorInvalidValue;
  if (mode == GEMM_SWIGLU ? (!g.o_hi || !g.o_lo) : !g.out) return hipErrorInvalidValue;
  if (g.n_more > 2 || (g.n_more && mode != GEMM_STORE)) return hipErrorInvalidValue;
  if (g.type == T_Q4_K && (!g.x_hi || !g.x_lo || (uint64_t)g.P * (g.K / 32) * 2 >= BUF_INVALID))
    return hipErrorInvalidValue;
  for (uint32_t i = 0; i < g.n_more; ++i)
    if (!g.more[i].w || !g.more[i].out || g.more[i].N == 0 || (uint64_t)g.more[i].N * g.row_bytes >= BUF_INVALID)
      return hipErrorInvalidValue;
  switch (mode) {
    case GEMM_STORE: {
      if (hipError_t e = gemm_go<GEMM_STORE>(g, s)) return e;
      if (g.ksplit < 2) return hipSuccess;
      hipLaunchKernelGGL(k_split_store, dim3((g.P * gemm_cols(g) + 255) / 256), dim3(256), 0, s, g.partial, g.ksplit, g);
      return hipGetLastError();
    }
    case GEMM_RESID: {
      if (hipError_t e = gemm_go<GEMM_RESID>(g, s)) return e;
      if (g.ksplit < 2) return hipSuccess;
      hipLaunchKernelGGL(k_split_sum, dim3((g.P * g.N + 255) / 256), dim3(256), 0, s, g.partial, g.ksplit, g.P, g.N,
                         g.out, g.ldo);
      return hipGetLastError();
    }
    case GEMM_SWIGLU: {
      if (hipError_t e = gemm_go<GEMM_SWIGLU>(g, s)) return e;
      if (g.ksplit < 2) return hipSuccess;
      hipLaunchKernelGGL(k_split_swiglu, dim3((g.P * g.N + 255) / 256), dim3(256), 0, s, g.partial, g.ksplit, g.P, g.N,
                         g.o_hi, g.o_lo, g.ldo);
      return hipGetLastError();
    }
  }
  return hipErrorInvalidValue;
}

// ---- RoPE of q/k rows and KV append (model.rs:193-217, 346-356) -----------------------
// Row r is position pos0 + r.  Same rotation as the decode kernel: no FMA
// contraction, table from the host.
__global__ __launch_bounds__(256) void k_rope_kv_rows(float* __restrict__ q, const float* __restrict__ k,
                                                      const float* __restrict__ v, const float* __restrict__ cs,
                                                      float* __restrict__ kc, float* __restrict__ vc, uint32_t nh,
                                                      uint32_t nkv, uint32_t hd, uint32_t pos0) {
  const uint32_t r = blockIdx.x, pos = pos0 + r, half = hd / 2, qd = nh * hd, kvd = nkv * hd;
  const float* cr = cs + (size_t)pos * hd;
  for (uint32_t i = threadIdx.x; i < (nh + nkv) * half; i += 256) {
    const uint32_t h = i / half, j = i % half;
    const float* src = h < nh ? q + (size_t)r * qd + h * hd : k + (size_t)r * kvd + (h - nh) * hd;
    const float a0 = src[j], b0 = src[j + half], c0 = cr[j], s0 = cr[half + j];
    const float r0 = __fsub_rn(__fmul_rn(a0, c0), __fmul_rn(b0, s0));
    const float r1 = __fadd_rn(__fmul_rn(a0, s0), __fmul_rn(b0, c0));
    float* dst = h < nh ? q + (size_t)r * qd + h * hd : kc + (size_t)pos * kvd + (h - nh) * hd;
    dst[j] = r0;
    dst[j + half] = r1;
  }
  for (uint32_t i = threadIdx.x; i < kvd; i += 256) vc[(size_t)pos * kvd + i] = v[(size_t)r * kvd + i];
}

hipError_t launch_rope_kv_rows(float* q, const float* k, const float* v, const float* cs, float* kc, float* vc,
                               uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t pos0, uint32_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_rope_kv_rows, dim3(n), dim3(256), 0, s, q, k, v, cs, kc, vc, nh, nkv, hd, pos0);
  return hipGetLastError();
}

// ---- K/V of a layer as bf16 planes for the prefill attention -------------------------
// Keys 0 .. T: K as hi / lo planes [T][kvd] (the cache's row layout) and V
// transposed, Vt [kvd][Tp] (Tp = T rounded up to 32, zeros past T), with
// the keys of every 16-key group stored in the order the P.V MFMA reads
// them: position 8h + i of a group holds key 8(i/4) + 4h + i%4.
__host__ __device__ constexpr uint32_t kv_pos16(uint32_t j) { return 8u * ((j / 4) % 2) + 4u * (j / 8) + j % 4; }

__global__ __launch_bounds__(256) void k_kv_split(const float* __restrict__ kc, const float* __restrict__ vc,
                                                  uint32_t T, uint32_t Tp, uint32_t kvd, uint16_t* __restrict__ kh,
                                                  uint16_t* __restrict__ kl, uint16_t* __restrict__ vth,
                                                  uint16_t* __restrict__ vtl) {
  const uint32_t k0 = 16 * blockIdx.x;
  for (uint32_t d = threadIdx.x; d < kvd; d += 256) {
    float vv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t key = k0 + j;
      if (key < T) {
        const float kx = kc[(size_t)key * kvd + d];
        split1(kx, kh[(size_t)key * kvd + d], kl[(size_t)key * kvd + d]);
        vv[kv_pos16(j)] = vc[(size_t)key * kvd + d];
      } else {
        vv[kv_pos16(j)] = 0.0f;
      }
    }
#pragma unroll
    for (int p = 0; p < 16; p += 8) {
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = vv[p + i];
      uint4 hi, lo;
      split8(y, hi, lo);
      *(uint4*)(vth + (size_t)d * Tp + k0 + p) = hi;
      *(uint4*)(vtl + (size_t)d * Tp + k0 + p) = lo;
    }
  }
}

hipError_t launch_kv_split(const float* kc, const float* vc, uint32_t T, uint32_t kvd, uint16_t* planes,
                           hipStream_t s) {
  const uint32_t Tp = (T + 31) / 32 * 32;
  uint16_t* kh = planes;
  uint16_t* kl = kh + (size_t)Tp * kvd;
  uint16_t* vth = kl + (size_t)Tp * kvd;
  uint16_t* vtl = vth + (size_t)Tp * kvd;
  hipLaunchKernelGGL(k_kv_split, dim3(Tp / 16), dim3(256), 0, s, kc, vc, T, Tp, kvd, kh, kl, vth, vtl);
  return hipGetLastError();
}

// ---- causal attention of a block of query rows on MFMA (model.rs:371-438) ------------
// Block: 128 query rows from q0 of query head h; wave w owns rows
// q0 + 32w .. +32 and runs every 32-key tile up to its last row.  The
// block stages each key tile once in LDS for its four waves (K rows and V^T
// rows, both planes; the next tile's bytes load into registers while the
// current one computes).  On v_mfma_f32_32x32x16_bf16 with every operand
// split hi + lo (three products: hi.hi, hi.lo, lo.hi).  Lane l supplies
// A[l%32][8(l/32) .. +8] and B[8(l/32) .. +8][l%32]; register v of lane l
// is C[8(v/4) + 4(l/32) + v%4][l%32]:
//  - S^T (keys x queries) = K Q^T over the head dims, 16 dims per MFMA:
//    lane l takes dims 16c + 8(l/32) .. +8 of key row l%32 and of query
//    row l%32 (split once).  Lane l then holds the scores of query l%32 for
//    16 keys; the softmax's running max and sum are 16 in-lane values and
//    one exchange with lane l^32.
//  - O^T (dims x queries) += V^T P^T, 16 keys per MFMA: B = P^T is lane l's
//    own 8 scores of the half (split), k-index 8(l/32) + i standing for key
//    8(i/4) + 4(l/32) + i%4 of the 16; A = V^T comes from Vt, whose keys
//    are stored in that order.
// Key-tile chunks of query block qb (128 rows from row 128 qb, positions
// pos0 + row): its tiles of 32 keys up to its last row, in chunks of kchunk
// tiles, so that the late (long) query blocks run as several blocks.
__host__ __device__ inline uint32_t attn_chunks(uint32_t qb, uint32_t pos0, uint32_t n, uint32_t kchunk) {
  const uint32_t last = pos0 + min(n, qb * 128 + 128) - 1;
  return (last / 32 + kchunk) / kchunk;
}

template <int HD>
__global__ __launch_bounds__(256, 2) void k_attn_rows_mfma(const float* __restrict__ q, const uint16_t* __restrict__ kh,
                                                           const uint16_t* __restrict__ kl,
                                                           const uint16_t* __restrict__ vth,
                                                           const uint16_t* __restrict__ vtl, uint32_t Tp,
                                                           uint16_t* __restrict__ out_hi,
                                                           uint16_t* __restrict__ out_lo, uint32_t nh, uint32_t nkv,
                                                           uint32_t pos0, uint32_t n, float scale, uint32_t kchunk,
                                                           float* __restrict__ part, uint32_t nchm) {
  constexpr int DT = HD / 32, NC = HD / 16;
  constexpr int KP = HD + 8, VP = 40;  // LDS row pitches (bf16): 16-byte reads of 16 rows hit distinct banks
  constexpr int KE = 32 * KP, VE = HD * VP;
  __shared__ __attribute__((aligned(16))) uint16_t ks[2][2][KE];  // [buffer][plane]
  __shared__ __attribute__((aligned(16))) uint16_t vs[2][2][VE];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, hh = lane >> 5, col = lane & 31;
  const uint32_t h = blockIdx.y, g = h / (nh / nkv), qd = nh * HD, kvd = nkv * HD;
  // block x: chunk c of the key tiles of query block qb (attn_chunks)
  uint32_t qb = 0, c = blockIdx.x;
  while (c >= attn_chunks(qb, pos0, n, kchunk)) c -= attn_chunks(qb++, pos0, n, kchunk);
  const uint32_t nch = attn_chunks(qb, pos0, n, kchunk);
  const uint32_t q0 = qb * 128, qw = q0 + 32 * w, qi = qw + col;
  const bool wave_on = qw < n;
  const uint32_t qr = qi < n ? qi : n - 1;  // lanes past the rows redo row n - 1, not stored
  const uint32_t qpos = pos0 + qr;
  const uint32_t last_w = pos0 + min(n, qw + 32) - 1, last_b = pos0 + min(n, q0 + 128) - 1;
  // tile loaders: K row t / 8 (HD / 8 values from 16 * (t % 8) * HD / 128), V^T row
  // t * HD / 256 (32 * HD / 256 keys)
  constexpr int KV = HD / 8, VV = HD / 8;  // bf16 per thread per plane
  constexpr int KL = KV / 8, VL = VV / 8;  // 16-byte loads per plane
  const uint32_t kr = t / 8, kc0 = (t % 8) * KV;
  const uint32_t vr = t / (256 / HD), vk0 = (t % (256 / HD)) * VV;
  // the next tile's bytes, through buffer loads (plain loads of these
  // arrays were kept in scratch memory by the compiler)
  const rsrc_t rkh = make_rsrc(kh, Tp * kvd * 2), rkl = make_rsrc(kl, Tp * kvd * 2);
  const rsrc_t rvh = make_rsrc(vth, Tp * kvd * 2), rvl = make_rsrc(vtl, Tp * kvd * 2);
  uint4 pkh[KL], pkl[KL], pvh[VL], pvl[VL];
  auto fetch = [&](uint32_t kt) {
    const uint32_t ko = 2 * (min(kt * 32 + kr, last_b) * kvd + g * HD + kc0);
    const uint32_t vo = 2 * ((g * HD + vr) * Tp + kt * 32 + vk0);
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      pkh[i] = bl128(rkh, ko + 16 * i);
      pkl[i] = bl128(rkl, ko + 16 * i);
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      pvh[i] = bl128(rvh, vo + 16 * i);
      pvl[i] = bl128(rvl, vo + 16 * i);
    }
  };
  auto put = [&](int b) {
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      *(uint4*)&ks[b][0][kr * KP + kc0 + 8 * i] = pkh[i];
      *(uint4*)&ks[b][1][kr * KP + kc0 + 8 * i] = pkl[i];
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      *(uint4*)&vs[b][0][vr * VP + vk0 + 8 * i] = pvh[i];
      *(uint4*)&vs[b][1][vr * VP + vk0 + 8 * i] = pvl[i];
    }
  };
  // the lane's query dims 16c + 8 hh .. +8, split
  bf16x8 qh_[NC], ql_[NC];
  {
    const float* qrow = q + (size_t)qr * qd + h * HD + 8 * hh;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const float4 a = *(const float4*)(qrow + 16 * c), b = *(const float4*)(qrow + 16 * c + 4);
      const float y[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      uint4 hi, lo;
      split8(y, hi, lo);
      qh_[c] = __builtin_bit_cast(bf16x8, hi);
      ql_[c] = __builtin_bit_cast(bf16x8, lo);
    }
  }
  f32x16 o[DT];
#pragma unroll
  for (int tt = 0; tt < DT; ++tt)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[tt][v] = 0.f;
  float m = -INFINITY, lsum = 0.f;
  const uint32_t k_lo = c * kchunk, ntiles = min(last_b / 32 + 1, k_lo + kchunk);
  fetch(k_lo);
  put(0);
  __syncthreads();
  for (uint32_t kt = k_lo; kt < ntiles; ++kt) {
    const int b = (kt - k_lo) & 1;
    if (kt + 1 < ntiles) fetch(kt + 1);
    if (wave_on && kt * 32 <= last_w) {
      f32x16 sc;
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[v] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const bf16x8 a_h = *(const bf16x8*)&ks[b][0][col * KP + 16 * c + 8 * hh];
        const bf16x8 a_l = *(const bf16x8*)&ks[b][1][col * KP + 16 * c + 8 * hh];
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, qh_[c], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, ql_[c], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_l, qh_[c], sc, 0, 0, 0);
      }
      // scale and causal mask (model.rs:384-397), then the online softmax
      float mx = m;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t key = kt * 32 + 8 * (v / 4) + 4 * hh + (v & 3);
        sc[v] = key <= qpos ? sc[v] * scale : -INFINITY;
        mx = fmaxf(mx, sc[v]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float ms = mx == -INFINITY ? 0.f : mx;  // no unmasked key yet: keep the exponents finite
      const float cf = expf(m - ms);
      float ps = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        sc[v] = expf(sc[v] - ms);
        ps += sc[v];
      }
      ps += __shfl_xor(ps, 32, 64);
      lsum = lsum * cf + ps;
      m = mx;
#pragma unroll
      for (int tt = 0; tt < DT; ++tt)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[tt][v] *= cf;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = sc[8 * s + i];
        uint4 phi, plo;
        split8(y, phi, plo);
        const bf16x8 b_h = __builtin_bit_cast(bf16x8, phi), b_l = __builtin_bit_cast(bf16x8, plo);
#pragma unroll
        for (int tt = 0; tt < DT; ++tt) {
          const uint32_t vo = (32 * tt + col) * VP + 16 * s + 8 * hh;
          const bf16x8 a_h = *(const bf16x8*)&vs[b][0][vo], a_l = *(const bf16x8*)&vs[b][1][vo];
          o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, b_h, o[tt], 0, 0, 0);
          o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, b_l, o[tt], 0, 0, 0);
          o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_l, b_h, o[tt], 0, 0, 0);
        }
      }
    }
    if (kt + 1 < ntiles) put(b ^ 1);
    __syncthreads();
  }
  // the o-proj GEMM's operand form: bf16 hi + lo planes; lane l holds dims
  // 32t + 8(v/4) + 4(l/32) + v%4 of query l%32
  if (!wave_on || qi >= n) return;
  if (nch > 1) {  // chunk c's (o, m, l) of the row, merged by k_attn_rows_merge
    float* pr = part + (((size_t)h * n + qi) * nchm + c) * (HD + 2);
#pragma unroll
    for (int tt = 0; tt < DT; ++tt)
#pragma unroll
      for (int v = 0; v < 16; ++v) pr[32 * tt + 8 * (v / 4) + 4 * hh + (v & 3)] = o[tt][v];
    if (hh == 0) {
      pr[HD] = m;
      pr[HD + 1] = lsum;
    }
    return;
  }
  const float inv = 1.0f / lsum;
  const size_t ob = (size_t)qi * qd + h * HD + 4 * hh;
#pragma unroll
  for (int tt = 0; tt < DT; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint32_t hi[2], lo[2];
      split2(o[tt][4 * r] * inv, o[tt][4 * r + 1] * inv, hi[0], lo[0]);
      split2(o[tt][4 * r + 2] * inv, o[tt][4 * r + 3] * inv, hi[1], lo[1]);
      *(uint2*)(out_hi + ob + 32 * tt + 8 * r) = make_uint2(hi[0], hi[1]);
      *(uint2*)(out_lo + ob + 32 * tt + 8 * r) = make_uint2(lo[0], lo[1]);
    }
}

// The chunks of a row's query block merged (x = sum e^(m_c - M) o_c /
// sum e^(m_c - M) l_c, chunks in order) into the output planes; rows of
// one-chunk blocks were written by the attention kernel.
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_rows_merge(const float* __restrict__ part, uint16_t* __restrict__ out_hi,
                                                        uint16_t* __restrict__ out_lo, uint32_t nh, uint32_t pos0,
                                                        uint32_t n, uint32_t kchunk, uint32_t nchm) {
  const uint32_t r = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const uint32_t nch = attn_chunks(r / 128, pos0, n, kchunk);
  if (nch < 2) return;
  const float* pr = part + ((size_t)h * n + r) * nchm * (HD + 2);
  float M = -INFINITY;
  for (uint32_t c = 0; c < nch; ++c) M = fmaxf(M, pr[c * (HD + 2) + HD]);
  float O = 0.f, L = 0.f;
  for (uint32_t c = 0; c < nch; ++c) {
    const float mc = pr[c * (HD + 2) + HD], e = mc == -INFINITY ? 0.f : expf(mc - M);
    O += pr[c * (HD + 2) + d] * e;
    L += pr[c * (HD + 2) + HD + 1] * e;
  }
  split1(O * (1.0f / L), out_hi[(size_t)r * nh * HD + h * HD + d], out_lo[(size_t)r * nh * HD + h * HD + d]);
}

size_t attn_rows_part_floats(uint32_t nh, uint32_t hd, uint32_t rows) { return (size_t)nh * rows * ATTN_ROWS_CHUNKS * (hd + 2); }

hipError_t launch_attn_rows(const float* q, const uint16_t* kv_planes, uint16_t* out_hi, uint16_t* out_lo, uint32_t nh,
                            uint32_t nkv, uint32_t hd, uint32_t pos0, uint32_t n, float scale, float* part,
                            hipStream_t s) {
  if (n == 0 || nkv == 0 || nh % nkv) return hipErrorInvalidValue;
  const uint32_t T = pos0 + n, Tp = (T + 31) / 32 * 32, kvd = nkv * hd;
  const uint16_t* kh = kv_planes;
  const uint16_t* kl = kh + (size_t)Tp * kvd;
  const uint16_t* vth = kl + (size_t)Tp * kvd;
  const uint16_t* vtl = vth + (size_t)Tp * kvd;
  // chunks of at least 16 key tiles (512 keys; 32 measured the same at 7B
  // and 5 % slower at a 1024-token 1.5B prompt), at most ATTN_ROWS_CHUNKS
  // per query block; without a partial buffer, one chunk
  const uint32_t qbs = (n + 127) / 128, tiles = (T - 1) / 32 + 1;
  const uint32_t kchunk = part ? std::max<uint32_t>(16, (tiles + ATTN_ROWS_CHUNKS - 1) / ATTN_ROWS_CHUNKS) : tiles;
  uint32_t blocks = 0;
  for (uint32_t qb = 0; qb < qbs; ++qb) blocks += attn_chunks(qb, pos0, n, kchunk);
  const uint32_t nchm = attn_chunks(qbs - 1, pos0, n, kchunk);
  dim3 grid(blocks, nh);
  if (hd == 128)
    hipLaunchKernelGGL((k_attn_rows_mfma<128>), grid, dim3(256), 0, s, q, kh, kl, vth, vtl, Tp, out_hi, out_lo, nh, nkv,
                       pos0, n, scale, kchunk, part, nchm);
  else if (hd == 64)
    hipLaunchKernelGGL((k_attn_rows_mfma<64>), grid, dim3(256), 0, s, q, kh, kl, vth, vtl, Tp, out_hi, out_lo, nh, nkv,
                       pos0, n, scale, kchunk, part, nchm);
  else
    return hipErrorInvalidValue;
  if (hipError_t e = hipGetLastError()) return e;
  if (nchm < 2) return hipSuccess;
  if (hd == 128)
    hipLaunchKernelGGL((k_attn_rows_merge<128>), dim3(n, nh), dim3(128), 0, s, part, out_hi, out_lo, nh, pos0, n,
                       kchunk, nchm);
  else
    hipLaunchKernelGGL((k_attn_rows_merge<64>), dim3(n, nh), dim3(64), 0, s, part, out_hi, out_lo, nh, pos0, n, kchunk,
                       nchm);
  return hipGetLastError();
}

// ---- end of a prefill: argmax of the last row's logits, position += n -------------------
__global__ __launch_bounds__(1024) void k_prefill_end(StepState* st, const uint64_t* __restrict__ best,
                                                      uint32_t n_best, uint32_t n) {
  __shared__ uint64_t wb[16];
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
    const uint32_t idx = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull);
    st->next_tok = idx;
    st->tok = idx;
    st->pos += n;
  }
}

hipError_t launch_prefill_end(StepState* st, const uint64_t* best, uint32_t n_best, uint32_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_prefill_end, dim3(1), dim3(1024), 0, s, st, best, n_best, n);
  return hipGetLastError();
}

}  // namespace frn
