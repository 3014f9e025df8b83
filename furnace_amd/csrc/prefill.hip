// gfx950 kernels of the prefill: the prompt's tokens processed as a block
// of rows per layer (Model::forward_cached with seq > 1, model.rs:579-592,
// layer_forward_cached model.rs:444-478).
//
//  - k_embed_rows     embedding rows of the block's token ids
//  - k_row_inv        1/sqrt(mean(x^2) + eps) per row (the rmsnorm factor)
//  - k_gemm_q         C = A' . W^T with W in its raw GGUF blocks: each
//                     k-step dequantizes a 64x32 weight tile (bit-exact f32,
//                     the same formulas as the dequant kernel) and a 64x32
//                     activation tile (rmsnorm applied on load) into LDS and
//                     runs v_mfma_f32_32x32x2f32 on them; epilogues: store +
//                     bias, residual add, SwiGLU of two weights
//  - k_rope_kv_rows   RoPE of q and k rows at their positions, KV append
//  - k_attn_rows_mfma causal GQA attention of 32 query rows of one head over
//                     the cache on v_mfma_f32_32x32x2f32 (S^T = K Q^T, then
//                     O^T += V^T P^T), online softmax over 32-key tiles
//
// The MFMA operands are exact f32 (the dequantized weights are exact), so
// the GEMM differs from the CPU path only by the order of its sums.
#include "formats.hpp"
#include "kernels.hpp"

namespace frn {

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float4 u4f_(uint4 v) {
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

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

// ---- rmsnorm factor per row (tensor.rs:164-185) -------------------------------------
__global__ __launch_bounds__(256) void k_row_inv(const float* __restrict__ x, uint32_t cols, float eps,
                                                 float* __restrict__ inv) {
  __shared__ float red[4];
  const float* row = x + (size_t)blockIdx.x * cols;
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < cols; i += 256) ss += row[i] * row[i];
  ss = group_reduce<64>(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) inv[blockIdx.x] = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)cols + eps);
}

hipError_t launch_row_inv(const float* x, uint32_t rows, uint32_t cols, float eps, float* inv, hipStream_t s) {
  hipLaunchKernelGGL(k_row_inv, dim3(rows), dim3(256), 0, s, x, cols, eps, inv);
  return hipGetLastError();
}

// ---- quantized GEMM on MFMA ----------------------------------------------------
// Eight consecutive weights w[n][k .. k + 8) (k % 8 == 0, inside one 32-value
// group) of a row at byte offset `row` (BUF_INVALID: zeros), bit-exact as
// decode_elem.  Raw bytes are fetched by load(), decoded by decode().
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
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t b = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      y[i] = dd * (float)((b >> sh) & 0x0Fu) - mm;
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
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lo = ((i < 4 ? ql.x : ql.y) >> (8 * (i & 3) + lsh)) & 0x0Fu;
      const uint32_t hi = ((i < 4 ? qh.x : qh.y) >> (8 * (i & 3) + hsh)) & 3u;
      y[i] = dsc * (float)((int32_t)(lo | (hi << 4)) - 32);
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

// Block tile GM = 64 * MT rows of A (tokens) x 64 weight rows, k-steps of
// 32; 4 waves, wave (wm, wn) owns the 32 * MT x 32 output sub-tile (wm, wn)
// and runs 16 * MT v_mfma_f32_32x32x2f32 per k-step and weight matrix, so a
// dequantized weight tile feeds MT times the MFMAs (the single-weight
// GEMMs are bound by the dequantization at MT 1).  Lane l supplies
// A[l%32][l/32] and W[l%32][l/32] of each k-pair; the accumulator's
// register v of lane l is C[8(v/4) + 4(l/32) + v%4][l%32] (layouts checked
// on gfx950).
constexpr int GN = 64, GK = 32, GKP = GK + 1;  // LDS rows padded against bank conflicts

template <uint32_t T, int MODE, int MT>
__global__ __launch_bounds__(256) void k_gemm_q(GemmArgs g) {
  constexpr int NW = MODE == GEMM_SWIGLU ? 2 : 1, GM = 64 * MT;
  __shared__ float As[GM * GKP];
  __shared__ float Ws[NW][GN * GKP];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, wm = wave & 1, wn = wave >> 1;
  const uint32_t r0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
  // tile loaders: thread t fills rows t/4 + 64 m (m < MT) of A and row t/4
  // of W, k sub-range 8*(t%4)
  const uint32_t lr = t / 4, lk = 8 * (t % 4);
  const rsrc_t ra = make_rsrc(g.a, g.P * g.K * 4);
  const rsrc_t rw[2] = {make_rsrc(g.w, g.N * g.row_bytes), make_rsrc(NW == 2 ? g.w2 : g.w, g.N * g.row_bytes)};
  const bool wrow = n0 + lr < g.N;
  uint32_t a_off[MT];
  float inv[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const uint32_t r = r0 + lr + 64 * m;
    a_off[m] = r < g.P ? 4 * (r * g.K + lk) : BUF_INVALID;
    inv[m] = (g.inv && r < g.P) ? g.inv[r] : 1.0f;
  }
  const uint32_t w_off = wrow ? (n0 + lr) * g.row_bytes : BUF_INVALID;
  const rsrc_t rn = make_rsrc(g.nw, g.nw ? g.K * 4 : 0);

  float4 pa0[MT], pa1[MT], pn0, pn1;
  Deq8<T> pw[NW];
  auto fetch = [&](uint32_t k0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      pa0[m] = u4f_(bl128(ra, a_off[m] == BUF_INVALID ? BUF_INVALID : a_off[m] + 4 * k0));
      pa1[m] = u4f_(bl128(ra, a_off[m] == BUF_INVALID ? BUF_INVALID : a_off[m] + 4 * k0 + 16));
    }
    if (g.nw) {
      pn0 = u4f_(bl128(rn, 4 * (k0 + lk)));
      pn1 = u4f_(bl128(rn, 4 * (k0 + lk) + 16));
    }
#pragma unroll
    for (int i = 0; i < NW; ++i) pw[i].load(rw[i], w_off, k0 + lk);
  };
  auto stage = [&](uint32_t k0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float av[8] = {pa0[m].x, pa0[m].y, pa0[m].z, pa0[m].w, pa1[m].x, pa1[m].y, pa1[m].z, pa1[m].w};
      if (g.nw) {  // rmsnorm on load: (x * inv) * w (tensor.rs:181-183)
        const float nv[8] = {pn0.x, pn0.y, pn0.z, pn0.w, pn1.x, pn1.y, pn1.z, pn1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) av[i] = av[i] * inv[m] * nv[i];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) As[(lr + 64 * m) * GKP + lk + i] = av[i];
    }
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      float y[8];
      pw[w].decode(k0 + lk, y);
#pragma unroll
      for (int i = 0; i < 8; ++i) Ws[w][lr * GKP + lk + i] = y[i];
    }
  };

  f32x16 acc[MT][NW];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int w = 0; w < NW; ++w)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[m][w][v] = 0.f;
  const uint32_t nk = g.K / GK;
  fetch(0);
  stage(0);
  __syncthreads();
  // wave (wm, wn): A rows wm * 32 * MT + 32 m + lane % 32, W rows wn * 32 + lane % 32
  const int ar = wm * 32 * MT + (lane & 31), wr = wn * 32 + (lane & 31), kh = lane >> 5;
  for (uint32_t kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) fetch((kt + 1) * GK);
#pragma unroll
    for (int kk = 0; kk < GK; kk += 2) {
      float wv[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) wv[w] = Ws[w][wr * GKP + kk + kh];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float a = As[(ar + 32 * m) * GKP + kk + kh];
#pragma unroll
        for (int w = 0; w < NW; ++w) acc[m][w] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, wv[w], acc[m][w], 0, 0, 0);
      }
    }
    __syncthreads();
    if (kt + 1 < nk) {
      stage((kt + 1) * GK);
      __syncthreads();
    }
  }
  // epilogue: register v of lane l is C[8(v/4) + 4(l/32) + v%4][l%32]
  const uint32_t n = n0 + wn * 32 + (lane & 31);
  if (n >= g.N) return;
  const float bias = (MODE == GEMM_STORE && g.bias) ? g.bias[n] : 0.f;
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const uint32_t r = r0 + wm * 32 * MT + 32 * m + 8 * (v / 4) + 4 * (lane >> 5) + (v & 3);
      if (r >= g.P) continue;
      float* o = g.out + (size_t)r * g.ldo + n;
      if (MODE == GEMM_STORE) *o = g.bias ? acc[m][0][v] + bias : acc[m][0][v];  // model.rs:179-183
      if (MODE == GEMM_RESID) *o = *o + acc[m][0][v];                            // tensor.rs:232
      if (MODE == GEMM_SWIGLU) {                                                 // tensor.rs:224
        const float gg = acc[m][0][v];
        *o = gg / (1.0f + expf(-gg)) * acc[m][NW - 1][v];
      }
    }
}

// Row blocks of 128 (MT 2) once the prompt block has the rows to keep the
// grid full; 64 below.  Measured: 7B 2048-token prefill 8,090 -> 8,185
// tokens/s, 1.5B 4096-token 34,790 -> 35,480 (the GEMMs are not bound by
// the dequantization alone).
template <int MODE, int MT>
static hipError_t gemm_go_mt(const GemmArgs& g, hipStream_t s) {
  dim3 grid((g.N + GN - 1) / GN, (g.P + 64 * MT - 1) / (64 * MT));
  switch (g.type) {
    case T_Q4_K: hipLaunchKernelGGL((k_gemm_q<T_Q4_K, MODE, MT>), grid, dim3(256), 0, s, g); break;
    case T_Q6_K: hipLaunchKernelGGL((k_gemm_q<T_Q6_K, MODE, MT>), grid, dim3(256), 0, s, g); break;
    case T_Q8_0: hipLaunchKernelGGL((k_gemm_q<T_Q8_0, MODE, MT>), grid, dim3(256), 0, s, g); break;
    case T_Q5_0: hipLaunchKernelGGL((k_gemm_q<T_Q5_0, MODE, MT>), grid, dim3(256), 0, s, g); break;
    case T_F32: hipLaunchKernelGGL((k_gemm_q<T_F32, MODE, MT>), grid, dim3(256), 0, s, g); break;
    case T_F16: hipLaunchKernelGGL((k_gemm_q<T_F16, MODE, MT>), grid, dim3(256), 0, s, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int MODE>
static hipError_t gemm_go(const GemmArgs& g, hipStream_t s) {
  return g.P >= 512 ? gemm_go_mt<MODE, 2>(g, s) : gemm_go_mt<MODE, 1>(g, s);
}

hipError_t launch_gemm(const GemmArgs& g, GemmMode mode, hipStream_t s) {
  if (g.K % GK || g.P == 0 || g.N == 0) return hipErrorInvalidValue;
  if ((uint64_t)g.N * g.row_bytes >= BUF_INVALID || (uint64_t)g.P * g.K * 4 >= BUF_INVALID) return hipErrorInvalidValue;
  switch (mode) {
    case GEMM_STORE: return gemm_go<GEMM_STORE>(g, s);
    case GEMM_RESID: return gemm_go<GEMM_RESID>(g, s);
    case GEMM_SWIGLU: return gemm_go<GEMM_SWIGLU>(g, s);
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

// ---- causal attention of a block of query rows on MFMA (model.rs:371-438) ------------
// Block (32 query rows from q0, query head h), 4 waves; wave w takes the
// 32-key tiles w, w + 4, ... up to the block's last query position.  With
// v_mfma_f32_32x32x2f32 (lane l supplies A[l%32][l/32] and B[l/32][l%32];
// accumulator register v of lane l is C[8(v/4) + 4(l/32) + v%4][l%32]):
//  - S^T (keys x queries) = K Q^T over the head dims.  Both operands take
//    the dims in the same permuted order (half l/32 of k-step 4j + c reads
//    dim 8j + 4(l/32) + c), so each lane loads float4s of its key row and
//    of its query row.  Lane l then holds the scores of query l%32 for 16
//    keys; the softmax's running max and sum are 16 in-lane values and one
//    exchange with lane l^32.
//  - O^T (dims x queries) += V^T P^T.  The B operand P^T is the S^T
//    accumulator itself: k-step i takes keys 8(i/4) + 4(l/32) + i%4, the
//    keys whose scores lane l holds in register i.  A = V^T comes from one
//    load per lane and k-step, dims DPL*(l%32) .. +DPL of the key's row
//    (DPL = HD/32); component t feeds M-tile t, whose row m is dim DPL*m + t.
// The waves' partials (O, m, l) are merged in wave order through LDS.  All
// products and sums are f32, so only the order of the sums differs from the
// CPU path (model.rs:371-438).
template <int HD>
__global__ __launch_bounds__(256) void k_attn_rows_mfma(const float* __restrict__ q, const float* __restrict__ kc,
                                                        const float* __restrict__ vc, float* __restrict__ out,
                                                        uint32_t nh, uint32_t nkv, uint32_t pos0, uint32_t n,
                                                        float scale) {
  constexpr int NW = 4, DPL = HD / 32, NQ = HD / 8, OLD = HD + 1;  // O rows padded against bank conflicts
  __shared__ float mls[NW][2][32];
  __shared__ float os[32 * OLD];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hh = lane >> 5, col = lane & 31;
  const uint32_t h = blockIdx.y, g = h / (nh / nkv), qd = nh * HD, kvd = nkv * HD;
  const uint32_t q0 = blockIdx.x * 32, qi = q0 + col;
  const uint32_t qr = qi < n ? qi : n - 1;  // lanes past the block's rows redo row n - 1, not stored
  const uint32_t qpos = pos0 + qr, last = pos0 + min(n, q0 + 32) - 1;
  float4 qv[NQ];
  const float* qrow = q + (size_t)qr * qd + h * HD + 4 * hh;
#pragma unroll
  for (int j = 0; j < NQ; ++j) qv[j] = *(const float4*)(qrow + 8 * j);
  f32x16 o[DPL];
#pragma unroll
  for (int t = 0; t < DPL; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[t][v] = 0.f;
  float m = -INFINITY, lsum = 0.f;
  const float* kbase = kc + (size_t)g * HD + 4 * hh;
  const float* vbase = vc + (size_t)g * HD + DPL * col;
  const uint32_t ntiles = last / 32 + 1;
  for (uint32_t kt = w; kt < ntiles; kt += NW) {
    // key rows past the last query position are clamped to it (their scores are masked)
    const float* krow = kbase + (size_t)min(kt * 32 + col, last) * kvd;
    f32x16 sc;
#pragma unroll
    for (int v = 0; v < 16; ++v) sc[v] = 0.f;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const float4 kv = *(const float4*)(krow + 8 * j);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qv[j].x, sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qv[j].y, sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qv[j].z, sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qv[j].w, sc, 0, 0, 0);
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
    const float c = expf(m - ms);
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      sc[v] = expf(sc[v] - ms);
      ps += sc[v];
    }
    ps += __shfl_xor(ps, 32, 64);
    lsum = lsum * c + ps;
    m = mx;
#pragma unroll
    for (int t = 0; t < DPL; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[t][v] *= c;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t key = min(kt * 32 + 8 * (i / 4) + 4 * hh + (i & 3), last);
      const float* vrow = vbase + (size_t)key * kvd;
      if constexpr (DPL == 4) {
        const float4 vv = *(const float4*)vrow;
        o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, sc[i], o[0], 0, 0, 0);
        o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, sc[i], o[1], 0, 0, 0);
        o[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, sc[i], o[2], 0, 0, 0);
        o[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, sc[i], o[3], 0, 0, 0);
      } else {
        const float2 vv = *(const float2*)vrow;
        o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, sc[i], o[0], 0, 0, 0);
        o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, sc[i], o[1], 0, 0, 0);
      }
    }
  }
  // merge: M = max over the waves, partial w weighted by e^(m_w - M)
  if (hh == 0) {
    mls[w][0][col] = m;
    mls[w][1][col] = lsum;
  }
  __syncthreads();
  auto weight = [&](int ww, uint32_t qq, float M) {
    const float mw = mls[ww][0][qq];
    return mw == -INFINITY ? 0.f : expf(mw - M);
  };
  float M = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, mls[ww][0][col]);
  const float e = weight(w, col, M);
  for (int ww = 0; ww < NW; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int t = 0; t < DPL; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float* p = os + col * OLD + DPL * (8 * (v / 4) + 4 * hh + (v & 3)) + t;
          *p = ww == 0 ? e * o[t][v] : *p + e * o[t][v];
        }
    }
    __syncthreads();
  }
  // thread t writes query t / 8, dims [HD/8 * (t % 8), +HD/8)
  const uint32_t qq = threadIdx.x / 8, d0 = (threadIdx.x % 8) * (HD / 8);
  if (q0 + qq >= n) return;
  float Mq = -INFINITY, L = 0.f;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) Mq = fmaxf(Mq, mls[ww][0][qq]);
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) L += weight(ww, qq, Mq) * mls[ww][1][qq];
  float* orow = out + (size_t)(q0 + qq) * qd + h * HD + d0;
#pragma unroll
  for (int d = 0; d < HD / 8; ++d) orow[d] = os[qq * OLD + d0 + d] / L;
}

hipError_t launch_attn_rows(const float* q, const float* kc, const float* vc, float* out, uint32_t nh, uint32_t nkv,
                            uint32_t hd, uint32_t pos0, uint32_t n, float scale, hipStream_t s) {
  if (n == 0 || nkv == 0 || nh % nkv) return hipErrorInvalidValue;
  dim3 grid((n + 31) / 32, nh);
  if (hd == 128)
    hipLaunchKernelGGL((k_attn_rows_mfma<128>), grid, dim3(256), 0, s, q, kc, vc, out, nh, nkv, pos0, n, scale);
  else if (hd == 64)
    hipLaunchKernelGGL((k_attn_rows_mfma<64>), grid, dim3(256), 0, s, q, kc, vc, out, nh, nkv, pos0, n, scale);
  else
    return hipErrorInvalidValue;
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
