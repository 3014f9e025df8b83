// gfx950 kernels of the token loop: dequant, fused dequant-GEMV, embedding,
// RoPE + KV-cache write, split-sequence GQA decode attention, argmax.
#include "formats.hpp"
#include "items.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace frn {

constexpr int ATT_CHUNK = ATTENTION_CHUNK;  // positions per attention block (one wave per softmax row)
uint32_t attention_splits(uint32_t max_ctx, uint32_t cap) {
  const uint32_t t = (max_ctx + ATT_CHUNK - 1) / ATT_CHUNK;
  return t < cap ? t : cap;
}

// ---- reductions -----------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) { return group_reduce<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_reduce<64>(v, OpMax()); }
// Sum over a block of NW waves, in wave order; every thread gets the result.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r += red[i];
  __syncthreads();
  return r;
}

// GEMV blocks: NT threads (4 waves, two blocks per CU, for in <= 4096; 8
// waves, one block per CU, for the long in of the FFN down projection, so
// each CU stages its 35 KB of activations once and every thread converts
// half as many values).  Whether x is staged as int8 digits (in <= 4096,
// where the rmsnorm also occurs) and whether the f32 form is padded
// (xf_pad4; with 4-wave blocks only while two blocks per CU still fit).
__host__ __device__ constexpr bool gemv_dig(int nx, int nt) { return nx * 8 * nt <= 4096; }
__host__ __device__ constexpr bool gemv_pad(int nx, int nt) { return !gemv_dig(nx, nt) && (nt >= 512 || nx <= 5); }

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


// ---- activation staging ------------------------------------------------------
// Thread t owns the 8-value groups u = t + NT i (i < NX) of x.  Their loads
// (and the rmsnorm gain's) are issued first, before any weight load, so the
// staging waits only on them while the first weight batch stays in flight.
__device__ __forceinline__ float4 u4f(uint4 v) {
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
// XF: the items read the f32 copy of x (every format but the K-quants in
// the int8 form); DSUM: they read the chunks' digit sums (Q6_K and the
// formats not known to skip them; Q4_K and Q8_0 read only the chunk
// scale and sum(x)).
template <int NX, bool NORM, bool ATT, bool DIG, bool PAD = false, bool XF = true, bool DSUM = true, int NT = 256>
struct XStage {
  // ATT: x is the attention output, merged here from the per-split partials
  // (o, m, l) of the attention kernel: NB splits are loaded up front with
  // the other staging loads, further splits (long contexts) afterwards.
  static constexpr int NB = ATT ? 8 / NX : 1;
  float4 x[NX][2], w[NORM ? NX : 1][2];
  float2 pm[ATT ? NX : 1][NB];
  float4 po[ATT ? NX : 1][NB][2];
  uint32_t ns = 0;
  // per group i: byte offset of split 0 of its 8 values (BUF_INVALID: no
  // group) and from there to the split's (m, l); bytes per split.  The
  // divisions by the head size happen once here, so the per-split offsets
  // are selects (a division in the offset made the compiler branch around
  // every load and re-read the kernel arguments each time).
  uint32_t pbase[ATT ? NX : 1], pml[ATT ? NX : 1], pstride = 0;
  __device__ __forceinline__ void att_setup(const GemvArgs& a) {
    pstride = 4u * (a.att_hd + 2);
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const uint32_t u = threadIdx.x + (uint32_t)NT * i, h = 8u * u / a.att_hd, d0 = 8u * u % a.att_hd;
      pbase[i] = u < a.in / 8 ? 4u * (h * a.att_ms * (a.att_hd + 2) + d0) : BUF_INVALID;
      pml[i] = 4u * (a.att_hd - d0);
    }
  }
  __device__ __forceinline__ void load_batch(rsrc_t rp, uint32_t sp0) {
#pragma unroll
    for (int i = 0; i < NX; ++i) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint32_t sp = sp0 + b;
        const uint32_t o = (pbase[i] != BUF_INVALID && sp < ns) ? pbase[i] + sp * pstride : BUF_INVALID;
        po[i][b][0] = u4f(bl128(rp, o));
        po[i][b][1] = u4f(bl128(rp, o + 16u));
        const uint2 q = bl64(rp, o == BUF_INVALID ? BUF_INVALID : o + pml[i]);
        pm[i][b] = make_float2(__uint_as_float(q.x), __uint_as_float(q.y));
      }
    }
  }
  // the first batch is loaded before the step position is known (splits
  // past the step's count are loaded and then ignored), so its loads
  // overlap the read of st->pos
  __device__ __forceinline__ void load_att(const GemvArgs& a, rsrc_t rp) {
    ns = NB;
    att_setup(a);
    load_batch(rp, 0);
    const uint32_t T = a.st->pos + 1, len = attention_split_len(T);
    ns = (T + len - 1) / len;
  }
  // softmax merge of the splits (model.rs:371-438 evaluated split-wise):
  // x = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s, M = max_s m_s, one
  // batch of NB splits at a time (the first batch was loaded up front)
  __device__ __forceinline__ void merge_att(const GemvArgs& a, rsrc_t rp) {
    float M[NX], L[NX], o[NX][8];
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      M[i] = -INFINITY;
      L[i] = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) o[i][k] = 0.f;
    }
    for (uint32_t sp0 = 0; sp0 < ns; sp0 += NB) {
      if (sp0) load_batch(rp, sp0);
#pragma unroll
      for (int i = 0; i < NX; ++i) {
        float Mb = M[i];
#pragma unroll
        for (int b = 0; b < NB; ++b)
          if (sp0 + b < ns) Mb = fmaxf(Mb, pm[i][b].x);
        const float c = expf(M[i] - Mb);  // rescale of the earlier batches (0 when there were none)
        L[i] *= c;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[i][k] *= c;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          // splits past the step's count were loaded before the count was
          // known and may hold anything (even NaN): select, do not scale
          if (sp0 + b >= ns) continue;
          const float e = expf(pm[i][b].x - Mb);
          L[i] += e * pm[i][b].y;
          o[i][0] += e * po[i][b][0].x; o[i][1] += e * po[i][b][0].y;
          o[i][2] += e * po[i][b][0].z; o[i][3] += e * po[i][b][0].w;
          o[i][4] += e * po[i][b][1].x; o[i][5] += e * po[i][b][1].y;
          o[i][6] += e * po[i][b][1].z; o[i][7] += e * po[i][b][1].w;
        }
        M[i] = Mb;
      }
    }
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const float il = L[i] > 0.f ? 1.0f / L[i] : 0.f;
      x[i][0] = make_float4(o[i][0] * il, o[i][1] * il, o[i][2] * il, o[i][3] * il);
      x[i][1] = make_float4(o[i][4] * il, o[i][5] * il, o[i][6] * il, o[i][7] * il);
    }
  }
  __device__ __forceinline__ void load(rsrc_t rx, rsrc_t rn) {
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const uint32_t o = 32u * (threadIdx.x + (uint32_t)NT * i);
      x[i][0] = u4f(bl128(rx, o));
      x[i][1] = u4f(bl128(rx, o + 16u));
      if (NORM) {
        w[i][0] = u4f(bl128(rn, o));
        w[i][1] = u4f(bl128(rn, o + 16u));
      }
    }
  }
  // rmsnorm (tensor.rs:164-185: x * (1 / sqrt(mean(x^2) + eps)) * w) when
  // norm; then the f32 values and, in the f32 form (!DIG), the sum of every
  // 16-value chunk, or, in the int8 form (DIG), every 32-value chunk split
  // into the digit planes and metadata (XLds in formats.hpp).  The threads
  // of a chunk are adjacent lanes; groups past K were loaded as zeros and
  // are not stored.
  __device__ __forceinline__ void finish(uint32_t K, bool norm, float eps, float* xf, uint8_t* pl, float* red4) {
    float inv = 1.0f;
    if (NORM && norm) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NX; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) ss += x[i][h].x * x[i][h].x + x[i][h].y * x[i][h].y + x[i][h].z * x[i][h].z +
                                          x[i][h].w * x[i][h].w;
      ss = block_sum<NT / 64>(ss, red4);
      inv = 1.0f / sqrtf(ss / (float)K + eps);
    }
    const uint32_t n16 = K / 16;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      if ((uint32_t)NT * i >= K / 8) break;  // block-uniform: no thread has group i
      const uint32_t u = threadIdx.x + (uint32_t)NT * i;
      const bool live = u < K / 8;
      float4 a = x[i][0], b = x[i][1];
      if (NORM && norm) {
        const float4 wa = w[i][0], wb = w[i][1];
        a.x = a.x * inv * wa.x; a.y = a.y * inv * wa.y; a.z = a.z * inv * wa.z; a.w = a.w * inv * wa.w;
        b.x = b.x * inv * wb.x; b.y = b.y * inv * wb.y; b.z = b.z * inv * wb.z; b.w = b.w * inv * wb.w;
      }
      if (live && (XF || !DIG)) {
        const uint32_t f = PAD ? xf_pad4(2 * u) : 2 * u;  // 2u, 2u + 1 share a chunk
        ((float4*)xf)[f] = a;
        ((float4*)xf)[f + 1] = b;
      }
      if (!DIG) {
        float s16 = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        s16 = group_reduce<2>(s16);
        if (live && (u & 1) == 0) ((float*)pl)[u >> 1] = s16;
        continue;
      }
      const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      float amax = 0.f, xsum = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        amax = fmaxf(amax, fabsf(v[j]));
        xsum += v[j];
      }
      amax = group_reduce<4>(amax, OpMax());  // over the 32-value chunk
      // hardware reciprocals: the digits only need cs * inv_s = 2^-14 to
      // f32 precision, not correctly rounded quotients
      const float inv_s = amax > 0.f ? 127.0f * __builtin_amdgcn_rcpf(amax) : 0.f;
      const float cs = amax > 0.f ? __builtin_amdgcn_rcpf(inv_s) * (1.0f / 16384.0f) : 0.f;
      uint32_t w0[2] = {0, 0}, w1[2] = {0, 0}, w2[2] = {0, 0};
      int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float t = v[j] * inv_s;
        float r0 = rintf(t), e0 = (t - r0) * 128.0f;
        float r1 = rintf(e0), e1 = (e0 - r1) * 128.0f;
        float r2 = rintf(e1);
        int d0 = (int)r0, d1 = (int)r1, d2 = (int)r2;
        w0[j >> 2] |= (uint32_t)(d0 & 0xFF) << (8 * (j & 3));
        w1[j >> 2] |= (uint32_t)(d1 & 0xFF) << (8 * (j & 3));
        w2[j >> 2] |= (uint32_t)(d2 & 0xFF) << (8 * (j & 3));
        s0 += d0;
        s1 += d1;
        s2 += d2;
      }
      // per 16-value record: the two threads u, u^1
      xsum = group_reduce<2>(xsum);
      if (DSUM) {
        s0 = group_reduce<2>(s0);
        s1 = group_reduce<2>(s1);
        s2 = group_reduce<2>(s2);
      }
      if (live) {
        const uint32_t c = u >> 1, off = 16u * swz(c, n16) + 8u * (u & 1);
        *(uint2*)(pl + off) = make_uint2(w0[0], w0[1]);
        *(uint2*)(pl + K + off) = make_uint2(w1[0], w1[1]);
        *(uint2*)(pl + 2 * K + off) = make_uint2(w2[0], w2[1]);
        if ((u & 1) == 0)
          *(float4*)(pl + 3 * K + 16u * swz(c, n16)) =
              make_float4(cs, xsum, DSUM ? __int_as_float(-32 * s0) : 0.f,
                          DSUM ? __int_as_float(-32 * (128 * s1 + s2)) : 0.f);
      }
    }
    __syncthreads();
  }
};


// ---- fused dequant-GEMV -----------------------------------------------------------
#ifndef GEMV_MAX_GRID
#define GEMV_MAX_GRID 512
#endif
// A block stages x (and applies the rmsnorm) once; then each of its NW =
// NT / 64 waves works alone through "units" of G = 64 / LPR rows, one group
// of LPR lanes per row (SWIGLU: per gate/up row pair).  Wave w of block b
// takes units NW b + w, NW b + w + NW nblk, ...  A unit is S steps; in step s lane gl of a
// row loads items (s * BI + j) * LPR + gl, j < BI.  The steps of all the
// wave's units form one flat pipeline: the loads of step f + 1 are issued
// before step f is computed, and the first step's before the staging.
template <uint32_t T, int LPR, int MODE, int NX, bool NORM, bool ONE, int NT>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, const GemvSeg& sg, uint32_t blk, uint32_t nblk,
                                          float* xf, uint8_t* pl, float* red4, uint64_t* best_s) {
  using F = Fmt<T>;
  using Raw = typename F::Raw;
  constexpr int R = MODE == GEMV_SWIGLU ? 2 : 1;
  constexpr int BI = gemv_bi(T, MODE), B = BI * R, G = 64 / LPR;
  constexpr bool ATT = MODE == GEMV_RESID_ATT;  // x = merged attention partials, then as RESID
  constexpr bool RES = MODE == GEMV_RESID || ATT;
  constexpr bool EX = MODE == GEMV_STORE || RES;  // per-row bias / residual input
  constexpr int NCX = F::NC > 0 ? F::NC : 1;
  constexpr bool PRELOAD = F::NC > 0 && F::NC <= 2;  // register budget: 16-17 VGPRs per chunk
  // x as int8 digits (cheaper dot) for in <= 4096; the f32 form (far
  // cheaper staging: no digits) for the long in of the FFN down projection,
  // where each block would otherwise split 8960+ values into digits.
  // Measured per launch (1.5B): down 11.6 -> 9.8 us with the f32 form;
  // gate_up 9.9 vs 11.3 and o_proj 6.2 vs 6.7 us in favour of the digits.
  constexpr bool DIG = gemv_dig(NX, NT);
  constexpr int NW = NT / 64;
  using XT = typename std::conditional<DIG, XC, XF>::type;
  // the f32 form stages x padded (xf_pad4) for the K-quant items (gemv_pad)
  constexpr bool PAD = gemv_pad(NX, NT) && (T == T_Q4_K || T == T_Q6_K);
  // the wave index through readfirstlane: the compiler then knows every
  // per-wave quantity below is uniform (scalar loop control, no exec masks)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gl = lane % LPR, g = lane / LPR;
  const bool pr = ((a.in / 32) % 2) == 0;
  const int n_items = items_per_row(T, a.in, pr);
  const uint32_t S = (uint32_t)(n_items + LPR * BI - 1) / (LPR * BI);
  const uint32_t n_units = (sg.rows + G - 1) / G, stride = NW * nblk, u0 = NW * blk + wave;
  const uint32_t n_steps = u0 < n_units ? (n_units - u0 + stride - 1) / stride * S : 0;
  const uint32_t wbytes = sg.rows * sg.row_bytes;
  const rsrc_t rw = make_rsrc(sg.w, wbytes), rw2 = make_rsrc(R == 2 ? sg.w2 : sg.w, wbytes);
  const float* exp_ = RES ? sg.resid : sg.bias;
  const rsrc_t rex = make_rsrc(exp_, exp_ ? sg.rows * 4 : 0);
  const XLds X{xf, pl, a.in};

  XStage<NX, NORM, ATT, DIG, PAD, !(T == T_Q4_K || T == T_Q6_K), !(T == T_Q4_K || T == T_Q8_0), NT> xs;
  const rsrc_t rp = make_rsrc(a.att_part, ATT ? a.att_part_bytes : 0);
  if (ATT)
    xs.load_att(a, rp);
  else
    xs.load(make_rsrc(a.x, a.in * 4), make_rsrc(a.norm_w, a.norm_w ? a.in * 4 : 0));
  __builtin_amdgcn_sched_barrier(0);  // keep the x loads ahead of the weight loads

  auto row_off = [&](uint32_t unit) -> uint32_t {
    const uint32_t row = unit * G + g;
    return row < sg.rows ? row * sg.row_bytes : BUF_INVALID;
  };
  // the bias / residual of the row rides along with the unit's last step,
  // so the epilogue issues no load of its own (which would have to wait for
  // the next step's loads too)
  auto issue = [&](uint32_t unit, uint32_t step, Raw(&raw)[B], float& ex) {
    const uint32_t ro = row_off(unit);
#pragma unroll
    for (int j = 0; j < BI; ++j) {
      const int it = (int)(step * BI + j) * LPR + gl;
      const uint32_t o = it < n_items ? ro : BUF_INVALID;
      raw[j * R] = F::load(rw, o, it, pr);
      if (R == 2) raw[j * R + R - 1] = F::load(rw2, o, it, pr);
    }
    if (EX) ex = __uint_as_float(bl32(rex, ro == BUF_INVALID ? BUF_INVALID : 4u * (unit * G + g)));
  };
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  uint64_t best = 0;
  // xget(j, itc, xc): the staged chunks of the lane's j-th item of the step
  auto consume = [&](uint32_t unit, uint32_t step, Raw(&raw)[B], float ex, auto&& xget) {
    const uint32_t row = unit * G + g, ro = row_off(unit);
#pragma unroll
    for (int j = 0; j < BI; ++j) {
      const int it = (int)(step * BI + j) * LPR + gl;
      const bool ok = it < n_items && ro != BUF_INVALID;
      const int itc = ok ? it : 0;  // masked items read chunk 0 of x and have zero weights
      XT xc[NCX];
      xget(j, itc, xc);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint8_t* rp = ok ? (r == 0 ? sg.w : sg.w2) + ro : nullptr;
        acc[r] += F::dot(raw[j * R + r], ro, rp, itc, xc, X, pr);
      }
    }
    if (step + 1 < S) return;
    const float acc0 = group_reduce<LPR>(acc[0]), acc1 = MODE == GEMV_SWIGLU ? group_reduce<LPR>(acc[R - 1]) : 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    if (gl == 0 && row < sg.rows) {
      if (MODE == GEMV_STORE) sg.out[row] = sg.bias ? acc0 + ex : acc0;  // model.rs:179-183
      if (RES) {
        float v = ex + acc0;  // tensor.rs:232
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
  };
  auto from_lds = [&](int, int itc, XT* xc) {
#pragma unroll
    for (int i = 0; i < F::NC; ++i) {
      if constexpr (DIG)
        xc[i] = X.chunk(F::chunk(itc, i, pr));
      else
        xc[i] = X.template fchunk<PAD>(F::chunk(itc, i, pr));
    }
  };

  Raw ra[B], rb[B];
  float ea = 0.f, eb = 0.f;
  uint32_t iu = u0, is = 0, cu = u0, cs = 0;
  auto next = [&](uint32_t& u, uint32_t& s) {
    if (++s == S) {
      s = 0;
      u += stride;
    }
  };
  // depth 2: step f + 1's loads in flight while step f is computed (ra
  // holds step 0 on entry)
  auto run = [&](auto&& xget) {
    for (uint32_t f = 0; f < n_steps; f += 2) {
      issue(iu, is, rb, eb);  // past the wave's last step: rows past the end, loads of zeros
      next(iu, is);
      consume(cu, cs, ra, ea, xget);
      next(cu, cs);
      if (f + 1 >= n_steps) break;
      issue(iu, is, ra, ea);
      next(iu, is);
      consume(cu, cs, rb, eb, xget);
      next(cu, cs);
    }
  };
  // ONE (one step per unit, S == 1, chosen by the host): the activation
  // chunks go to registers when the format allows.  (A third buffer in
  // flight for the multi-step launches measured slower: more registers,
  // and their steps are not bound by memory latency.)
  issue(iu, is, ra, ea);
  next(iu, is);
  __builtin_amdgcn_sched_barrier(0);
  if (ATT) xs.merge_att(a, rp);
  xs.finish(a.in, a.norm_w != nullptr, a.eps, xf, pl, red4);
  if constexpr (ONE && PRELOAD) {
    // one step per unit: the lane reads the same items of every row it
    // visits, so their staged chunks are read from LDS once, into registers
    XT xr[BI][NCX];
#pragma unroll
    for (int j = 0; j < BI; ++j) {
      const int it = j * LPR + gl;
      from_lds(j, it < n_items ? it : 0, xr[j]);
    }
    run([&](int j, int, XT* xc) {
#pragma unroll
      for (int i = 0; i < F::NC; ++i) xc[i] = xr[j][i];
    });
  } else {
    run(from_lds);
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
      for (int i = 1; i < NW; ++i) b = best_s[i] > b ? best_s[i] : b;
      a.best[blockIdx.x] = b;
    }
  }
}

// T0 serves every segment whose type is T0, T1 the others (T1 == T0 for
// single-format launches), so each kernel carries one or two format paths.
// NX: 8-value groups of x per thread (in <= 2048 * NX); NORM: rmsnorm
// support (only the small-in kernels, where the norms occur).  MODE
// GEMV_RESID_ATT stages x from the attention partials (in <= 4096).
template <uint32_t T0, uint32_t T1, int LPR, int MODE, int NX, bool ONE, int NT>
__global__ __launch_bounds__(NT, 512 / NT) void k_gemv(GemvArgs a) {
  constexpr bool NORM = gemv_dig(NX, NT);
  extern __shared__ float4 smem4[];
  __shared__ float red4[NT / 64];
  __shared__ uint64_t best_s[NT / 64];
  // LDS: x[in] f32 | 4 byte planes of in bytes (digits, metadata); the f32
  // form: x (padded as xf_pad4 room for NX <= 5) | the in/16 chunk sums
  float* xf = (float*)smem4;
  uint8_t* pl = (uint8_t*)(xf + (gemv_pad(NX, NT) ? xf_padded_floats(a.in) : a.in));
  // Only STORE launches carry several segments (launch_gemv checks): the
  // other modes read segment 0's fields at constant offsets, in the same
  // round trip as the rest of the arguments, not after a segment search.
  constexpr bool ONESEG = MODE != GEMV_STORE;
  int si = 0;
  if constexpr (!ONESEG)
    while (si + 1 < a.n_seg && blockIdx.x >= a.seg[si + 1].block0) ++si;
  const GemvSeg& sg = a.seg[ONESEG ? 0 : si];
  const uint32_t blk = ONESEG ? blockIdx.x : blockIdx.x - sg.block0;
  const uint32_t nblk = ONESEG ? gridDim.x : (si + 1 < a.n_seg ? a.seg[si + 1].block0 : gridDim.x) - sg.block0;
  if (T0 == T1 || sg.type == T0)
    gemv_body<T0, LPR, MODE, NX, NORM, ONE, NT>(a, sg, blk, nblk, xf, pl, red4, best_s);
  else
    gemv_body<T1, LPR, MODE, NX, NORM, ONE, NT>(a, sg, blk, nblk, xf, pl, red4, best_s);
}

// LDS of a launch: x as f32, then the int8 form's 4 planes of `in` bytes
// (in <= 4096), or the f32 form's in/16 chunk sums after x, with room for
// the padded layout.
size_t gemv_lds_bytes(uint32_t in, bool) {
  if (in <= 4096) return (size_t)in * 8 + in / 4;
  return (size_t)xf_padded_floats(in) * 4 + in / 4;  // 8-wave blocks: padded f32 form
}
// Threads per block of a launch with input length in and first-segment
// format t: 8 waves for the K-quants' long inputs (the padded f32 form), 4
// otherwise (the Q8_0 f32 form measured faster at 4 waves: 0.5B decode
// 1353 tokens/s with 8-wave down blocks against 1484 with 4).
__host__ __device__ constexpr bool gemv_wide(uint32_t in, uint32_t t) { return in > 4096 && (t == T_Q4_K || t == T_Q6_K); }
static uint32_t gemv_threads(uint32_t in, uint32_t t) { return gemv_wide(in, t) ? 512u : 256u; }


// Lanes per row: the choice in {16, 32, 64} with the shortest critical
// path, counted as the busiest wave's units times the steps of a unit, on
// the waves that are resident at once (ties: fewer lanes, so fewer blocks
// stage x).  E.g. the 1.5B SwiGLU pair (8960 rows of 48 items, 2 items per
// lane and step): 16 lanes -> 2240 units of 2 steps on 2048 waves, 4
// steps; 32 lanes -> 4480 units of 1 step, 3 steps.
static uint32_t max_blocks(uint32_t in, uint32_t t);
static int lanes_per_row(uint32_t total_rows, uint32_t in, uint32_t type, int mode, int n_items) {
  const uint32_t nw = gemv_threads(in, type) / 64, cap_waves = nw * max_blocks(in, type);
  int best_l = 16;
  uint64_t best = ~0ull;
  for (int l = 16; l <= 64; l *= 2) {
    const uint32_t slots = (uint32_t)(l * gemv_bi(type, mode)), steps = ((uint32_t)n_items + slots - 1) / slots;
    const uint32_t units = (total_rows + 64 / l - 1) / (64 / l);
    const uint32_t waves = std::min(nw * ((units + nw - 1) / nw), cap_waves);
    const uint64_t cost = (uint64_t)((units + waves - 1) / waves) * steps;
    if (cost < best) {
      best = cost;
      best_l = l;
    }
  }
  return best_l;
}

// Grid cap: 2 blocks (8 waves) per CU for in <= 4096, one block per CU
// above.  (A cap of 4 per CU, which LDS would allow for small in, measured
// no faster: the kernels are VALU-bound, not short of waves.)
static uint32_t max_blocks(uint32_t in, uint32_t t) {
  if (gemv_threads(in, t) == 512) return 256;
  const size_t lds = gemv_lds_bytes(in, false);
  return lds > 80 * 1024 ? 256 : lds > 40 * 1024 ? 512 : GEMV_MAX_GRID;
}

// Blocks per segment in proportion to its units of 64 / LPR rows; each
// block runs 4 wave workers; at most as many blocks as are resident at once.
static uint32_t plan_blocks(GemvArgs& a, uint32_t rows_per_unit) {
  const uint32_t t = a.seg[0].type;
  uint32_t want[3], total = 0, cap = max_blocks(a.in, t), nw = gemv_threads(a.in, t) / 64;
  for (int i = 0; i < a.n_seg; ++i) {
    uint32_t units = (a.seg[i].rows + rows_per_unit - 1) / rows_per_unit;
    want[i] = (units + nw - 1) / nw;
    total += want[i];
  }
  uint32_t grid = total < cap ? total : cap, used = 0;
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
  int lpr = lanes_per_row(rows, in, type, GEMV_STORE, items_per_row(type, in, ((in / 32) % 2) == 0));
  const uint32_t nw = gemv_threads(in, type) / 64;
  uint32_t units = (rows + 64 / lpr - 1) / (64 / lpr), want = (units + nw - 1) / nw, cap = max_blocks(in, type);
  return want < cap ? want : cap;
}

template <uint32_t T0, uint32_t T1, int LPR, int MODE, int NX, bool ONE, int NT = 256>
static hipError_t go(GemvArgs a, hipStream_t s, uint32_t* nblocks) {
  uint32_t total = plan_blocks(a, 64 / LPR);
  if (nblocks) *nblocks = total;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL((k_gemv<T0, T1, LPR, MODE, NX, ONE, NT>), dim3(total), dim3(NT), gemv_lds_bytes(a.in, false), s,
                     a);
  return hipGetLastError();
}

// in <= 4096 (the hidden-size inputs, with or without rmsnorm; 4-wave
// blocks) or, without rmsnorm and only for STORE/RESID, in <= 20480 (the
// FFN down projection; K-quants in 8-wave blocks, NX 3 up to 12288, NX 5
// above; other formats in 4-wave blocks, NX 5 up to 10240, NX 10 above).
template <uint32_t T0, uint32_t T1, int MODE, int LPR>
static hipError_t pick_nx(const GemvArgs& a, hipStream_t s, uint32_t* nb) {
  const int n_items = items_per_row(T0, a.in, ((a.in / 32) % 2) == 0);
  const bool one = n_items <= LPR * gemv_bi(T0, MODE);  // one step per unit
  if (a.in <= 2048) return one ? go<T0, T1, LPR, MODE, 1, true>(a, s, nb) : go<T0, T1, LPR, MODE, 1, false>(a, s, nb);
  if (a.in <= 4096) return one ? go<T0, T1, LPR, MODE, 2, true>(a, s, nb) : go<T0, T1, LPR, MODE, 2, false>(a, s, nb);
  if constexpr ((MODE == GEMV_STORE || MODE == GEMV_RESID) && (T0 == T_Q4_K || T0 == T_Q6_K)) {
    if (a.norm_w == nullptr && a.in <= 12288) return go<T0, T1, LPR, MODE, 3, false, 512>(a, s, nb);
    if (a.norm_w == nullptr && a.in <= 20480) return go<T0, T1, LPR, MODE, 5, false, 512>(a, s, nb);
  } else if constexpr (MODE == GEMV_STORE || MODE == GEMV_RESID) {
    if (a.norm_w == nullptr && a.in <= 10240) return go<T0, T1, LPR, MODE, 5, false>(a, s, nb);
    if (a.norm_w == nullptr && a.in <= 20480) return go<T0, T1, LPR, MODE, 10, false>(a, s, nb);
  }
  return hipErrorInvalidValue;
}

template <uint32_t T0, uint32_t T1, int MODE>
static hipError_t pick_lpr(const GemvArgs& a, hipStream_t s, uint32_t* nb) {
  uint32_t rows = 0;
  for (int i = 0; i < a.n_seg; ++i) rows += a.seg[i].rows;
  int lpr = lanes_per_row(rows, a.in, a.seg[0].type, MODE, items_per_row(a.seg[0].type, a.in, ((a.in / 32) % 2) == 0));
  if (lpr == 16) return pick_nx<T0, T1, MODE, 16>(a, s, nb);
  if (lpr == 32) return pick_nx<T0, T1, MODE, 32>(a, s, nb);
  return pick_nx<T0, T1, MODE, 64>(a, s, nb);
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
      case T_F16: return pick_lpr<T_F16, T_F16, MODE>(a, s, nb);
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
  if (a.n_seg < 1 || a.n_seg > 3 || (mode != GEMV_STORE && a.n_seg != 1)) return hipErrorInvalidValue;
  for (int i = 0; i < a.n_seg; ++i)  // buffer offsets are 32-bit with BUF_INVALID above the range
    if ((uint64_t)a.seg[i].rows * a.seg[i].row_bytes >= BUF_INVALID) return hipErrorInvalidValue;
  switch (mode) {
    case GEMV_STORE: return launch_split<GEMV_STORE>(a, s, nb);
    case GEMV_RESID: return launch_split<GEMV_RESID>(a, s, nb);
    case GEMV_SWIGLU: return launch_split<GEMV_SWIGLU>(a, s, nb);
    case GEMV_ARGMAX: return launch_split<GEMV_ARGMAX>(a, s, nb);
    case GEMV_RESID_ATT:
      if (!a.att_part || !a.st || a.in % 8 || a.att_hd % 8 || (uint64_t)a.att_part_bytes >= BUF_INVALID)
        return hipErrorInvalidValue;
      return launch_split<GEMV_RESID_ATT>(a, s, nb);
  }
  return hipErrorInvalidValue;
}

// Only the in > 4096 kernels can use more than the default 64 KiB of
// dynamic LDS.
template <uint32_t T0, uint32_t T1, int LPR>
static hipError_t prep_one(int bytes) {
  hipError_t e;
  const auto attr = hipFuncAttributeMaxDynamicSharedMemorySize;
  if constexpr (T0 == T_Q4_K || T0 == T_Q6_K) {
    if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_STORE, 3, false, 512>, attr, bytes))) return e;
    if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_STORE, 5, false, 512>, attr, bytes))) return e;
    if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_RESID, 3, false, 512>, attr, bytes))) return e;
    return hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_RESID, 5, false, 512>, attr, bytes);
  } else {
    if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_STORE, 5, false, 256>, attr, bytes))) return e;
    if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_STORE, 10, false, 256>, attr, bytes))) return e;
    if ((e = hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_RESID, 5, false, 256>, attr, bytes))) return e;
    return hipFuncSetAttribute((const void*)k_gemv<T0, T1, LPR, GEMV_RESID, 10, false, 256>, attr, bytes);
  }
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
      (e = prep_types<T_F32, T_F32>(b)) || (e = prep_types<T_F16, T_F16>(b)) || (e = prep_types<T_Q4_K, T_Q6_K>(b)) || (e = prep_types<T_Q6_K, T_Q4_K>(b)))
    return e;
  return hipSuccess;
}

// ---- embedding row (model.rs:482-506) --------------------------------------
__global__ void k_embed(const uint8_t* __restrict__ table, uint32_t type, uint32_t hidden, uint32_t row_bytes,
                        StepState* st, float* __restrict__ x, const float* __restrict__ rope, uint32_t hd,
                        float* __restrict__ rope_cur) {
  uint32_t tok = st->tok;
  if (blockIdx.x == 0 && threadIdx.x < hd) rope_cur[threadIdx.x] = rope[(size_t)st->pos * hd + threadIdx.x];
  const uint8_t* row = table + (size_t)tok * row_bytes;
  int be = blk_elems(type), bb = blk_bytes(type);
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
    x[i] = type == T_F32 ? ((const float*)row)[i] : decode_elem(type, row + (size_t)(i / be) * bb, (int)(i % be));
}

hipError_t launch_embed(const uint8_t* table, uint32_t type, uint32_t hidden, uint32_t row_bytes, StepState* st,
                        float* x, const float* rope, uint32_t hd, float* rope_cur, hipStream_t s) {
  if (hd > 256) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_embed, dim3((hidden + 255) / 256), dim3(256), 0, s, table, type, hidden, row_bytes, st, x, rope,
                     hd, rope_cur);
  return hipGetLastError();
}

// ---- decode attention (model.rs:193-217, 346-356, 371-438) ---------------------
// One launch per layer.  Block (kv head g, split s, head group z) covers the
// split's positions (attention_split_len(pos + 1) of them, in sub-tiles of
// 64) for query heads g * gq + z * GQ + [0, nhb) of the gq sharing g (nhb =
// min(GQ, gq - z * GQ)); the z > 0 blocks read the K/V rows that block z = 0
// of the same (g, s) streams from HBM.  Block ids of one (g, s) differ by
// multiples of nkv * max_splits, a multiple of 8 at the usual shapes, so
// they land on one XCD and share its L2:
//  - rotates those query heads and head g's new key at the step position
//    (cs holds cos[hd/2] | sin[hd/2] of that position, the row the embed
//    kernel copied from the host-computed table, made with the CPU path's
//    powf/sinf/cosf; the rotation is evaluated without FMA contraction, so
//    q/k match the CPU bit for bit given equal inputs);
//  - the z = 0 block holding the step position appends head g's k/v to the
//    cache;
//  - per sub-tile: scores from K rows in registers, softmax with the
//    running max and sum of the split, P.V from V rows in LDS; the next
//    sub-tile's rows are loaded while this one's softmax and P.V run;
//  - writes its partial (o = sum_t e^(s_t - m) v_t, m, l = sum_t e^(s_t - m))
//    per query head to `part`; the o-proj GEMV (GEMV_RESID_ATT) merges the
//    splits while it stages its input (k_attn_merge in the long-context
//    form), so no block waits on another here.
template <int HD, int GQ>
__global__ __launch_bounds__(256) void k_attention(const float* __restrict__ q, const float* __restrict__ kn,
                                                   const float* __restrict__ vn, const float* __restrict__ cs,
                                                   float* __restrict__ kc, float* __restrict__ vc, uint32_t nh,
                                                   uint32_t nkv, uint32_t max_splits, uint32_t max_ctx, float scale,
                                                   float* __restrict__ part, const StepState* st, uint32_t cap,
                                                   uint32_t gq, uint32_t pre_all) {
  constexpr int C = ATT_CHUNK, TPP = 256 / C, DPT = HD / TPP, PARTS = 256 / HD, HALF = HD / 2, NP = C / PARTS;
  constexpr int RR = (GQ * HALF + HALF + 255) / 256;  // rotation rounds per thread
  // global loads: thread t moves float4 column lc of rows lr + RPI*i, so a
  // wave reads whole rows (contiguous 512 B for hd 128) per instruction
  constexpr int NC4 = HD / 4, RPI = 256 / NC4, LD = C / RPI;
  // K rows in LDS are padded to a stride of 64 mod 256 bytes: the score
  // reads (4 lanes per row, interleaved float4 columns) hit distinct banks
  constexpr int KLD = HD + 16;
  __shared__ __align__(16) float qs[GQ * HD];
  __shared__ __align__(16) float kcur[HD], vcur[HD];
  __shared__ __align__(16) float ks[C * KLD];
  __shared__ __align__(16) float vs[C * HD];
  __shared__ __align__(16) float ps[GQ * C];
  __shared__ float mrun[GQ], lrun[GQ], rescale[GQ];
  __shared__ float osum[PARTS * GQ * HD];
  const uint32_t g = blockIdx.x, split = blockIdx.y, hz = blockIdx.z;
  const uint32_t qh0 = g * gq + hz * GQ, nhb = min((uint32_t)GQ, gq - hz * GQ);  // the block's query heads
  const size_t kvd = (size_t)nkv * HD;
  const int p = threadIdx.x / TPP, sub = threadIdx.x % TPP;
  const int lc = threadIdx.x % NC4, lr = threadIdx.x / NC4;
  // Loads that do not depend on the step position go first, so they overlap
  // the read of st->pos: the first sub-tile's K/V rows as if the split
  // were 64 positions (it is, up to 1024 positions; rows at or past the
  // position are masked or replaced below), and the rotation's q/k inputs.
  // Only head group 0 streams the rows ahead when the grid holds splits
  // past the position (their blocks load the rows too before they know to
  // exit, and the other groups' copies would multiply that waste); a launch
  // whose grid is exactly the step's splits (pre_all) streams them in every
  // block.
  float4 kr[LD], vr[LD];
  if (hz == 0 || pre_all) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const uint32_t tp = split * C + lr + RPI * i;
      const size_t off = (size_t)(tp < max_ctx ? tp : 0) * kvd + (size_t)g * HD + 4 * lc;
      kr[i] = *(const float4*)(kc + off);
      vr[i] = *(const float4*)(vc + off);
    }
  }
  // rotation inputs: pair i < GQ*HALF of the query heads, then HALF of the key
  float ra[RR], rb[RR], rc[RR], rs[RR];
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    int i = threadIdx.x + 256 * r;
    if (i >= GQ * HALF + HALF) i = 0;  // clamped: loaded, not used
    const int h = i / HALF, j = i % HALF;
    // heads past the block's nhb rotate a copy of its last head (not stored)
    const float* src = h < GQ ? q + (size_t)(qh0 + min((uint32_t)h, nhb - 1)) * HD : kn + (size_t)g * HD;
    ra[r] = src[j];
    rb[r] = src[j + HALF];
  }
  const float vnew = vn[(size_t)g * HD + (threadIdx.x % HD)];
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    int i = threadIdx.x + 256 * r;
    if (i >= GQ * HALF + HALF) i = 0;
    const int j = i % HALF;
    rc[r] = cs[j];
    rs[r] = cs[HALF + j];
  }
  const uint32_t pos = st->pos, T = pos + 1;
  const uint32_t len = attention_split_len(T, cap), t0 = split * len;
  if (t0 >= T) return;
  const uint32_t ns = (T + len - 1) / len, tend = min(t0 + len, T), nsub = (tend - t0 + C - 1) / C;
  // rows of sub-tile k this thread loads: cached positions < pos only; the
  // step's own row comes from kcur/vcur, rows past the split are not used
  auto load_tile = [&](uint32_t k) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const uint32_t tp = t0 + k * C + lr + RPI * i;
      const size_t off = (size_t)((tp < tend && tp != pos) ? tp : 0) * kvd + (size_t)g * HD + 4 * lc;
      kr[i] = *(const float4*)(kc + off);
      vr[i] = *(const float4*)(vc + off);
    }
  };
  if (len != C || (hz != 0 && !pre_all)) load_tile(0);  // longer splits: the first sub-tile starts elsewhere
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    const int i = threadIdx.x + 256 * r;
    if (i < GQ * HALF + HALF) {
      const int h = i / HALF, j = i % HALF;
      float r0 = __fsub_rn(__fmul_rn(ra[r], rc[r]), __fmul_rn(rb[r], rs[r]));
      float r1 = __fadd_rn(__fmul_rn(ra[r], rs[r]), __fmul_rn(rb[r], rc[r]));
      float* dst = h < GQ ? qs + h * HD : kcur;
      dst[j] = r0;
      dst[j + HALF] = r1;
    }
  }
  if (threadIdx.x < HD) vcur[threadIdx.x] = vnew;
  if (threadIdx.x < GQ) {
    mrun[threadIdx.x] = -INFINITY;
    lrun[threadIdx.x] = 0.f;
  }
  __syncthreads();
  if (split == ns - 1 && hz == 0)  // KvCache::append of head g at pos
    for (int d = threadIdx.x; d < HD; d += 256) {
      kc[(size_t)pos * kvd + (size_t)g * HD + d] = kcur[d];
      vc[(size_t)pos * kvd + (size_t)g * HD + d] = vcur[d];
    }
  const int d = threadIdx.x % HD, prt = threadIdx.x / HD, wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float acc[GQ];
#pragma unroll
  for (int h = 0; h < GQ; ++h) acc[h] = 0.f;
  for (uint32_t k = 0; k < nsub; ++k) {
    // the sub-tile's rows to LDS (the step's own row from kcur/vcur, V rows
    // past the split as zeros), then the next sub-tile's loads go out
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int row = lr + RPI * i;
      const uint32_t tp = t0 + k * C + row;
      const bool valid = tp < tend, cur = valid && tp == pos;
      const float4 kv = cur ? ((const float4*)kcur)[lc] : kr[i];
      const float4 vv = cur ? ((const float4*)vcur)[lc] : valid ? vr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      *(float4*)(ks + row * KLD + 4 * lc) = kv;
      *(float4*)(vs + row * HD + 4 * lc) = vv;
    }
    if (k + 1 < nsub) load_tile(k + 1);  // in flight during this sub-tile's scores, softmax and P.V
    __syncthreads();
    {  // scores of position t0 + kC + p for all GQ heads at once (independent accumulators)
      const bool valid = t0 + k * C + p < tend;
      float sc[GQ];
#pragma unroll
      for (int h = 0; h < GQ; ++h) sc[h] = 0.f;
#pragma unroll
      for (int i = 0; i < DPT / 4; ++i) {
        const int c = TPP * i + sub;
        const float4 a = *(const float4*)(ks + p * KLD + 4 * c);
#pragma unroll
        for (int h = 0; h < GQ; ++h) {
          const float4 b = *(const float4*)(qs + h * HD + 4 * c);
          sc[h] += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
        }
      }
#pragma unroll
      for (int h = 0; h < GQ; ++h) sc[h] = group_reduce<TPP>(sc[h]);
      if (sub == 0)
#pragma unroll
        for (int h = 0; h < GQ; ++h) ps[h * C + p] = valid ? sc[h] * scale : -INFINITY;  // model.rs:397
    }
    __syncthreads();
    for (int h = wv; h < GQ; h += 4) {  // C == 64: one wave per softmax row, running max and sum
      const float v = ps[h * C + lane];
      const float m = fmaxf(wave_max(v), mrun[h]);
      const float e = expf(v - m);
      ps[h * C + lane] = e;
      const float l = wave_sum(e);
      if (lane == 0) {
        const float c = expf(mrun[h] - m);
        rescale[h] = c;
        lrun[h] = lrun[h] * c + l;
        mrun[h] = m;
      }
    }
    __syncthreads();
    // P.V: thread (d, prt) sums positions [NP prt, NP prt + NP) of the
    // sub-tile for all GQ heads; masked positions have p = 0, zero V rows
#pragma unroll
    for (int h = 0; h < GQ; ++h) acc[h] *= rescale[h];
#pragma unroll
    for (int j = 0; j < NP; j += 4) {
      const int t = prt * NP + j;
      const float v0 = vs[t * HD + d], v1 = vs[(t + 1) * HD + d], v2 = vs[(t + 2) * HD + d], v3 = vs[(t + 3) * HD + d];
#pragma unroll
      for (int h = 0; h < GQ; ++h) {
        const float4 pp = *(const float4*)(ps + h * C + t);
        acc[h] += pp.x * v0 + pp.y * v1 + pp.z * v2 + pp.w * v3;
      }
    }
    __syncthreads();  // vs and ps are rewritten by the next sub-tile
  }
#pragma unroll
  for (int h = 0; h < GQ; ++h) osum[(prt * GQ + h) * HD + d] = acc[h];
  __syncthreads();
  for (int i = threadIdx.x; i < (int)nhb * HD; i += 256) {
    int h = i / HD, dd = i % HD;
    float o = 0.f;
#pragma unroll
    for (int pp = 0; pp < PARTS; ++pp) o += osum[(pp * GQ + h) * HD + dd];
    float* dst = part + ((size_t)(qh0 + h) * max_splits + split) * (HD + 2);
    dst[dd] = o;
    if (dd == 0) {
      dst[HD] = mrun[h];
      dst[HD + 1] = lrun[h];
    }
  }
}

// One query head per block (the short form's blocks): the same partials
// as k_attention, with no K/V staging in LDS.  Thread (column c, row group
// r) holds dims 4c .. 4c + 3 of rows r, r + RPI, ... of each 64-position
// sub-tile in registers, with its own 4 dims of the rotated query and new
// key; a row's score is the sum over the NC4 lanes of its row group.  Each
// wave keeps its own running max, sum and output over its rows (a wave
// whose rows are all masked so far keeps m = -inf and adds nothing), and
// the waves' partials merge once at the end: one barrier per launch
// instead of five per sub-tile.
template <int HD, int NT>
__global__ __launch_bounds__(NT) void k_attention1(const float* __restrict__ q, const float* __restrict__ kn,
                                                    const float* __restrict__ vn, const float* __restrict__ cs,
                                                    float* __restrict__ kc, float* __restrict__ vc, uint32_t nh,
                                                    uint32_t nkv, uint32_t max_splits, uint32_t max_ctx, float scale,
                                                    float* __restrict__ part, const StepState* st, uint32_t cap,
                                                    uint32_t gq, uint32_t pre_all) {
  constexpr int C = ATT_CHUNK, NC4 = HD / 4, RPI = NT / NC4, LD = C / RPI, HALF = HD / 2, NW = NT / 64;
  __shared__ float wm[NW], wl[NW];
  __shared__ __align__(16) float wo[NW][HD];
  const uint32_t g = blockIdx.x, split = blockIdx.y, hz = blockIdx.z, qh = g * gq + hz;
  const size_t kvd = (size_t)nkv * HD;
  const int lc = threadIdx.x % NC4, lr = threadIdx.x / NC4, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // the first sub-tile's rows before the position is known (see k_attention)
  float4 kr[LD], vr[LD];
  if (hz == 0 || pre_all) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const uint32_t tp = split * C + lr + RPI * i;
      const size_t off = (size_t)(tp < max_ctx ? tp : 0) * kvd + (size_t)g * HD + 4 * lc;
      kr[i] = *(const float4*)(kc + off);
      vr[i] = *(const float4*)(vc + off);
    }
  }
  // this thread's dims of the rotated query and key (model.rs:193-217; the
  // rotation pairs dim j with j + hd/2, no FMA contraction)
  const bool lo_half = 4 * lc < HALF;
  const int j0 = lo_half ? 4 * lc : 4 * lc - HALF;
  const float* qp = q + (size_t)qh * HD;
  const float* kp = kn + (size_t)g * HD;
  const float4 qa = *(const float4*)(qp + j0), qb = *(const float4*)(qp + j0 + HALF);
  const float4 ka = *(const float4*)(kp + j0), kb = *(const float4*)(kp + j0 + HALF);
  const float4 cc = *(const float4*)(cs + j0), sn = *(const float4*)(cs + HALF + j0);
  const float4 vnew = *(const float4*)(vn + (size_t)g * HD + 4 * lc);
  auto rot = [&](float a, float b, float c, float s) {
    return lo_half ? __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s)) : __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
  };
  const float4 q4 = make_float4(rot(qa.x, qb.x, cc.x, sn.x), rot(qa.y, qb.y, cc.y, sn.y), rot(qa.z, qb.z, cc.z, sn.z),
                                rot(qa.w, qb.w, cc.w, sn.w));
  const float4 k4 = make_float4(rot(ka.x, kb.x, cc.x, sn.x), rot(ka.y, kb.y, cc.y, sn.y), rot(ka.z, kb.z, cc.z, sn.z),
                                rot(ka.w, kb.w, cc.w, sn.w));
  const uint32_t pos = st->pos, T = pos + 1;
  const uint32_t len = attention_split_len(T, cap), t0 = split * len;
  if (t0 >= T) return;
  const uint32_t ns = (T + len - 1) / len, tend = min(t0 + len, T), nsub = (tend - t0 + C - 1) / C;
  if (split == ns - 1 && hz == 0 && lr == 0) {  // KvCache::append of head g at pos
    *(float4*)(kc + (size_t)pos * kvd + (size_t)g * HD + 4 * lc) = k4;
    *(float4*)(vc + (size_t)pos * kvd + (size_t)g * HD + 4 * lc) = vnew;
  }
  auto load_tile = [&](uint32_t k) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const uint32_t tp = t0 + k * C + lr + RPI * i;
      const size_t off = (size_t)((tp < tend && tp != pos) ? tp : 0) * kvd + (size_t)g * HD + 4 * lc;
      kr[i] = *(const float4*)(kc + off);
      vr[i] = *(const float4*)(vc + off);
    }
  };
  if (len != C || (hz != 0 && !pre_all)) load_tile(0);
  float m = -INFINITY, l = 0.f;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t k = 0; k < nsub; ++k) {
    float sc[LD];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const uint32_t tp = t0 + k * C + lr + RPI * i;
      const bool cur = tp == pos;
      const float4 kk = cur ? k4 : kr[i];
      if (cur) vr[i] = vnew;
      float d = kk.x * q4.x + kk.y * q4.y + kk.z * q4.z + kk.w * q4.w;
      d = group_reduce<NC4>(d);
      sc[i] = tp < tend ? d * scale : -INFINITY;  // model.rs:397
      mx = fmaxf(mx, sc[i]);
    }
    const float mn = fmaxf(m, wave_max(mx));
    if (mn != -INFINITY) {  // wave-uniform
      const float c = expf(m - mn);
      float ls = 0.f;
      float4 os = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int i = 0; i < LD; ++i) {
        const float e = expf(sc[i] - mn);
        ls += e;
        os.x += e * vr[i].x;
        os.y += e * vr[i].y;
        os.z += e * vr[i].z;
        os.w += e * vr[i].w;
      }
      // the wave's other row groups (same dims, other rows)
#pragma unroll
      for (int sh = NC4; sh < 64; sh *= 2) {
        ls += __shfl_xor(ls, sh, 64);
        os.x += __shfl_xor(os.x, sh, 64);
        os.y += __shfl_xor(os.y, sh, 64);
        os.z += __shfl_xor(os.z, sh, 64);
        os.w += __shfl_xor(os.w, sh, 64);
      }
      l = l * c + ls;
      o = make_float4(o.x * c + os.x, o.y * c + os.y, o.z * c + os.z, o.w * c + os.w);
      m = mn;
    }
    if (k + 1 < nsub) load_tile(k + 1);
  }
  if (lane < NC4) *(float4*)(&wo[wave][4 * lc]) = o;
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
  __syncthreads();
  if (threadIdx.x < HD) {
    const int dd = threadIdx.x;
    float M = wm[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, wm[w]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float e = wm[w] == -INFINITY ? 0.f : expf(wm[w] - M);
      O += wo[w][dd] * e;
      L += wl[w] * e;
    }
    float* dst = part + ((size_t)qh * max_splits + split) * (HD + 2);
    dst[dd] = O;
    if (dd == 0) {
      dst[HD] = M;
      dst[HD + 1] = L;
    }
  }
}

size_t attention_part_floats(uint32_t nh, uint32_t hd, uint32_t max_ctx) {
  return (size_t)nh * attention_splits(max_ctx, ATTENTION_MAX_SPLITS_LONG) * (hd + 2);
}

// Long-context merge of the splits of one query head (block h): thread
// (d, q) of the 4 HD threads holds dimension d of the splits q, q + 4, ...
// Its o loads go out first, over all ms splits of the buffer (in bounds;
// those past the step's count are not used), so they do not wait for the
// position; the splits' maxima and sums go through LDS; each thread sums
// its splits with the weights e^(m_s - M), and the four partial sums of a
// dimension are added in q order.
template <int HD>
__global__ __launch_bounds__(4 * HD) void k_attn_merge(const float* __restrict__ part, float* __restrict__ out,
                                                       uint32_t ms, const StepState* st) {
  constexpr int NQ = 4, PER = ATTENTION_MAX_SPLITS_LONG / NQ;
  __shared__ float msl[2 * ATTENTION_MAX_SPLITS_LONG];
  __shared__ float po[NQ][HD], pl[NQ];
  const uint32_t h = blockIdx.x, d = threadIdx.x % HD, q = threadIdx.x / HD;
  const float* base = part + (size_t)h * ms * (HD + 2);
  float ov[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t sp = q + NQ * i;
    ov[i] = sp < ms ? base[(size_t)sp * (HD + 2) + d] : 0.f;
  }
  const uint32_t T = st->pos + 1, len = attention_split_len(T, ATTENTION_MAX_SPLITS_LONG);
  const uint32_t ns = (T + len - 1) / len;
  for (uint32_t sp = threadIdx.x; sp < ns; sp += NQ * HD) {
    msl[2 * sp] = base[(size_t)sp * (HD + 2) + HD];
    msl[2 * sp + 1] = base[(size_t)sp * (HD + 2) + HD + 1];
  }
  __syncthreads();
  float M = -INFINITY;
  for (uint32_t sp = 0; sp < ns; ++sp) M = fmaxf(M, msl[2 * sp]);
  float o = 0.f, L = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t sp = q + NQ * i;
    if (sp < ns) {
      const float e = expf(msl[2 * sp] - M);  // model.rs:371-438, evaluated split-wise
      L += e * msl[2 * sp + 1];
      o += e * ov[i];
    }
  }
  po[q][d] = o;
  if (d == 0) pl[q] = L;
  __syncthreads();
  if (q == 0) {
    float O = po[0][d], Lt = pl[0];
#pragma unroll
    for (int k = 1; k < NQ; ++k) {
      O += po[k][d];
      Lt += pl[k];
    }
    out[(size_t)h * HD + d] = Lt > 0.f ? O / Lt : 0.f;
  }
}

hipError_t launch_attn_merge(const float* part, float* out, uint32_t nh, uint32_t hd, uint32_t max_ctx,
                             const StepState* st, hipStream_t s) {
  const uint32_t ms = attention_splits(max_ctx, ATTENTION_MAX_SPLITS_LONG);
  if (hd == 128)
    hipLaunchKernelGGL(k_attn_merge<128>, dim3(nh), dim3(4 * 128), 0, s, part, out, ms, st);
  else if (hd == 64)
    hipLaunchKernelGGL(k_attn_merge<64>, dim3(nh), dim3(4 * 64), 0, s, part, out, ms, st);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// threads per one-head attention block (64 positions per sub-tile)
constexpr int ATT1_THREADS = 256;
template <int HD, int GQ>
static void att_go(dim3 grid, hipStream_t s, const float* q, const float* k, const float* v, const float* cs,
                   float* kc, float* vc, uint32_t nh, uint32_t nkv, uint32_t ms, uint32_t max_ctx, float scale,
                   float* part, const StepState* st, uint32_t cap, uint32_t gq, uint32_t pre_all) {
  if constexpr (GQ == 1)
    hipLaunchKernelGGL((k_attention1<HD, ATT1_THREADS>), grid, dim3(ATT1_THREADS), 0, s, q, k, v, cs, kc, vc, nh, nkv,
                       ms, max_ctx, scale, part, st, cap, gq, pre_all);
  else
    hipLaunchKernelGGL((k_attention<HD, GQ>), grid, dim3(256), 0, s, q, k, v, cs, kc, vc, nh, nkv, ms, max_ctx, scale,
                       part, st, cap, gq, pre_all);
}

template <int HD>
static hipError_t att_gq(uint32_t hpb, dim3 grid, hipStream_t s, const float* q, const float* k, const float* v,
                         const float* cs, float* kc, float* vc, uint32_t nh, uint32_t nkv, uint32_t ms,
                         uint32_t max_ctx, float scale, float* part, const StepState* st, uint32_t cap, uint32_t gq,
                         uint32_t pre_all) {
  switch (hpb) {
#define FRN_ATT_GQ(n) \
  case n: att_go<HD, n>(grid, s, q, k, v, cs, kc, vc, nh, nkv, ms, max_ctx, scale, part, st, cap, gq, pre_all); break;
    FRN_ATT_GQ(1) FRN_ATT_GQ(2) FRN_ATT_GQ(3) FRN_ATT_GQ(4) FRN_ATT_GQ(5) FRN_ATT_GQ(6) FRN_ATT_GQ(7) FRN_ATT_GQ(8)
#undef FRN_ATT_GQ
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

#ifndef FRN_ATT_HEADS_PER_BLOCK
#define FRN_ATT_HEADS_PER_BLOCK 1
#endif
// Query heads per attention block.  The short form (at most 16 splits of
// one 64-position sub-tile each, below 1024 positions) runs few blocks, each
// busy with the scores, softmax and P.V of its whole group: splitting the
// group over blocks shortens that chain.  Measured at 1.5B (6 heads per kv
// head, 128-383 positions): 6.73 us per launch with the whole group, 5.67
// with 3 heads, 5.25 with 2, 4.90 with 1 (decode 1024 -> 1103 tokens/s).
// The long form already fills the GPU with splits; there, head groups would
// multiply the KV rows every XCD streams.
uint32_t attention_heads_per_block(uint32_t gq, uint32_t cap) {
  if (cap != ATTENTION_MAX_SPLITS) return gq;
  return gq < FRN_ATT_HEADS_PER_BLOCK ? gq : FRN_ATT_HEADS_PER_BLOCK;
}

bool attention_supported(uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim) {
  return n_kv_heads && n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= 8 && (head_dim == 64 || head_dim == 128);
}


hipError_t launch_attention(const float* q, const float* k, const float* v, const float* cs, float* kc, float* vc,
                            uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_ctx, float scale, float* part,
                            const StepState* st, uint32_t cap, uint32_t live, hipStream_t s) {
  if (!attention_supported(nh, nkv, hd) || (cap != ATTENTION_MAX_SPLITS && cap != ATTENTION_MAX_SPLITS_LONG))
    return hipErrorInvalidValue;
  const uint32_t ms = attention_splits(max_ctx, cap), gq = nh / nkv, hpb = attention_heads_per_block(gq, cap);
  if (live && (cap != ATTENTION_MAX_SPLITS || live > ms)) return hipErrorInvalidValue;
  dim3 grid(nkv, live ? live : ms, (gq + hpb - 1) / hpb);
  const uint32_t pre = live ? 1u : 0u;
  if (hd == 128)
    return att_gq<128>(hpb, grid, s, q, k, v, cs, kc, vc, nh, nkv, ms, max_ctx, scale, part, st, cap, gq, pre);
  return att_gq<64>(hpb, grid, s, q, k, v, cs, kc, vc, nh, nkv, ms, max_ctx, scale, part, st, cap, gq, pre);
}

// ---- step bookkeeping and argmax (generate.rs:69-77) ------------------------
// 1024 threads: max over the lm_head blocks' packed candidates (largest
// logit, then smallest row), then advance the position.
__global__ __launch_bounds__(1024) void k_step_end(StepState* st, const uint64_t* __restrict__ best,
                                                   uint32_t n_best, uint32_t* __restrict__ hist) {
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
      if (hist) hist[st->pos] = idx;
    }
  }
  if (threadIdx.x == 0) st->pos += 1;
}

hipError_t launch_step_end(StepState* st, const uint64_t* best, uint32_t n_best, uint32_t* hist, hipStream_t s) {
  hipLaunchKernelGGL(k_step_end, dim3(1), dim3(1024), 0, s, st, best, n_best, hist);
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
