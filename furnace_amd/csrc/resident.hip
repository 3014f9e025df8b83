// Resident decode on gfx950: the greedy token loop of generate.rs:110-136
// (forward_cached, model.rs:579-592, then argmax, generate.rs:69-77) for
// many positions in ONE persistent launch, one block per CU.
//
// MI355X has 8 XCDs of 32 CUs; each XCD has its own L2, and a value one CU
// stores is visible to the other CUs of its XCD through that L2 (an
// agent-scope load misses the L1 and finds it there), while CUs of other
// XCDs only see values written through to memory.  So the XCDs play the
// ranks of a tensor-parallel layer:
//  - XCD x owns query heads [nh x/8, nh (x+1)/8) (with their kv heads) and
//    FFN rows [f0, f1) (128-value units split evenly);
//  - q/k/v rows, attention, the o-proj over its heads' columns, gate/up rows
//    and the down projection over its FFN columns all run inside the XCD,
//    exchanging through its L2;
//  - the o-proj and down partial sums (one [hidden] vector per XCD) are the
//    only values that cross XCDs: CU c of every XCD sums rows
//    [c H/32, (c+1) H/32) of the eight partials in XCD order, adds the
//    residual, and republishes the rows in its own XCD.
// Values travel as 8-byte (value, epoch) pairs: a reader knows a value is
// current from its epoch, so one round trip both waits and reads.  Every
// wait is bounded: a block that gives up raises ctl->abort and every block
// leaves the launch (the host reports the failure and falls back to the
// per-kernel step graphs).
//
// Per layer (model.rs:444-478), a block's phases:
//  A  rmsnorm(x) -> q|k|v rows of the XCD's heads (+bias)    -> local
//  B  RoPE, KV append, attention of one (head, split) job   -> local
//  C  merge the splits -> o-proj partial over the XCD's head columns -> cross
//  D  x' = x + sum of the 8 partials, this CU's rows        -> local
//  E  rmsnorm(x') -> gate/up rows of the XCD's FFN slice, SwiGLU -> local
//  F  down partial over the XCD's FFN columns               -> cross
//  G  x'' = x' + sum of the 8 partials, this CU's rows      -> local
// then, per token: rmsnorm + lm_head rows of the block (all 256 blocks) +
// argmax candidates (cross), and every block reduces them to the next id.
// A wave issues its first weight loads before it waits for its phase's
// input, so the weights stream while the exchange settles.
#include "formats.hpp"
#include "items.hpp"
#include "kernels.hpp"
#include "resident.hpp"

#include <type_traits>

namespace frn {
namespace {

constexpr int RT = (int)RES_THREADS, NWAVE = RT / 64;
constexpr uint32_t POLL_LIMIT = 1u << 18;  // polls per wait (each >= ~0.3 us): a wait gives up after ~0.1-0.3 s
constexpr uint32_t MAX_SPLIT_PAIRS = 32 * (128 + 2);  // heads x splits x (hd + 2) a block merges

__device__ __forceinline__ uint32_t hw_xcc() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 0xFu;
}
// Pointers read out of the argument struct are generic; the exchange
// helpers access them through the global address space, so the compiler
// emits global_* (not flat_*) instructions, which count only against vmcnt.
#if defined(__HIP_DEVICE_COMPILE__)
#define GAS __attribute__((address_space(1)))
#else
#define GAS
#endif
template <class T>
__device__ __forceinline__ GAS T* gl(T* p) {
  return (GAS T*)p;
}
__device__ __forceinline__ uint64_t pack(uint32_t bits, uint32_t ep) { return ((uint64_t)ep << 32) | bits; }
__device__ __forceinline__ uint64_t ld_pair(const uint2* p) {
  return __hip_atomic_load((const GAS uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load((const GAS uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// within the XCD: the store stays in the XCD's L2
__device__ __forceinline__ void st_local(uint2* p, float v, uint32_t ep) {
  __hip_atomic_store((GAS uint64_t*)p, pack(__float_as_uint(v), ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// to other XCDs: written through to memory
__device__ __forceinline__ void st_cross_bits(uint2* p, uint32_t bits, uint32_t ep) {
  __hip_atomic_store((GAS uint64_t*)p, pack(bits, ep), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_cross(uint2* p, float v, uint32_t ep) { st_cross_bits(p, __float_as_uint(v), ep); }

__device__ __forceinline__ void raise_abort(ResCtl* ctl, uint32_t code) {
  uint32_t expect = 0;
  __hip_atomic_compare_exchange_strong((GAS uint32_t*)&ctl->err, &expect, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store((GAS uint32_t*)&ctl->abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave 0 of a block is its communication wave: it alone polls exchange
// buffers, so the only loads in its queue are polls (a wave's loads
// complete in order, and the compute waves keep weight loads in flight).
//
// poll_wave: wave 0 waits for pairs src(i), i < n, to carry epoch ep and
// writes their 32-bit payloads to dst[i] (LDS).  pre() runs once, right
// after the first round of loads is issued and before its values are
// checked.  Returns false when the wait gave up (then ctl->abort is set).
struct NoPre {
  __device__ __forceinline__ void operator()() const {}
};
template <class Src, class Pre = NoPre>
__device__ __forceinline__ bool poll_wave(uint32_t n, Src&& src, uint32_t ep, uint32_t* dst, ResCtl* ctl,
                                          uint32_t where, Pre&& pre = Pre()) {
  constexpr int K = 24;
  const uint32_t lane = threadIdx.x & 63;
  bool ok = true, pre_done = false;
  for (uint32_t i0 = 0; (i0 < n || !pre_done) && ok; i0 += K * 64) {
    uint32_t pend = 0;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (i0 + lane + 64 * k < n) pend |= 1u << k;
    for (uint32_t it = 0;; ++it) {
      uint64_t v[K];
#pragma unroll
      for (int k = 0; k < K; ++k) v[k] = (pend >> k) & 1u ? ld_pair(src(i0 + lane + 64 * k)) : 0ull;
      if (!pre_done) {
        __builtin_amdgcn_sched_barrier(0);
        pre();
        __builtin_amdgcn_sched_barrier(0);
        pre_done = true;
      }
#pragma unroll
      for (int k = 0; k < K; ++k)
        if (((pend >> k) & 1u) && (uint32_t)(v[k] >> 32) == ep) {
          dst[i0 + lane + 64 * k] = (uint32_t)v[k];
          pend &= ~(1u << k);
        }
      if (!__any(pend != 0)) break;
      if (it >= POLL_LIMIT || ((it & 255u) == 255u && ld_agent(&ctl->abort))) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  if (!ok && lane == 0) raise_abort(ctl, RES_ERR_WAIT | where);
  return ok;
}

// poll: the communication wave polls (poll_wave), the compute waves run
// pre() (their first weight loads); then the block meets at a barrier that
// publishes dst.  `carry`: a failure of an earlier wave-0-only step.  False
// for the whole block when a wait gave up.
template <class Src, class Pre = NoPre>
__device__ __forceinline__ bool poll(uint32_t n, Src&& src, uint32_t ep, uint32_t* dst, ResCtl* ctl, uint32_t where,
                                     Pre&& pre = Pre(), bool carry = true) {
  bool ok = carry;
  if (threadIdx.x < 64) {
    if (ok) ok = poll_wave(n, src, ep, dst, ctl, where, pre);
  } else {
    pre();
  }
  return __syncthreads_and(ok);
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = group_reduce<64>(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < NWAVE; ++i) r += red[i];
  __syncthreads();
  return r;
}

// K values (LDS, f32; K <= 4096, a multiple of 32) -> the int8 digit form of
// XLds (formats.hpp) at pl, after rmsnorm with gain nw (tensor.rs:164-185)
// when nw is given.  Thread t owns the 8-value groups t + RT i; the 4
// threads of a 32-value chunk are adjacent lanes.  Collective.
__device__ __forceinline__ void stage(const float* src, uint32_t K, const GAS float* nw, float eps, uint8_t* pl, float* red) {
  constexpr int NG = RES_MAX_K / 8 / RT;
  float v[NG][8];
  float4 wa[NG], wb[NG];
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    const uint32_t u = threadIdx.x + RT * i;
    const bool live = u < K / 8;
    wa[i] = wb[i] = make_float4(1.f, 1.f, 1.f, 1.f);
    if (nw && live) {
      wa[i] = ((const GAS float4*)nw)[2 * u];
      wb[i] = ((const GAS float4*)nw)[2 * u + 1];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) v[i][j] = live ? src[8 * u + j] : 0.f;
  }
  if (nw) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[i][j] * v[i][j];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const float w[8] = {wa[i].x, wa[i].y, wa[i].z, wa[i].w, wb[i].x, wb[i].y, wb[i].z, wb[i].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = v[i][j] * inv * w[j];
    }
  }
#pragma unroll
  for (int i = 0; i < NG; ++i) {
    if (RT * i >= K / 8) break;  // block-uniform: no thread has group i
    const uint32_t u = threadIdx.x + RT * i;
    const bool live = u < K / 8;
    float amax = 0.f, xsum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      amax = fmaxf(amax, fabsf(v[i][j]));
      xsum += v[i][j];
    }
    amax = group_reduce<4>(amax, OpMax());
    // x ~= s (d0 + d1/128 + d2/16384) per 32-value chunk, |error| <= max|x| 2^-22
    const float inv_s = amax > 0.f ? 127.0f * __builtin_amdgcn_rcpf(amax) : 0.f;
    const float cs = amax > 0.f ? __builtin_amdgcn_rcpf(inv_s) * (1.0f / 16384.0f) : 0.f;
    uint32_t w0[2] = {0, 0}, w1[2] = {0, 0}, w2[2] = {0, 0};
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float t = v[i][j] * inv_s;
      const float r0 = rintf(t), e0 = (t - r0) * 128.0f;
      const float r1 = rintf(e0), e1 = (e0 - r1) * 128.0f;
      const float r2 = rintf(e1);
      const int d0 = (int)r0, d1 = (int)r1, d2 = (int)r2;
      w0[j >> 2] |= (uint32_t)(d0 & 0xFF) << (8 * (j & 3));
      w1[j >> 2] |= (uint32_t)(d1 & 0xFF) << (8 * (j & 3));
      w2[j >> 2] |= (uint32_t)(d2 & 0xFF) << (8 * (j & 3));
      s0 += d0;
      s1 += d1;
      s2 += d2;
    }
    xsum = group_reduce<2>(xsum);
    s0 = group_reduce<2>(s0);
    s1 = group_reduce<2>(s1);
    s2 = group_reduce<2>(s2);
    if (live) {
      const uint32_t n16 = K / 16, c = u >> 1, off = 16u * swz(c, n16) + 8u * (u & 1);
      *(uint2*)(pl + off) = make_uint2(w0[0], w0[1]);
      *(uint2*)(pl + K + off) = make_uint2(w1[0], w1[1]);
      *(uint2*)(pl + 2 * K + off) = make_uint2(w2[0], w2[1]);
      if ((u & 1) == 0)
        *(float4*)(pl + 3 * K + 16u * swz(c, n16)) =
            make_float4(cs, xsum, __int_as_float(-32 * s0), __int_as_float(-32 * (128 * s1 + s2)));
    }
  }
  __syncthreads();
}

// Items of a column range [c0, c0 + n) of a row (32-value items for the
// K-quants, 64-value block pairs for Q8_0).
__device__ __forceinline__ uint32_t item_of(uint32_t t, uint32_t c) { return t == T_Q8_0 ? c / 64 : c / 32; }

// A wave's GEMV rows: units of G = 64/LPR rows of [row0, row0 + nrows) of a
// matrix, the wave's units u0, u0 + us, ...; lane group gl of a row covers
// items it0 + (s BI + j) LPR + gl of step s.  The steps of all the wave's
// units form one pipeline of depth 2 (step f + 1's loads in flight while
// step f is computed).  R = 2: row pairs of two matrices (gate, up).
template <uint32_t T, int LPR, int BI, int R>
struct Pipe {
  using F = Fmt<T>;
  using Raw = typename F::Raw;
  static constexpr int B = BI * R, G = 64 / LPR;
  Raw ra[B], rb[B];
  float acc[R];
  rsrc_t rw, rw2;
  uint32_t row0, nrows, rbytes, it0, nit, cb, S, us, iu, is, cu, cs, nsteps, gl, g;

  __device__ __forceinline__ void setup(const uint8_t* w, const uint8_t* w2, uint32_t mrows, uint32_t row_bytes,
                                        uint32_t r0, uint32_t nr, uint32_t i0, uint32_t ni, uint32_t cbase,
                                        uint32_t u0, uint32_t ustride) {
    const uint32_t lane = threadIdx.x & 63;
    gl = lane % LPR;
    g = lane / LPR;
    rw = make_rsrc(w, mrows * row_bytes);
    rw2 = make_rsrc(R == 2 ? w2 : w, mrows * row_bytes);
    row0 = r0;
    nrows = nr;
    rbytes = row_bytes;
    it0 = i0;
    nit = ni;
    cb = cbase;
    S = (nit + LPR * BI - 1) / (LPR * BI);
    const uint32_t nu = (nrows + G - 1) / G;
    nsteps = u0 < nu ? (nu - u0 + ustride - 1) / ustride * S : 0;
    iu = cu = u0;
    is = cs = 0;
    us = ustride;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
  }
  __device__ __forceinline__ uint32_t row_off(uint32_t unit) const {
    const uint32_t r = unit * G + g;
    return r < nrows ? (row0 + r) * rbytes : BUF_INVALID;
  }
  __device__ __forceinline__ void adv(uint32_t& u, uint32_t& s) const {
    if (++s == S) {
      s = 0;
      u += us;
    }
  }
  __device__ __forceinline__ void issue(Raw (&raw)[B]) {
    const uint32_t ro = row_off(iu);
#pragma unroll
    for (int j = 0; j < BI; ++j) {
      const uint32_t it = (is * BI + j) * LPR + gl;
      const uint32_t o = it < nit ? ro : BUF_INVALID;
      raw[j * R] = F::load(rw, o, (int)(it0 + it), true);
      if constexpr (R == 2) raw[j * R + 1] = F::load(rw2, o, (int)(it0 + it), true);
    }
    adv(iu, is);
  }
  template <class Out>
  __device__ __forceinline__ void consume(Raw (&raw)[B], const XLds& X, Out&& out) {
    const uint32_t ro = row_off(cu), row = cu * G + g;
#pragma unroll
    for (int j = 0; j < BI; ++j) {
      const uint32_t it = (cs * BI + j) * LPR + gl;
      const bool ok = it < nit && ro != BUF_INVALID;
      const int itc = (int)(it0 + (ok ? it : 0u));  // masked items: zero weights, a valid chunk of x
      XC xc[F::NC];
#pragma unroll
      for (int i = 0; i < F::NC; ++i) xc[i] = X.chunk(F::chunk(itc, i, true) - cb);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += F::dot(raw[j * R + r], ro, nullptr, itc, xc, X, true);
    }
    if (cs + 1 == S) {
      const float a0 = group_reduce<LPR>(acc[0]);
      const float a1 = R == 2 ? group_reduce<LPR>(acc[R - 1]) : 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.f;
      if (gl == 0 && row < nrows) out(row0 + row, a0, a1);
    }
    adv(cu, cs);
  }
  __device__ __forceinline__ void first() {
    if (nsteps) issue(ra);
  }
  // deep: step f + 1's loads in flight while step f is computed; else one
  // step at a time (fewer bytes in flight per wave)
  template <class Out>
  __device__ __forceinline__ void run(const XLds& X, Out&& out, bool deep = true) {
    if (!deep) {
      for (uint32_t f = 0; f < nsteps; ++f) {
        consume(ra, X, out);
        if (f + 1 < nsteps) issue(ra);
      }
      return;
    }
    for (uint32_t f = 0; f < nsteps; f += 2) {
      if (f + 1 < nsteps) issue(rb);
      consume(ra, X, out);
      if (f + 1 >= nsteps) break;
      if (f + 2 < nsteps) issue(ra);
      consume(rb, X, out);
    }
  }
};

// One matrix row range of a phase.  Its units are numbered from ubase in
// the phase's list; unit U goes to wave U mod nw of the wave set.
struct Seg {
  const uint8_t *w, *w2;
  uint32_t type, mrows, row_bytes, row0, nrows, it0, nit, cb, ubase;
};

// The GEMV part of a phase: each wave issues the first step of its first
// unit, then the block waits for the phase input (wait(): collective,
// returns false when the wait gave up), then the waves run their units.
// out(segment, row, a0, a1).  Segments of format T1 (!= T0) use a second
// pipeline; T1 == T0 for single-format phases.
template <uint32_t T0, uint32_t T1, int LPR, int BI, int R, int NSEG, class Wait, class Out>
__device__ __forceinline__ bool gemv_phase(const Seg (&sg)[NSEG], uint32_t wx, uint32_t nw, const XLds& X, Wait&& wait, Out&& out,
                                           bool early, bool deep = true) {
  constexpr uint32_t G = 64 / LPR;
  constexpr int BI0 = T0 == T_Q8_0 && BI > 2 ? 2 : BI, BI1 = T1 == T_Q8_0 && BI > 2 ? 2 : BI;
  Pipe<T0, LPR, BI0, R> p0;
  Pipe<T1, LPR, BI1, R> p1;
  uint32_t u0[NSEG], nu[NSEG];
  int first = -1;
#pragma unroll
  for (int i = 0; i < NSEG; ++i) {
    nu[i] = (sg[i].nrows + G - 1) / G;
    u0[i] = wx == ~0u ? ~0u : (wx + nw - sg[i].ubase % nw) % nw;  // ~0u: a wave without units
    if (first < 0 && u0[i] < nu[i]) first = i;
  }
  auto start = [&](const Seg& s, uint32_t u) __attribute__((always_inline)) {
    if (T0 == T1 || s.type == T0) {
      p0.setup(s.w, s.w2, s.mrows, s.row_bytes, s.row0, s.nrows, s.it0, s.nit, s.cb, u, nw);
      p0.first();
    } else {
      p1.setup(s.w, s.w2, s.mrows, s.row_bytes, s.row0, s.nrows, s.it0, s.nit, s.cb, u, nw);
      p1.first();
    }
  };
  auto pre = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NSEG; ++i)
      if (early && i == first) start(sg[i], u0[i]);
  };
  if (!wait(pre)) return false;
#pragma unroll
  for (int i = 0; i < NSEG; ++i) {
    if (first < 0 || i < first || u0[i] >= nu[i]) continue;
    if (i != first || !early) start(sg[i], u0[i]);
    auto o = [&](uint32_t row, float a0, float a1) __attribute__((always_inline)) { out(i, row, a0, a1); };
    if (T0 == T1 || sg[i].type == T0)
      p0.run(X, o, deep);
    else
      p1.run(X, o, deep);
  }
  return true;
}

// Calls body(integral_constant<T>) with the K-quant or Q8_0 format t
// (block-uniform, so the phase's barriers line up).
template <uint32_t FS, class Body>
__device__ __forceinline__ bool by_type(uint32_t t, Body&& body) {
  if constexpr (FS == RES_FS_KQUANT) {
    if (t == T_Q4_K) return body(std::integral_constant<uint32_t, T_Q4_K>());
    return body(std::integral_constant<uint32_t, T_Q6_K>());
  } else {
    return body(std::integral_constant<uint32_t, T_Q8_0>());
  }
}

// LDS carve-up (floats): x of the current layer [RES_MAX_K] | staging input
// [RES_MAX_K] | digit planes [4 RES_MAX_K bytes] | reductions [64] | this CU's
// rows of x' [128] | the 8 partials of those rows [8 x 128] | attention job
// scratch and split merge | per-wave argmax keys
constexpr size_t LDS_FLOATS = 2 * RES_MAX_K + RES_MAX_K + 64 + 128 + 8 * 128 + MAX_SPLIT_PAIRS + 2048 + 2 * NWAVE;
static_assert(LDS_FLOATS * 4 <= RES_LDS_BYTES, "LDS budget");

// One attention job: query head h, positions [t0, t1) of 0..pos
// (model.rs:371-438 evaluated split-wise), hd = HD.  q of h and k, v of kv
// head g come from the XCD's q|k|v pairs; RoPE at pos (model.rs:193-217,
// the host's cos|sin row; no FMA contraction, so the rotation is bit-exact);
// write_kv: KvCache::append of head g (model.rs:346-356), written through
// for the other XCDs.  Writes the split's partial (o[HD], m, l).
template <int HD>
__device__ __forceinline__ bool attn_job(const ResArgs& a, uint32_t l, uint32_t pos, uint32_t h, uint32_t g, uint32_t t0,
                         uint32_t t1, const uint2* qkv, uint32_t ep_in, uint2* dst, uint32_t ep_out, bool write_kv,
                         float* sm, uint32_t where) {
  constexpr int HALF = HD / 2, NPART = RT / HD, TPP = RT / 64, DPT = HD / TPP;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  float* raw = sm;            // [3 HD] q, k, v as produced
  float* qr = raw + 3 * HD;   // [HD] rotated q
  float* kr = qr + HD;        // [HD] rotated k
  float* ps = kr + HD;        // [64] scores, then probabilities
  float* osum = ps + 64;      // [RT] P.V parts
  float* mls = osum + RT;     // running max, sum, rescale
  const uint32_t qo = h * HD, ko = a.nh * HD + g * HD, vo = (a.nh + a.nkv) * HD + g * HD;
  const size_t kvd = (size_t)a.nkv * HD, lo = (size_t)l * a.max_ctx * kvd;
  float* kc = a.kc + lo;
  float* vc = a.vc + lo;
  // cached rows (< pos) through agent-scope buffer loads.  They do not
  // depend on this step, so the first tile's go out before the wait for
  // q, k, v; each later tile's while the previous one is scored.
  const uint32_t cbytes = (uint32_t)(a.max_ctx * kvd * 4);
  const rsrc_t rk = make_rsrc(kc, cbytes), rv = make_rsrc(vc, cbytes);
  const uint32_t p = tid / TPP, sub = tid % TPP, d = tid % HD, part = tid / HD;
  struct Tile {
    u32x4 k[DPT / 4];    // dims [sub DPT, +DPT) of the K row of position tb + p
    float v[64 / NPART];  // dim d of the V rows of positions tb + part + NPART i
  };
  auto load_tile = [&](uint32_t tb, Tile& T) __attribute__((always_inline)) {
    const uint32_t tp = tb + p;
    const uint32_t off = tp < t1 && tp < pos ? (uint32_t)(((size_t)tp * kvd + (size_t)g * HD + sub * DPT) * 4) : BUF_INVALID;
#pragma unroll
    for (int i = 0; i < DPT / 4; ++i)
      T.k[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(off == BUF_INVALID ? off : off + 16 * i), 0, 16);
#pragma unroll
    for (int k = 0; k < 64 / NPART; ++k) {
      const uint32_t tq = tb + part + NPART * k;
      const uint32_t o = tq < t1 && tq < pos ? (uint32_t)(((size_t)tq * kvd + (size_t)g * HD + d) * 4) : BUF_INVALID;
      T.v[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, (int)o, 0, 16));
    }
  };
  Tile cur;
  if (!poll(
          3 * HD, [&](uint32_t i) __attribute__((always_inline)) { return qkv + (i < HD ? qo + i : i < 2 * HD ? ko + i - HD : vo + i - 2 * HD); },
          ep_in, (uint32_t*)raw, a.ctl, where, [&]() __attribute__((always_inline)) { load_tile(t0, cur); }))
    return false;
  const GAS float* cs = gl(a.rope) + (size_t)pos * HD;
  if (tid < HD) {
    const int j = tid % HALF;
    const float* src = tid < HALF ? raw : raw + HD;
    float* o = tid < HALF ? qr : kr;
    const float x0 = src[j], x1 = src[j + HALF], c = cs[j], sn = cs[HALF + j];
    o[j] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
    o[j + HALF] = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
  }
  if (tid == 0) {
    mls[0] = -INFINITY;
    mls[1] = 0.f;
  }
  __syncthreads();
  const float* vr = raw + 2 * HD;
  if (write_kv && tid < 2 * HD) {
    // written through for the other XCDs; the wait before this block's
    // next exchange store (the next poll) orders it before that store
    const uint32_t dd = tid % HD;
    float* q = (tid < HD ? kc : vc) + (size_t)pos * kvd + (size_t)g * HD + dd;
    __hip_atomic_store((GAS uint32_t*)q, __float_as_uint(tid < HD ? kr[dd] : vr[dd]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  float acc = 0.f;
  for (uint32_t tb = t0; tb < t1; tb += 64) {
    Tile nxt;
    if (tb + 64 < t1) load_tile(tb + 64, nxt);
    {  // scores of positions tb + p: TPP threads per position, DPT dims each
      const uint32_t tp = tb + p;
      const bool valid = tp < t1, now = tp == pos;
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < DPT / 4; ++i) {
        float4 kk = make_float4(__uint_as_float(cur.k[i].x), __uint_as_float(cur.k[i].y), __uint_as_float(cur.k[i].z),
                                __uint_as_float(cur.k[i].w));
        if (now) kk = ((const float4*)(kr + sub * DPT))[i];
        const float4 qq = ((const float4*)(qr + sub * DPT))[i];
        s += kk.x * qq.x + kk.y * qq.y + kk.z * qq.z + kk.w * qq.w;
      }
      s = group_reduce<TPP>(s);
      if (sub == 0) ps[p] = valid ? s * a.scale : -INFINITY;  // model.rs:397
    }
    __syncthreads();
    if (tid < 64) {  // running softmax (tensor.rs:188-203, split-wise)
      const float v = ps[lane];
      const float mo = mls[0], mn = fmaxf(mo, group_reduce<64>(v, OpMax()));
      const float e = expf(v - mn);
      ps[lane] = e;
      const float lt = group_reduce<64>(e);
      if (lane == 0) {
        const float c = expf(mo - mn);
        mls[2] = c;
        mls[1] = mls[1] * c + lt;
        mls[0] = mn;
      }
    }
    __syncthreads();
    {  // P.V: thread (d, part) sums positions part, part + NPART, ... of the tile
      acc *= mls[2];
#pragma unroll
      for (int k = 0; k < 64 / NPART; ++k) {
        const uint32_t tq = tb + part + NPART * k;
        const float vv = tq == pos ? vr[d] : cur.v[k];
        acc += ps[part + NPART * k] * vv;
      }
    }
    __syncthreads();
    cur = nxt;
  }
  osum[tid] = acc;
  __syncthreads();
  if (tid < HD) {
    float o = 0.f;
#pragma unroll
    for (int q = 0; q < NPART; ++q) o += osum[q * HD + tid];
    st_local(dst + tid, o, ep_out);
  } else if (tid == HD) {
    st_local(dst + HD, mls[0], ep_out);
  } else if (tid == HD + 1) {
    st_local(dst + HD + 1, mls[1], ep_out);
  }
  __syncthreads();
  return true;
}

template <uint32_t FS>
__global__ __launch_bounds__(RES_THREADS, 1) void k_resident(const ResArgs* __restrict__ pa) {
  const ResArgs& a = *pa;  // in device memory: a kernel argument would be copied to scratch
  extern __shared__ __align__(16) float lds_f[];
  float* const s_xres = lds_f;
  float* const s_vin = s_xres + RES_MAX_K;
  uint8_t* const s_pl = (uint8_t*)(s_vin + RES_MAX_K);
  float* const s_red = (float*)(s_pl + 4 * RES_MAX_K);
  float* const s_rowv = s_red + 64;
  float* const s_ared = s_rowv + 128;
  float* const s_att = s_ared + 8 * 128;
  uint64_t* const s_keys = (uint64_t*)(s_att + MAX_SPLIT_PAIRS + 2048);
  __shared__ uint32_t s_rank, s_ok;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  ResCtl* ctl = a.ctl;
  const uint32_t xcd = hw_xcc();

  // ---- which CU of which XCD this block is; all 256 blocks present, 32 per XCD ----
  if (tid == 0) {
    uint32_t ok = xcd < RES_XCDS, r = 0;
    if (ok) r = __hip_atomic_fetch_add((GAS uint32_t*)&ctl->ticket[32 * xcd], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ok = ok && r < RES_CUS;
    for (uint32_t it = 0; ok; ++it) {
      uint32_t tot = 0;
      for (uint32_t y = 0; y < RES_XCDS; ++y) tot += ld_agent(&ctl->ticket[32 * y]);
      if (tot >= RES_BLOCKS) {
        for (uint32_t y = 0; y < RES_XCDS; ++y) ok = ok && ld_agent(&ctl->ticket[32 * y]) == RES_CUS;
        break;
      }
      if (it >= POLL_LIMIT || ld_agent(&ctl->abort)) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!ok) raise_abort(ctl, RES_ERR_LAYOUT);
    s_rank = r;
    s_ok = ok;
  }
  __syncthreads();
  if (!s_ok) return;
  const uint32_t rank = s_rank;

  // ---- this XCD's share ----
  const uint32_t H = a.H, HD = a.hd, gq = a.nh / a.nkv;
  const uint32_t h0 = a.nh * xcd / RES_XCDS, h1 = a.nh * (xcd + 1) / RES_XCDS, nhx = h1 - h0;
  const uint32_t g0 = h0 / gq, g1 = nhx ? (h1 - 1) / gq + 1 : g0;
  const uint32_t fu = a.F / 128, f0 = 128 * (fu * xcd / RES_XCDS), f1 = 128 * (fu * (xcd + 1) / RES_XCDS);
  const uint32_t RPC = (H + RES_CUS - 1) / RES_CUS, r0 = rank * RPC, nr = r0 < H ? min(RPC, H - r0) : 0u;
  // compute waves (1..NWAVE-1): the XCD's compute waves numbered blocks first
  // (wx), and within the block (cw); ~0u for the communication wave
  // (RES_OPT_ALL_WAVES: wave 0 computes as well; RES_OPT_LATE_WEIGHTS: a
  // phase's first weight loads go out after its input has arrived)
  const bool allw = a.opts & RES_OPT_ALL_WAVES, early = !(a.opts & RES_OPT_LATE_WEIGHTS),
             deep = !(a.opts & RES_OPT_SHALLOW);
  const uint32_t NCW = allw ? NWAVE : NWAVE - 1, w1 = allw ? wave : wave - 1;
  const uint32_t cw = allw || wave ? w1 : ~0u, wx = allw || wave ? w1 * RES_CUS + rank : ~0u;
  const uint32_t bglob = rank * RES_XCDS + xcd;
  const uint32_t RPB = (a.V + RES_BLOCKS - 1) / RES_BLOCKS, lr0 = bglob * RPB,
                 lnr = lr0 < a.V ? min(RPB, a.V - lr0) : 0u;
  const uint32_t smax = nhx ? min(RES_MAX_SPLITS, max(1u, 32u / nhx)) : 1u;
  const ResLayout& Y = a.lay;
  uint2* const ex_loc = a.loc;
  uint2* const ex_glb = a.glb;
  auto loc = [&](uint32_t par) __attribute__((always_inline)) { return ex_loc + (size_t)(xcd * 2 + par) * Y.loc_stride; };
  auto glb = [&](uint32_t par) __attribute__((always_inline)) { return ex_glb + (size_t)par * Y.glb_stride; };
  auto ep = [&](uint32_t s, uint32_t l, uint32_t ph) __attribute__((always_inline)) { return a.epoch0 + ((s * (a.L + 1) + l) << 3) + ph; };
  auto where = [&](uint32_t l, uint32_t ph) __attribute__((always_inline)) { return (l << 8) | ph; };

  uint64_t* trace = nullptr;
  uint32_t s = 0;
#define TR(L_, K_)                                                                                   \
  do {                                                                                               \
    if (trace && tid == 0)                                                                           \
      trace[(((size_t)s * (a.L + 1) + (L_)) * RES_TR_K + (K_)) * RES_BLOCKS + bglob] =               \
          __builtin_amdgcn_s_memrealtime();                                                          \
  } while (0)
  // the end of a compute phase, stamped by a compute wave
#define TRC(L_, K_)                                                                                  \
  do {                                                                                               \
    if (trace && tid == 64)                                                                          \
      trace[(((size_t)s * (a.L + 1) + (L_)) * RES_TR_K + (K_)) * RES_BLOCKS + bglob] =               \
          __builtin_amdgcn_s_memrealtime();                                                          \
  } while (0)
  uint32_t pos = gl(a.st)->pos, tok = gl(a.st)->tok, done = 0;
  bool alive = true, stop = false, comm_ok = true;
  for (s = 0; s < a.n_steps && alive && !stop; ++s) {
    trace = s < a.trace_steps ? a.trace : nullptr;
    TR(a.L, RES_TR_START);
    // ---- embed (model.rs:482-506): every block dequantizes the row itself ----
    {
      const uint8_t* row = a.embd + (size_t)tok * a.rbe;
      const int be = blk_elems(a.te), bb = blk_bytes(a.te);
      for (uint32_t i = tid; i < H; i += RT)
        s_xres[i] = a.te == T_F32 ? ((const float*)row)[i] : decode_elem(a.te, row + (size_t)(i / be) * bb, (int)(i % be));
      __syncthreads();
      TR(a.L, RES_TR_EMBED);
    }
    const uint32_t T = pos + 1;
    const uint32_t NSPL = min(smax, (T + 31) / 32), SLEN = (T + NSPL - 1) / NSPL;
    for (uint32_t l = 0; l < a.L && alive; ++l) {
      const ResLayer Ly = gl(a.layers)[l];
      const uint32_t par = l & 1;
      uint2* LX = loc(par);
      uint2* GX = glb(par);
      TR(l, RES_TR_START);
      // ---- A: rmsnorm + q, k, v rows of the XCD's heads (model.rs:456-459) ----
      {
        Seg sg[3];
        const uint32_t nq = nhx * HD, nk = (g1 - g0) * HD;
        sg[0] = Seg{Ly.wq, nullptr, Ly.tq, a.nh * HD, Ly.rq, h0 * HD, nq, 0, item_of(Ly.tq, H), 0, 0};
        sg[1] = Seg{Ly.wk, nullptr, Ly.tk, a.nkv * HD, Ly.rk, g0 * HD, nk, 0, item_of(Ly.tk, H), 0, nq / 4};
        sg[2] = Seg{Ly.wv, nullptr, Ly.tv, a.nkv * HD, Ly.rv, g0 * HD, nk, 0, item_of(Ly.tv, H), 0, (nq + nk) / 4};
        const XLds X{nullptr, s_pl, H};
        auto wait = [&](auto&& pre) __attribute__((always_inline)) {
          if (l == 0)
            pre();
          else if (!poll(
                       H, [&](uint32_t i) __attribute__((always_inline)) { return loc((l - 1) & 1) + Y.o_x + i; },
                       ep(s, l - 1, 7), (uint32_t*)s_xres, ctl, where(l, 1), pre, comm_ok))
            return false;
          TR(l, RES_TR_A_POLL);
          stage(s_xres, H, gl(Ly.an), a.eps, s_pl, s_red);
          TR(l, RES_TR_A_IN);
          return true;
        };
        const uint32_t e1 = ep(s, l, 1);
        auto out = [&](int si, uint32_t row, float v, float) __attribute__((always_inline)) {
          const GAS float* bias = gl(si == 0 ? Ly.bq : si == 1 ? Ly.bk : Ly.bv);
          const uint32_t o = si == 0 ? 0u : si == 1 ? a.nh * HD : (a.nh + a.nkv) * HD;
          st_local(LX + Y.o_qkv + o + row, v + bias[row], e1);  // model.rs:179-183
        };
        bool ok;
        if constexpr (FS == RES_FS_KQUANT) {
          const bool all4 = Ly.tq == T_Q4_K && Ly.tk == T_Q4_K && Ly.tv == T_Q4_K;
          const bool all6 = Ly.tq == T_Q6_K && Ly.tk == T_Q6_K && Ly.tv == T_Q6_K;
          if (all4)
            ok = gemv_phase<T_Q4_K, T_Q4_K, 16, 3, 1>(sg, wx, RES_CUS * NCW, X, wait, out, early, deep);
          else if (all6)
            ok = gemv_phase<T_Q6_K, T_Q6_K, 16, 3, 1>(sg, wx, RES_CUS * NCW, X, wait, out, early, deep);
          else
            ok = gemv_phase<T_Q4_K, T_Q6_K, 16, 3, 1>(sg, wx, RES_CUS * NCW, X, wait, out, early, deep);
        } else {
          ok = gemv_phase<T_Q8_0, T_Q8_0, 16, 2, 1>(sg, wx, RES_CUS * NCW, X, wait, out, early, deep);
        }
        if (!ok) {
          alive = false;
          break;
        }
        TRC(l, RES_TR_A);
      }
      // ---- B: RoPE, KV append, attention; jobs (head, split) over the XCD's blocks ----
      for (uint32_t j = rank; j < nhx * NSPL && alive; j += RES_CUS) {
        const uint32_t h = h0 + j / NSPL, sp = j % NSPL, g = h / gq;
        const uint32_t t0 = sp * SLEN, t1 = min(T, t0 + SLEN);
        uint2* dst = LX + Y.o_att + (h * RES_MAX_SPLITS + sp) * (HD + 2);
        const bool wkv = sp == 0 && h == g * gq;  // the group's first head writes its cache row
        const bool ok = HD == 128 ? attn_job<128>(a, l, pos, h, g, t0, t1, LX + Y.o_qkv, ep(s, l, 1), dst,
                                                  ep(s, l, 2), wkv, s_att, where(l, 2))
                                  : attn_job<64>(a, l, pos, h, g, t0, t1, LX + Y.o_qkv, ep(s, l, 1), dst,
                                                 ep(s, l, 2), wkv, s_att, where(l, 2));
        if (!ok) alive = false;
      }
      if (!alive) break;
      TR(l, RES_TR_B);
      // ---- C: merge the splits (model.rs:436-438), o-proj partial over the XCD's head columns ----
      {
        Seg sg[1];
        const uint32_t c0 = h0 * HD, nc = nhx * HD;
        sg[0] = Seg{Ly.wo, nullptr, Ly.to, H, Ly.ro, r0, nhx ? nr : 0u, item_of(Ly.to, c0), item_of(Ly.to, nc),
                    c0 / 16, 0};
        const XLds X{nullptr, s_pl, nc};
        auto wait = [&](auto&& pre) __attribute__((always_inline)) {
          if (!nhx) {
            pre();
            return true;
          }
          const uint32_t per = NSPL * (HD + 2);
          if (!poll(
                  nhx * per,
                  [&](uint32_t i) __attribute__((always_inline)) {
                    const uint32_t hh = i / per, r = i % per;
                    return LX + Y.o_att + ((h0 + hh) * RES_MAX_SPLITS) * (HD + 2) + r;
                  },
                  ep(s, l, 2), (uint32_t*)s_att, ctl, where(l, 3), pre))
            return false;
          TR(l, RES_TR_C_POLL);
          for (uint32_t i = tid; i < nc; i += RT) {
            const uint32_t hh = i / HD, d = i % HD;
            const float* P = s_att + hh * per;
            float M = -INFINITY;
            for (uint32_t q = 0; q < NSPL; ++q) M = fmaxf(M, P[q * (HD + 2) + HD]);
            float o = 0.f, L = 0.f;
            for (uint32_t q = 0; q < NSPL; ++q) {
              const float e = expf(P[q * (HD + 2) + HD] - M);
              L += e * P[q * (HD + 2) + HD + 1];
              o += e * P[q * (HD + 2) + d];
            }
            s_vin[i] = L > 0.f ? o / L : 0.f;
          }
          __syncthreads();
          stage(s_vin, nc, (const GAS float*)nullptr, 0.f, s_pl, s_red);
          TR(l, RES_TR_C_IN);
          return true;
        };
        const uint32_t e3 = ep(s, l, 3);
        auto out = [&](int, uint32_t row, float v, float) __attribute__((always_inline)) { st_cross(GX + Y.o_po + xcd * H + row, v, e3); };
        if (!by_type<FS>(Ly.to, [&](auto tc) __attribute__((always_inline)) {
              constexpr uint32_t TT = decltype(tc)::value;
              return gemv_phase<TT, TT, 4, 2, 1>(sg, cw, NCW, X, wait, out, early, deep);
            })) {
          alive = false;
          break;
        }
        if (!nhx && tid < nr) st_cross(GX + Y.o_po + xcd * H + r0 + tid, 0.f, e3);
        TRC(l, RES_TR_C);
      }
      // ---- D: x' = x + o-proj (tensor.rs:229-234), this CU's rows ----
      {
        // the communication wave alone (no barrier: the compute waves go on
        // to their gate/up loads); a failure reaches the block at E's barrier
        if (tid < 64) {
          comm_ok = poll_wave(
              8 * nr, [&](uint32_t i) __attribute__((always_inline)) { return GX + Y.o_po + (i / nr) * H + r0 + i % nr; },
              ep(s, l, 3), (uint32_t*)s_ared, ctl, where(l, 4));
          for (uint32_t i = lane; comm_ok && i < nr; i += 64) {
            float v = s_ared[i];
#pragma unroll
            for (int y = 1; y < (int)RES_XCDS; ++y) v += s_ared[y * nr + i];
            const float x2 = s_xres[r0 + i] + v;
            s_rowv[i] = x2;
            st_local(LX + Y.o_x2 + r0 + i, x2, ep(s, l, 4));
          }
        }
        TR(l, RES_TR_D);
      }
      // ---- E: rmsnorm + gate/up rows of the XCD's FFN slice + SwiGLU (model.rs:473-476) ----
      {
        Seg sg[1];
        sg[0] = Seg{Ly.wg, Ly.wu, Ly.tg, a.F, Ly.rg, f0, f1 - f0, 0, item_of(Ly.tg, H), 0, 0};
        const XLds X{nullptr, s_pl, H};
        auto wait = [&](auto&& pre) __attribute__((always_inline)) {
          if (!poll(
                  H, [&](uint32_t i) __attribute__((always_inline)) { return LX + Y.o_x2 + i; }, ep(s, l, 4), (uint32_t*)s_vin, ctl,
                  where(l, 5), pre, comm_ok))
            return false;
          TR(l, RES_TR_E_POLL);
          stage(s_vin, H, gl(Ly.fn), a.eps, s_pl, s_red);
          TR(l, RES_TR_E_IN);
          return true;
        };
        const uint32_t e5 = ep(s, l, 5);
        auto out = [&](int, uint32_t row, float gv, float uv) __attribute__((always_inline)) {
          st_local(LX + Y.o_act + row, gv / (1.0f + expf(-gv)) * uv, e5);  // tensor.rs:224
        };
        if (!by_type<FS>(Ly.tg, [&](auto tc) __attribute__((always_inline)) {
              constexpr uint32_t TT = decltype(tc)::value;
              return gemv_phase<TT, TT, 16, 3, 2>(sg, wx, RES_CUS * NCW, X, wait, out, early, deep);
            })) {
          alive = false;
          break;
        }
        TRC(l, RES_TR_E);
      }
      // ---- F: down partial over the XCD's FFN columns (model.rs:476-477) ----
      {
        Seg sg[1];
        const uint32_t nc = f1 - f0;
        sg[0] = Seg{Ly.wd, nullptr, Ly.td, H, Ly.rd, r0, nc ? nr : 0u, item_of(Ly.td, f0), item_of(Ly.td, nc),
                    f0 / 16, 0};
        const XLds X{nullptr, s_pl, nc};
        auto wait = [&](auto&& pre) __attribute__((always_inline)) {
          if (!nc) {
            pre();
            return true;
          }
          if (!poll(
                  nc, [&](uint32_t i) __attribute__((always_inline)) { return LX + Y.o_act + f0 + i; }, ep(s, l, 5), (uint32_t*)s_vin, ctl,
                  where(l, 6), pre))
            return false;
          TR(l, RES_TR_F_POLL);
          stage(s_vin, nc, (const GAS float*)nullptr, 0.f, s_pl, s_red);
          TR(l, RES_TR_F_IN);
          return true;
        };
        const uint32_t e6 = ep(s, l, 6);
        auto out = [&](int, uint32_t row, float v, float) __attribute__((always_inline)) { st_cross(GX + Y.o_pd + xcd * H + row, v, e6); };
        if (!by_type<FS>(Ly.td, [&](auto tc) __attribute__((always_inline)) {
              constexpr uint32_t TT = decltype(tc)::value;
              return gemv_phase<TT, TT, 8, 5, 1>(sg, cw, NCW, X, wait, out, early, deep);
            })) {
          alive = false;
          break;
        }
        if (!nc && tid < nr) st_cross(GX + Y.o_pd + xcd * H + r0 + tid, 0.f, e6);
        TRC(l, RES_TR_F);
      }
      // ---- G: x'' = x' + down (tensor.rs:229-234), this CU's rows ----
      {
        if (tid < 64) {  // the communication wave alone, as D
          comm_ok = poll_wave(
              8 * nr, [&](uint32_t i) __attribute__((always_inline)) { return GX + Y.o_pd + (i / nr) * H + r0 + i % nr; },
              ep(s, l, 6), (uint32_t*)s_ared, ctl, where(l, 7));
          for (uint32_t i = lane; comm_ok && i < nr; i += 64) {
            float v = s_ared[i];
#pragma unroll
            for (int y = 1; y < (int)RES_XCDS; ++y) v += s_ared[y * nr + i];
            st_local(LX + Y.o_x + r0 + i, s_rowv[i] + v, ep(s, l, 7));
          }
        }
        TR(l, RES_TR_G);
      }
    }
    if (!alive) break;
    // ---- last_row_logits (model.rs:594-600): rmsnorm + this block's lm_head rows + argmax candidate ----
    {
      uint64_t best = 0;
      Seg sg[1];
      sg[0] = Seg{a.lm, nullptr, a.tl, a.V, a.rbl, lr0, lnr, 0, item_of(a.tl, H), 0, 0};
      const XLds X{nullptr, s_pl, H};
      auto wait = [&](auto&& pre) __attribute__((always_inline)) {
        if (!poll(
                H, [&](uint32_t i) __attribute__((always_inline)) { return loc((a.L - 1) & 1) + Y.o_x + i; }, ep(s, a.L - 1, 7),
                (uint32_t*)s_xres, ctl, where(a.L, 1), pre, comm_ok))
          return false;
        stage(s_xres, H, gl(a.onorm), a.eps, s_pl, s_red);
        TR(a.L, RES_TR_H_IN);
        return true;
      };
      auto out = [&](int, uint32_t row, float v, float) __attribute__((always_inline)) {
        gl(a.logits)[row] = v;
        const uint64_t k = argmax_key(v, row);
        best = k > best ? k : best;
      };
        if (!by_type<FS>(a.tl, [&](auto tc) __attribute__((always_inline)) {
              constexpr uint32_t TT = decltype(tc)::value;
              return gemv_phase<TT, TT, 16, 3, 1>(sg, wave, NWAVE, X, wait, out, early, deep);
            })) {
        alive = false;
        break;
      }
      for (int o = 32; o > 0; o >>= 1) {
        const uint64_t other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
      }
      if (lane == 0) s_keys[wave] = best;
      __syncthreads();
      if (tid == 0) {
        uint64_t b = s_keys[0];
        for (int i = 1; i < NWAVE; ++i) b = s_keys[i] > b ? s_keys[i] : b;
        uint2* C = glb(s & 1) + Y.o_lmc + 2 * bglob;
        st_cross_bits(C, (uint32_t)(b >> 32), ep(s, a.L, 1));
        st_cross_bits(C + 1, (uint32_t)b, ep(s, a.L, 1));
      }
      TRC(a.L, RES_TR_H);
    }
    // ---- argmax over the 256 candidates (generate.rs:69-77), in every block ----
    {
      uint32_t* kb = (uint32_t*)s_ared;
      if (!poll(
              2 * RES_BLOCKS, [&](uint32_t i) __attribute__((always_inline)) { return glb(s & 1) + Y.o_lmc + i; }, ep(s, a.L, 1), kb, ctl,
              where(a.L, 2))) {
        alive = false;
        break;
      }
      uint64_t b = tid < RES_BLOCKS ? ((uint64_t)kb[2 * tid] << 32) | kb[2 * tid + 1] : 0ull;
      for (int o = 32; o > 0; o >>= 1) {
        const uint64_t other = __shfl_xor(b, o, 64);
        b = other > b ? other : b;
      }
      if (lane == 0) s_keys[wave] = b;
      __syncthreads();
      b = s_keys[0];
      for (int i = 1; i < NWAVE; ++i) b = s_keys[i] > b ? s_keys[i] : b;
      __syncthreads();
      tok = 0xFFFFFFFFu - (uint32_t)(b & 0xFFFFFFFFull);
      if (xcd == 0 && rank == 0 && tid == 0) gl(a.hist)[pos] = tok;
      pos += 1;
      done = s + 1;
      for (uint32_t k = 0; k < a.n_stop; ++k) stop = stop || tok == a.stop[k];  // generate.rs:125-127
      TR(a.L, RES_TR_I);
    }
  }
#undef TR
#undef TRC
  if (alive && xcd == 0 && rank == 0 && tid == 0) {
    gl(a.st)->pos = pos;
    gl(a.st)->tok = tok;
    gl(a.st)->next_tok = tok;
    ctl->n_done = done;
  }
}

}  // namespace

ResLayout res_layout(uint32_t H, uint32_t F, uint32_t nh, uint32_t nkv, uint32_t hd) {
  auto al = [](uint32_t v) { return (v + 511u) & ~511u; };  // 4 KiB regions
  ResLayout l{};
  l.o_x = 0;
  l.o_qkv = al(H);
  l.o_att = l.o_qkv + al((nh + 2 * nkv) * hd);
  l.o_x2 = l.o_att + al(nh * RES_MAX_SPLITS * (hd + 2));
  l.o_act = l.o_x2 + al(H);
  l.loc_stride = l.o_act + al(F);
  l.o_po = 0;
  l.o_pd = al(RES_XCDS * H);
  l.o_lmc = l.o_pd + al(RES_XCDS * H);
  l.glb_stride = l.o_lmc + al(2 * RES_BLOCKS);
  return l;
}

size_t res_exchange_pairs(const ResLayout& l) {
  return (size_t)RES_XCDS * 2 * l.loc_stride + 2 * (size_t)l.glb_stride;
}

const char* res_unsupported(uint32_t H, uint32_t F, uint32_t nh, uint32_t nkv, uint32_t hd, const uint32_t* types,
                            size_t n_types, uint32_t lm_type, uint32_t o_gran, uint32_t* fset) {
  if (hd != 64 && hd != 128) return "head_dim not 64 or 128";
  if (nh % nkv || nh / nkv > 8) return "query heads per kv head";
  // an XCD's heads' splits fit the merge buffer (32 x (128 + 2) pairs)
  if ((nh + RES_XCDS - 1) / RES_XCDS > 32) return "more than 32 query heads per XCD";
  if (H > RES_MAX_K || H % 32) return "hidden size above 4096 or not a multiple of 32";
  if (F % 128) return "ffn not a multiple of 128";
  if ((F / 128 + RES_XCDS - 1) / RES_XCDS * 128 > RES_MAX_K) return "ffn slice above 4096";
  if (nh * hd != H) return "heads x head_dim != hidden";
  bool kq = true, q8 = true;
  for (size_t i = 0; i < n_types; ++i) {
    kq = kq && (types[i] == T_Q4_K || types[i] == T_Q6_K);
    q8 = q8 && types[i] == T_Q8_0;
  }
  kq = kq && (lm_type == T_Q4_K || lm_type == T_Q6_K);
  q8 = q8 && lm_type == T_Q8_0;
  if (!kq && !q8) return "matrix formats (all Q4_K/Q6_K or all Q8_0)";
  // item-aligned column slices: K-quant rows are whole superblocks; Q6_K
  // items span 128 values, Q4_K and Q8_0 items 64
  if (kq && H % 256) return "hidden not a multiple of 256 (K-quant rows)";
  if (q8 && (H / 32) % 2) return "hidden not an even number of Q8_0 blocks";
  for (uint32_t x = 0; x < RES_XCDS; ++x)
    if ((nh * x / RES_XCDS) * hd % o_gran) return "o-proj head columns not aligned to the format's items";
  *fset = kq ? RES_FS_KQUANT : RES_FS_Q8_0;
  return nullptr;
}

hipError_t res_prepare() {
  hipError_t e;
  if ((e = hipFuncSetAttribute((const void*)k_resident<RES_FS_KQUANT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               RES_LDS_BYTES)))
    return e;
  return hipFuncSetAttribute((const void*)k_resident<RES_FS_Q8_0>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             RES_LDS_BYTES);
}

hipError_t launch_resident(const ResArgs* host, ResArgs* dev, hipStream_t s) {
  hipError_t e;
  if ((e = hipMemsetAsync(host->ctl, 0, sizeof(ResCtl), s)) ||
      (e = hipMemcpyAsync(dev, host, sizeof(ResArgs), hipMemcpyHostToDevice, s)))
    return e;
  const ResArgs* arg = dev;
  void* args[] = {(void*)&arg};
  const void* f =
      host->fset == RES_FS_Q8_0 ? (const void*)k_resident<RES_FS_Q8_0> : (const void*)k_resident<RES_FS_KQUANT>;
  return hipLaunchCooperativeKernel(f, dim3(RES_BLOCKS), dim3(RES_THREADS), args, RES_LDS_BYTES, s);
}

}  // namespace frn
