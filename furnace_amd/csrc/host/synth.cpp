// Seeded synthetic GGUF models and block encoders.
//
// furnace has no quantizer (it only decodes, src/quant.rs:17-133), so the
// encoders here are written from its block layouts: each one emits blocks
// that quant.rs's dequantizers decode, choosing scales by simple max-abs /
// min-max rules (round-to-nearest, f16 scales rounded before the quants are
// chosen).  Parity does not depend on encoder quality: the GPU and the CPU
// path decode the same bytes.
#include <fcntl.h>
#include <math.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <string>
#include <thread>
#include <vector>

#include "../../../include/furnace_host.h"
#include "../common.hpp"

namespace {

// ---- f16 -------------------------------------------------------------------
uint16_t f32_to_f16(float f) {  // IEEE round-to-nearest-even
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  int32_t e = (int32_t)((x >> 23) & 0xFF) - 127 + 15;
  uint32_t m = x & 0x7FFFFFu;
  if (((x >> 23) & 0xFF) == 0xFF) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0));
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    m |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - e);
    uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hm & 1))) ++hm;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = m >> 13, rem = m & 0x1FFFu;
  uint32_t h = sign | ((uint32_t)e << 10) | hm;
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) ++h;
  return (uint16_t)h;
}
float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, ex = (h >> 10) & 0x1F, m = h & 0x3FF, bits;
  if (ex == 0) {
    if (!m) {
      bits = sign;
    } else {
      int e = 0;
      while (!(m & 0x400u)) { m <<= 1; ++e; }
      bits = sign | ((uint32_t)(113 - e) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (ex == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((ex + 112) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}
// f16-round a scale, returning the encoded bits and the f32 value decoded
void f16_round(float v, uint16_t* bits, float* dec) {
  *bits = f32_to_f16(v);
  *dec = f16_to_f32(*bits);
}
void put16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
int iround(float v) { return (int)lrintf(v); }

// ---- encoders (inverse of quant.rs:17-133) -----------------------------------
void enc_q8_0(const float* x, uint8_t* b) {  // 34 B: f16 d | i8 q[32]
  float amax = 0;
  for (int i = 0; i < 32; ++i) amax = std::max(amax, fabsf(x[i]));
  uint16_t db;
  float d;
  f16_round(amax / 127.f, &db, &d);
  put16(b, db);
  for (int i = 0; i < 32; ++i) {
    int q = d > 0 ? iround(x[i] / d) : 0;
    b[2 + i] = (uint8_t)(int8_t)std::min(127, std::max(-127, q));
  }
}

void enc_q5_0(const float* x, uint8_t* b) {  // 22 B: f16 d | u32 qh | 16 nibble bytes
  float amax = 0, vmax = 0;
  for (int i = 0; i < 32; ++i)
    if (fabsf(x[i]) > amax) { amax = fabsf(x[i]); vmax = x[i]; }
  uint16_t db;
  float d;
  f16_round(vmax / -16.f, &db, &d);
  put16(b, db);
  uint32_t qh = 0;
  uint8_t q[32];
  for (int i = 0; i < 32; ++i) {
    int v = d != 0 ? iround(x[i] / d) + 16 : 16;
    q[i] = (uint8_t)std::min(31, std::max(0, v));
  }
  for (int j = 0; j < 16; ++j) {
    b[6 + j] = (uint8_t)((q[j] & 0x0F) | ((q[j + 16] & 0x0F) << 4));
    qh |= (uint32_t)((q[j] >> 4) & 1) << j;
    qh |= (uint32_t)((q[j + 16] >> 4) & 1) << (j + 16);
  }
  memcpy(b + 2, &qh, 4);
}

void enc_q4_k(const float* x, uint8_t* b) {  // 144 B
  float scale[8], mn[8];
  for (int j = 0; j < 8; ++j) {
    float lo = 0, hi = 0;
    for (int i = 0; i < 32; ++i) {
      lo = std::min(lo, x[32 * j + i]);
      hi = std::max(hi, x[32 * j + i]);
    }
    scale[j] = (hi - lo) / 15.f;
    mn[j] = -lo;
  }
  float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(mn, mn + 8);
  uint16_t db, dminb;
  float d, dmin;
  f16_round(ms / 63.f, &db, &d);
  f16_round(mm / 63.f, &dminb, &dmin);
  put16(b, db);
  put16(b + 2, dminb);
  uint8_t sc[8], m[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = (uint8_t)(d > 0 ? std::min(63, std::max(0, iround(scale[j] / d))) : 0);
    m[j] = (uint8_t)(dmin > 0 ? std::min(63, std::max(0, iround(mn[j] / dmin))) : 0);
    // a sub-block whose scale rounds to 0 keeps its values representable
    if (sc[j] == 0 && scale[j] > 0 && d > 0) sc[j] = 1;
  }
  uint8_t* s = b + 4;  // inverse of q4k_scale_min (quant.rs:78-88)
  memset(s, 0, 12);
  for (int j = 0; j < 4; ++j) {
    s[j] = sc[j] & 63;
    s[j + 4] = m[j] & 63;
  }
  for (int j = 4; j < 8; ++j) {
    s[j + 4] = (uint8_t)((sc[j] & 0x0F) | ((m[j] & 0x0F) << 4));
    s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
    s[j] |= (uint8_t)((m[j] >> 4) << 6);
  }
  uint8_t q[256];
  for (int j = 0; j < 8; ++j) {
    float dd = d * (float)sc[j], dm = dmin * (float)m[j];
    for (int i = 0; i < 32; ++i) {
      int v = dd > 0 ? iround((x[32 * j + i] + dm) / dd) : 0;
      q[32 * j + i] = (uint8_t)std::min(15, std::max(0, v));
    }
  }
  uint8_t* qs = b + 16;
  for (int j64 = 0; j64 < 4; ++j64)
    for (int l = 0; l < 32; ++l) qs[32 * j64 + l] = (uint8_t)(q[64 * j64 + l] | (q[64 * j64 + 32 + l] << 4));
}

void enc_q6_k(const float* x, uint8_t* b) {  // 210 B
  float sub[16];
  for (int j = 0; j < 16; ++j) {
    float amax = 0;
    for (int i = 0; i < 16; ++i) amax = std::max(amax, fabsf(x[16 * j + i]));
    sub[j] = amax / 31.f;
  }
  float smax = *std::max_element(sub, sub + 16);
  uint16_t db;
  float d;
  f16_round(smax / 127.f, &db, &d);
  memset(b, 0, 210);
  put16(b + 208, db);
  int8_t sc[16];
  for (int j = 0; j < 16; ++j) {
    int v = d > 0 ? iround(sub[j] / d) : 0;
    if (v == 0 && sub[j] > 0 && d > 0) v = 1;
    sc[j] = (int8_t)std::min(127, std::max(-128, v));
    b[192 + j] = (uint8_t)sc[j];
  }
  for (int e = 0; e < 256; ++e) {
    float dd = d * (float)sc[e / 16];
    int q = dd != 0 ? iround(x[e] / dd) : 0;
    uint32_t u = (uint32_t)(std::min(31, std::max(-32, q)) + 32);  // 6 bits
    int h = e / 128, r = e % 128, k = r / 32, l = r % 32;
    uint8_t* ql = b + 64 * h + l + ((k & 1) ? 32 : 0);
    *ql |= (uint8_t)((u & 0x0F) << ((k & 2) ? 4 : 0));
    b[128 + 32 * h + l] |= (uint8_t)((u >> 4) << (2 * k));
  }
}

void enc_f16(const float* x, uint8_t* b) { put16(b, f32_to_f16(x[0])); }  // IEEE half, round to nearest even

bool encoder(uint32_t type, void (**f)(const float*, uint8_t*), int* be, int* bb) {
  switch (type) {
    case 1: *f = enc_f16; *be = 1; *bb = 2; return true;
    case 8: *f = enc_q8_0; *be = 32; *bb = 34; return true;
    case 6: *f = enc_q5_0; *be = 32; *bb = 22; return true;
    case 12: *f = enc_q4_k; *be = 256; *bb = 144; return true;
    case 14: *f = enc_q6_k; *be = 256; *bb = 210; return true;
    default: return false;
  }
}

// ---- deterministic N(0, std) -------------------------------------------------
uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
// Values i and i+1 (i even) come from one Box-Muller pair keyed by (seed, i/2),
// so any index range can be generated independently.
void gaussian_range(uint64_t seed, float std, size_t begin, size_t end, float* out /* indexed from begin */) {
  for (size_t i = begin & ~(size_t)1; i < end; i += 2) {
    uint64_t r1 = splitmix64(seed ^ splitmix64(i)), r2 = splitmix64(r1);
    double u1 = ((double)(r1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
    double rad = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
    float z0 = (float)(rad * cos(th)) * std, z1 = (float)(rad * sin(th)) * std;
    if (i >= begin) out[i - begin] = z0;
    if (i + 1 >= begin && i + 1 < end) out[i + 1 - begin] = z1;
  }
}

// ---- GGUF writer ---------------------------------------------------------------
struct Buf {
  std::vector<uint8_t> d;
  void u32(uint32_t v) { for (int i = 0; i < 4; ++i) d.push_back((uint8_t)(v >> (8 * i))); }
  void u64(uint64_t v) { for (int i = 0; i < 8; ++i) d.push_back((uint8_t)(v >> (8 * i))); }
  void f32(float f) { uint32_t v; memcpy(&v, &f, 4); u32(v); }
  void str(const std::string& s) { u64(s.size()); d.insert(d.end(), s.begin(), s.end()); }
};

struct TSpec {
  std::string name;
  uint64_t in, out;  // out = 1 for 1-D
  uint32_t type;
  int kind;          // 0 gaussian, 1 ones
  uint64_t seed;
  uint64_t offset = 0, bytes = 0;
};

uint64_t tensor_bytes(uint32_t type, uint64_t n) {
  switch (type) {
    case 0: return n * 4;
    case 1: return n * 2;
    case 8: return n / 32 * 34;
    case 6: return n / 32 * 22;
    case 12: return n / 256 * 144;
    case 14: return n / 256 * 210;
  }
  return 0;
}

}  // namespace

extern "C" frn_status frn_quantize(uint32_t type, const float* x, size_t n, uint8_t* out) {
  void (*f)(const float*, uint8_t*);
  int be, bb;
  if (type == 0) {
    memcpy(out, x, n * 4);
    return FRN_OK;
  }
  if (!encoder(type, &f, &be, &bb)) return frn_fail(FRN_EDTYPE, "no encoder for ggml type %u", type);
  if (n % (size_t)be) return frn_fail(FRN_ESHAPE, "%zu values is not a multiple of %d", n, be);
  for (size_t i = 0; i < n / be; ++i) f(x + i * be, out + i * bb);
  return FRN_OK;
}

extern "C" frn_status frn_gaussian(uint64_t seed, float std, size_t n, float* out) {
  gaussian_range(seed, std, 0, n, out);
  return FRN_OK;
}

extern "C" frn_status frn_synth_write(const frn_synth_spec* sp, const char* path) {
  if (!sp || !path) return frn_fail(FRN_EINVAL, "frn_synth_write: null argument");
  const frn_synth_spec& S = *sp;
  if (!S.n_heads || S.hidden % S.n_heads || !S.n_kv_heads || S.n_heads % S.n_kv_heads)
    return frn_fail(FRN_ESHAPE, "frn_synth_write: bad head configuration");
  if (S.alignment & (S.alignment - 1))
    return frn_fail(FRN_EINVAL, "frn_synth_write: alignment %u is not a power of two", S.alignment);
  const uint64_t align = S.alignment ? S.alignment : 32;
  uint64_t H = S.hidden, hd = H / S.n_heads, qd = H, kd = (uint64_t)S.n_kv_heads * hd, F = S.ffn;
  auto lin_type = [&](int which, uint32_t layer) -> uint32_t {  // which: 0 q,1 k,2 v,3 o,4 gate,5 up,6 down
    switch (S.mix) {
      case FRN_MIX_ALL_Q8_0: return 8;
      case FRN_MIX_ALL_Q4_K: return 12;
      case FRN_MIX_ALL_Q6_K: return 14;
      case FRN_MIX_ALL_Q5_0: return 6;
      case FRN_MIX_ALL_F32: return 0;
      case FRN_MIX_ALL_F16: return 1;
      case FRN_MIX_Q4_K_M_LLAMA: {
        // llama.cpp's Q4_K_M (llama_tensor_get_type, use_more_bits): Q6_K
        // for attn_v and ffn_down on the first and last eighth of the
        // layers and on every third layer between them, Q4_K elsewhere
        const uint32_t n = S.n_layers, e = n / 8;
        const bool more = layer < e || layer >= 7 * n / 8 || (layer - e) % 3 == 2;
        return ((which == 2 || which == 6) && more) ? 14 : 12;
      }
      default:  // Q4_K_M: Q6_K for attn_v and ffn_down on even layers
        return ((which == 2 || which == 6) && layer % 2 == 0) ? 14 : 12;
    }
  };
  std::vector<TSpec> ts;
  uint64_t tid = 0;
  auto add = [&](const std::string& name, uint64_t in, uint64_t out, uint32_t type, int kind) {
    TSpec t{name, in, out, type, kind, splitmix64(S.seed ^ (0x51ED270B27A1C0DEull * (++tid)))};
    ts.push_back(t);
  };
  add("token_embd.weight", H, S.vocab, S.embd_type, 0);
  for (uint32_t l = 0; l < S.n_layers; ++l) {
    std::string p = "blk." + std::to_string(l) + ".";
    add(p + "attn_norm.weight", H, 1, 0, 1);
    add(p + "attn_q.weight", H, qd, lin_type(0, l), 0);
    add(p + "attn_q.bias", qd, 1, 0, 0);
    add(p + "attn_k.weight", H, kd, lin_type(1, l), 0);
    add(p + "attn_k.bias", kd, 1, 0, 0);
    add(p + "attn_v.weight", H, kd, lin_type(2, l), 0);
    add(p + "attn_v.bias", kd, 1, 0, 0);
    add(p + "attn_output.weight", qd, H, lin_type(3, l), 0);
    add(p + "ffn_norm.weight", H, 1, 0, 1);
    add(p + "ffn_gate.weight", H, F, lin_type(4, l), 0);
    add(p + "ffn_up.weight", H, F, lin_type(5, l), 0);
    add(p + "ffn_down.weight", F, H, lin_type(6, l), 0);
  }
  add("output_norm.weight", H, 1, 0, 1);
  if (!S.tied) add("output.weight", H, S.vocab, S.output_type, 0);
  for (auto& t : ts) {
    size_t be = t.type == 12 || t.type == 14 ? 256 : t.type <= 1 ? 1 : 32;
    if (t.in % be) return frn_fail(FRN_ESHAPE, "tensor %s: in dim %llu not a multiple of %zu", t.name.c_str(),
                                   (unsigned long long)t.in, be);
  }
  // header + metadata + tensor infos
  Buf h;
  h.d.insert(h.d.end(), {'G', 'G', 'U', 'F'});
  h.u32(3);
  h.u64(ts.size());
  uint64_t n_kv = 15 + (S.vocab > 151645 ? 2 : 0) + (S.alignment ? 1 : 0);
  h.u64(n_kv);
  auto kv_u32 = [&](const char* k, uint32_t v) { h.str(k); h.u32(4); h.u32(v); };
  auto kv_f32 = [&](const char* k, float v) { h.str(k); h.u32(6); h.f32(v); };
  auto kv_str = [&](const char* k, const char* v) { h.str(k); h.u32(8); h.str(v); };
  kv_str("general.architecture", "qwen2");
  if (S.alignment) kv_u32("general.alignment", S.alignment);
  kv_str("general.name", "furnace-hip synthetic");
  kv_u32("qwen2.block_count", S.n_layers);
  kv_u32("qwen2.context_length", S.context_length);
  kv_u32("qwen2.embedding_length", S.hidden);
  kv_u32("qwen2.feed_forward_length", S.ffn);
  kv_u32("qwen2.attention.head_count", S.n_heads);
  kv_u32("qwen2.attention.head_count_kv", S.n_kv_heads);
  kv_f32("qwen2.rope.freq_base", S.rope_theta);
  kv_f32("qwen2.attention.layer_norm_rms_epsilon", S.rms_eps);
  kv_str("tokenizer.ggml.model", "gpt2");
  kv_str("tokenizer.ggml.pre", "qwen2");
  h.str("tokenizer.ggml.tokens");
  h.u32(9);
  h.u32(8);
  h.u64(S.vocab);
  for (uint32_t i = 0; i < S.vocab; ++i) h.str("<" + std::to_string(i) + ">");
  h.str("tokenizer.ggml.token_type");
  h.u32(9);
  h.u32(5);
  h.u64(S.vocab);
  for (uint32_t i = 0; i < S.vocab; ++i) h.u32(1);
  h.str("tokenizer.ggml.merges");
  h.u32(9);
  h.u32(8);
  h.u64(0);
  if (S.vocab > 151645) {
    kv_u32("tokenizer.ggml.eos_token_id", 151645);
    kv_u32("tokenizer.ggml.bos_token_id", 151643);
  }
  uint64_t off = 0;
  for (auto& t : ts) {
    h.str(t.name);
    if (t.out == 1) {
      h.u32(1);
      h.u64(t.in);
    } else {
      h.u32(2);
      h.u64(t.in);
      h.u64(t.out);
    }
    h.u32(t.type);
    t.offset = off;
    t.bytes = tensor_bytes(t.type, t.in * t.out);
    h.u64(off);
    off += (t.bytes + align - 1) / align * align;
  }
  while (h.d.size() % align) h.d.push_back(0);
  uint64_t total = h.d.size() + off;
  int fd = ::open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) return frn_fail(FRN_EINVAL, "cannot create %s", path);
  if (ftruncate(fd, (off_t)total)) {
    ::close(fd);
    return frn_fail(FRN_EINVAL, "cannot size %s to %llu bytes", path, (unsigned long long)total);
  }
  uint8_t* map = (uint8_t*)mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) return frn_fail(FRN_EINVAL, "mmap of %s failed", path);
  memcpy(map, h.d.data(), h.d.size());
  uint8_t* data = map + h.d.size();
  // work items: (tensor, row chunk); rows of a tensor are independent
  struct Work { size_t t; uint64_t r0, r1; };
  std::vector<Work> work;
  for (size_t i = 0; i < ts.size(); ++i) {
    uint64_t rows = ts[i].out, chunk = std::max<uint64_t>(1, (1u << 20) / std::max<uint64_t>(1, ts[i].in));
    for (uint64_t r = 0; r < rows; r += chunk) work.push_back({i, r, std::min(rows, r + chunk)});
  }
  std::atomic<size_t> next{0};
  std::atomic<int> err{0};
  unsigned nth = S.threads ? S.threads : std::max(1u, std::thread::hardware_concurrency());
  auto worker = [&]() {
    std::vector<float> row;
    for (size_t w; (w = next.fetch_add(1)) < work.size();) {
      const TSpec& t = ts[work[w].t];
      uint64_t in = t.in, r0 = work[w].r0, r1 = work[w].r1;
      row.resize((size_t)(in * (r1 - r0)));
      if (t.kind == 1) std::fill(row.begin(), row.end(), 1.0f);
      else gaussian_range(t.seed, S.weight_std, (size_t)(r0 * in), (size_t)(r1 * in), row.data());
      uint64_t rb = tensor_bytes(t.type, in);
      if (frn_quantize(t.type, row.data(), row.size(), data + t.offset + r0 * rb)) err = 1;
    }
  };
  std::vector<std::thread> pool;
  for (unsigned i = 0; i < nth; ++i) pool.emplace_back(worker);
  for (auto& th : pool) th.join();
  munmap(map, total);
  if (err) return frn_fail(FRN_EINVAL, "quantization failed");
  return FRN_OK;
}
