// furnace-hip: command-line driver over the engine ABI, mirroring furnace's
// `run` (src/main.rs:225-267, generate.rs:98-155 stderr lines) and
// `dump-tensor` (src/main.rs:128-160), plus `synth` to write the seeded
// synthetic models.  Prompts are token ids (--prompt-ids), the form the
// synthetic models use; there is no tokenizer on this path.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "../../../include/furnace_host.h"

static double now_s() {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + ts.tv_nsec * 1e-9;
}

static int die(const char* what) {
  fprintf(stderr, "Error: %s: %s\n", what, frn_last_error());
  return 1;
}

static std::vector<uint32_t> parse_ids(const char* s) {
  std::vector<uint32_t> v;
  while (*s) {
    char* end;
    unsigned long x = strtoul(s, &end, 10);
    if (end == s) break;
    v.push_back((uint32_t)x);
    s = *end ? end + 1 : end;
  }
  return v;
}

static int cmd_run(int argc, char** argv) {
  if (argc < 1)
    return fprintf(stderr, "usage: furnace-hip run MODEL --prompt-ids a,b,c [-n N] [--temp T] [--top-k K] [--top-p P] "
                           "[--repeat-penalty R] [--seed S] [--max-ctx C] [--device D] [--timings]\n"),
           2;
  const char* model = argv[0];
  std::vector<uint32_t> ids;
  uint32_t max_new = 50, max_ctx = 0;
  int device = 0;
  bool timings = false, eager = false, have_seed = false;
  // sampler settings and defaults of main.rs:42-58
  float temp = 0.7f, top_p = 0.9f, repeat_penalty = 1.0f;
  uint32_t top_k = 40;
  uint64_t seed = 0;
  for (int i = 1; i < argc; ++i) {
    if (!strcmp(argv[i], "--prompt-ids") && i + 1 < argc) ids = parse_ids(argv[++i]);
    else if ((!strcmp(argv[i], "-n") || !strcmp(argv[i], "--max-tokens")) && i + 1 < argc) max_new = (uint32_t)atoi(argv[++i]);
    else if (!strcmp(argv[i], "--max-ctx") && i + 1 < argc) max_ctx = (uint32_t)atoi(argv[++i]);
    else if (!strcmp(argv[i], "--device") && i + 1 < argc) device = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--timings")) timings = true;
    else if (!strcmp(argv[i], "--eager")) eager = true;
    else if (!strcmp(argv[i], "--temp") && i + 1 < argc) temp = (float)atof(argv[++i]);
    else if (!strcmp(argv[i], "--top-k") && i + 1 < argc) top_k = (uint32_t)atoi(argv[++i]);
    else if (!strcmp(argv[i], "--top-p") && i + 1 < argc) top_p = (float)atof(argv[++i]);
    else if (!strcmp(argv[i], "--repeat-penalty") && i + 1 < argc) repeat_penalty = (float)atof(argv[++i]);
    else if (!strcmp(argv[i], "--seed") && i + 1 < argc) {
      seed = strtoull(argv[++i], nullptr, 10);
      have_seed = true;
    } else return fprintf(stderr, "Error: unknown argument %s\n", argv[i]), 2;
  }
  if (ids.empty()) return fprintf(stderr, "Error: --prompt-ids is required\n"), 2;
  double t0 = now_s();
  frn_gguf* g;
  if (frn_gguf_open(model, &g)) return die("open");
  frn_config cfg;
  uint32_t ctx_len = 0;
  if (frn_gguf_config(g, &cfg, &ctx_len)) return die("config");
  // generate.rs:91 caps at min(context_length, 4096); an explicit --max-ctx
  // lifts the cap (long-context runs need 4608 positions)
  if (!max_ctx) max_ctx = ctx_len < 4096 ? ctx_len : 4096;
  if (ids.size() + max_new > max_ctx) {
    fprintf(stderr, "Error: prompt (%zu) + max tokens (%u) exceeds context cap %u\n", ids.size(), max_new, max_ctx);
    return 1;
  }
  frn_ctx* ctx;
  if (frn_model_load(g, device, max_ctx, eager ? FRN_FLAG_EAGER : 0, &ctx)) return die("load");
  fprintf(stderr, "weights: uploaded raw to HBM in %.2f s\n", now_s() - t0);
  fprintf(stderr, "prompt: %zu tokens\n", ids.size());
  uint32_t stop[2];
  uint32_t n_stop = 0;
  if (!frn_gguf_meta_u32(g, "tokenizer.ggml.eos_token_id", &stop[n_stop])) ++n_stop;
  if (!frn_gguf_meta_u32(g, "tokenizer.ggml.bos_token_id", &stop[n_stop])) ++n_stop;
  size_t kv_bytes = 2ull * cfg.n_layers * max_ctx * cfg.n_kv_heads * cfg.head_dim * 4;
  fprintf(stderr, "kv cache: %.0f MB for %u positions\n", kv_bytes / (1024.0 * 1024.0), max_ctx);
  frn_timings_enable(ctx, timings);
  if (frn_step_times_enable(ctx, 1)) return die("step times");
  std::vector<uint32_t> out(max_new);
  frn_gen_stats st;
  uint64_t draws = 0;
  if (!have_seed) {  // main.rs:253-259: clock nanoseconds xor the process id
    struct timespec ts;
    clock_gettime(CLOCK_REALTIME, &ts);
    seed = ((uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec) ^ (uint64_t)getpid();
  }
  fprintf(stderr, "sampler: temp %g top-k %u top-p %g repeat-penalty %g seed %llu\n", (double)temp, top_k,
          (double)top_p, (double)repeat_penalty, (unsigned long long)seed);
  // Sampler::sample at temperature 0 is the argmax of the penalized logits
  // (sampler.rs:86-108); without a penalty that is the plain argmax, which
  // the device loop feeds back step to step with no host round trip
  if (temp == 0.0f && repeat_penalty == 1.0f) {
    if (frn_generate_greedy(ctx, ids.data(), (uint32_t)ids.size(), max_new, stop, n_stop, out.data(), &st))
      return die("generate");
  } else {
    if (frn_generate_sampled(ctx, ids.data(), (uint32_t)ids.size(), max_new, temp, top_k, top_p, repeat_penalty,
                             seed, stop, n_stop, out.data(), &st, &draws))
      return die("generate");
  }
  fprintf(stderr, "prefill: %zu tokens in %.3f s (%.3f ms/token)\n", ids.size(), st.prefill_s,
          st.prefill_s * 1000.0 / ids.size());
  // generate.rs:137-140: one line per decode forward, the cache length after it
  std::vector<float> step_ms(st.decode_steps ? st.decode_steps : 1);
  uint32_t n_ms = 0;
  if (frn_step_times(ctx, step_ms.data(), (uint32_t)step_ms.size(), &n_ms)) return die("step times");
  for (uint32_t k = 0; k < n_ms; ++k)
    fprintf(stderr, "[decode %3u: seq %4zu, %8.3f ms/token]\n", k, ids.size() + k + 1, (double)step_ms[k]);
  if (st.decode_steps)
    fprintf(stderr, "decode: %u steps, %.3f ms/token average (%.1f tokens/s)\n", st.decode_steps,
            st.decode_s * 1000.0 / st.decode_steps, st.decode_steps / st.decode_s);
  if (timings) {  // perf.rs:69-96 over the decode phase (reset after the prefill)
    const double wall = st.decode_s * 1000.0;
    frn_timing t[32];
    uint32_t nt = 0;
    if (frn_timings(ctx, t, 32, &nt)) return die("timings");
    fprintf(stderr, "decode op breakdown (%.3f ms wall):\n", wall);
    double accounted = 0.0;
    for (uint32_t i = 0; i < nt; ++i) {
      if (!t[i].calls) continue;
      accounted += t[i].ms;
      fprintf(stderr, "  %-12s %9.3f ms  %5.1f%%  %7llu calls\n", t[i].name, t[i].ms,
              wall > 0 ? 100.0 * t[i].ms / wall : 0.0, (unsigned long long)t[i].calls);
    }
    fprintf(stderr, "  %-12s %9.3f ms  %5.1f%%\n", "unaccounted", wall - accounted,
            wall > 0 ? 100.0 * (wall - accounted) / wall : 0.0);
  }
  fprintf(stderr, "sampler: %llu RNG draws\n", (unsigned long long)draws);
  fprintf(stderr, "generated ids: [");
  for (uint32_t i = 0; i < st.n_generated; ++i) fprintf(stderr, "%s%u", i ? ", " : "", out[i]);
  fprintf(stderr, "]\n");
  frn_destroy(ctx);
  frn_gguf_close(g);
  return 0;
}

static int cmd_dump(int argc, char** argv) {
  if (argc < 2) return fprintf(stderr, "usage: furnace-hip dump-tensor MODEL NAME [--count N] [--offset K]\n"), 2;
  size_t count = 10, offset = 0;
  for (int i = 2; i + 1 < argc; i += 2) {
    if (!strcmp(argv[i], "--count")) count = strtoull(argv[i + 1], nullptr, 10);
    else if (!strcmp(argv[i], "--offset")) offset = strtoull(argv[i + 1], nullptr, 10);
  }
  frn_gguf* g;
  if (frn_gguf_open(argv[0], &g)) return die("open");
  uint32_t type, nd;
  uint64_t dims[4];
  const void* data;
  size_t bytes;
  if (frn_gguf_tensor(g, argv[1], &type, dims, &nd, &data, &bytes)) return die("tensor");
  uint64_t n = 1;
  for (uint32_t d = 0; d < nd; ++d) n *= dims[d];
  if (count == 0 || offset + count > n) {
    fprintf(stderr, "Error: range [%zu, %zu+%zu) out of bounds, tensor has %llu elements\n", offset, offset, count,
            (unsigned long long)n);
    return 1;
  }
  size_t be = type == 12 || type == 14 ? 256 : type == 0 ? 1 : 32, bb = bytes / (n / be);
  size_t first = offset / be, last = (offset + count + be - 1) / be;  // main.rs:144-153
  size_t nv = (last - first) * be;
  void *draw, *dout;
  if (hipMalloc(&draw, (last - first) * bb + 256) || hipMalloc(&dout, nv * 4)) return fprintf(stderr, "Error: hipMalloc\n"), 1;
  if (hipMemcpy(draw, (const char*)data + first * bb, (last - first) * bb, hipMemcpyHostToDevice)) return 1;
  if (frn_dequant(type, draw, (last - first) * bb, nv, (float*)dout, nullptr)) return die("dequant");
  std::vector<float> v(nv);
  if (hipMemcpy(v.data(), dout, nv * 4, hipMemcpyDeviceToHost)) return 1;
  for (size_t i = offset - first * be; i < offset - first * be + count; ++i) printf("%.9g\n", v[i]);
  frn_gguf_close(g);
  return 0;
}

static int cmd_synth(int argc, char** argv) {
  if (argc < 2) return fprintf(stderr, "usage: furnace-hip synth OUT.gguf 0.5b-q8_0|1.5b-q4_k_m|7b-q4_k_m [--seed S]\n"), 2;
  frn_synth_spec s{};
  s.rope_theta = 1e6f;
  s.rms_eps = 1e-6f;
  s.weight_std = 0.02f;
  s.context_length = 32768;
  s.seed = 0;
  for (int i = 2; i + 1 < argc; i += 2)
    if (!strcmp(argv[i], "--seed")) s.seed = strtoull(argv[i + 1], nullptr, 0);
  std::string which = argv[1];
  if (which == "0.5b-q8_0") {
    s.n_layers = 24; s.n_heads = 14; s.n_kv_heads = 2; s.hidden = 896; s.ffn = 4864; s.vocab = 151936;
    s.mix = FRN_MIX_ALL_Q8_0; s.tied = 1; s.embd_type = 8;
  } else if (which == "1.5b-q4_k_m") {
    s.n_layers = 28; s.n_heads = 12; s.n_kv_heads = 2; s.hidden = 1536; s.ffn = 8960; s.vocab = 151936;
    s.mix = FRN_MIX_Q4_K_M; s.tied = 1; s.embd_type = 14;
  } else if (which == "7b-q4_k_m") {
    s.n_layers = 28; s.n_heads = 28; s.n_kv_heads = 4; s.hidden = 3584; s.ffn = 18944; s.vocab = 152064;
    s.mix = FRN_MIX_Q4_K_M; s.tied = 0; s.embd_type = 12; s.output_type = 14;
  } else {
    return fprintf(stderr, "Error: unknown model %s\n", which.c_str()), 2;
  }
  double t0 = now_s();
  if (frn_synth_write(&s, argv[0])) return die("synth");
  fprintf(stderr, "wrote %s in %.1f s\n", argv[0], now_s() - t0);
  return 0;
}

int main(int argc, char** argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: furnace-hip run|dump-tensor|synth ...\n");
    return 2;
  }
  if (!strcmp(argv[1], "run")) return cmd_run(argc - 2, argv + 2);
  if (!strcmp(argv[1], "dump-tensor")) return cmd_dump(argc - 2, argv + 2);
  if (!strcmp(argv[1], "synth")) return cmd_synth(argc - 2, argv + 2);
  fprintf(stderr, "Error: unknown command %s\n", argv[1]);
  return 2;
}
