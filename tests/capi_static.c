/*
 * A C caller of the engine ABI, linked statically against libfurnace_hip.a
 * (the link a Rust build.rs makes with `cargo:rustc-link-lib=static=furnace_hip`).
 * It loads a GGUF the way furnace's Model::load does (src/model.rs:520-552:
 * one frn_upload per tensor, by name), then prefills the prompt and decodes
 * greedily with frn_decode_greedy, and compares the ids with the expected
 * ones.
 *
 * usage: capi_static MODEL.gguf PROMPT_IDS EXPECTED_IDS   (ids comma-separated)
 * exit status 0 when every expected id matches.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../include/furnace_host.h"

#define MAX_IDS 4096

static int parse_ids(const char* s, uint32_t* out) {
  int n = 0;
  while (*s && n < MAX_IDS) {
    char* end;
    unsigned long v = strtoul(s, &end, 10);
    if (end == s) break;
    out[n++] = (uint32_t)v;
    s = *end ? end + 1 : end;
  }
  return n;
}

static int fail(const char* what) {
  fprintf(stderr, "capi_static: %s: %s\n", what, frn_last_error());
  return 2;
}

/* one tensor from the file to the device, by name (Model::load's lookups) */
static int upload(frn_ctx* ctx, const frn_gguf* g, const char* name) {
  uint32_t type = 0, nd = 0;
  uint64_t dims[4] = {0, 0, 0, 0};
  const void* data = NULL;
  size_t bytes = 0;
  if (frn_gguf_tensor(g, name, &type, dims, &nd, &data, &bytes)) return fail(name);
  uint64_t in = nd ? dims[0] : 1, out = 1;
  for (uint32_t d = 1; d < nd; ++d) out *= dims[d];
  if (frn_upload(ctx, name, type, out, in, data, bytes)) return fail(name);
  return 0;
}

int main(int argc, char** argv) {
  static uint32_t prompt[MAX_IDS], want[MAX_IDS], got[MAX_IDS];
  if (argc != 4) {
    fprintf(stderr, "usage: %s MODEL.gguf PROMPT_IDS EXPECTED_IDS\n", argv[0]);
    return 2;
  }
  const int n_prompt = parse_ids(argv[2], prompt), n_want = parse_ids(argv[3], want);
  if (n_prompt < 1 || n_want < 1) return fprintf(stderr, "capi_static: empty id list\n"), 2;
  frn_gguf* g = NULL;
  if (frn_gguf_open(argv[1], &g)) return fail("open");
  frn_config cfg;
  uint32_t ctx_len = 0;
  if (frn_gguf_config(g, &cfg, &ctx_len)) return fail("config");
  cfg.max_ctx = (uint32_t)(n_prompt + n_want + 1);
  cfg.flags = 0;
  frn_ctx* ctx = NULL;
  if (frn_create(&cfg, 0, &ctx)) return fail("frn_create");
  char name[96];
  int rc = upload(ctx, g, "token_embd.weight") || upload(ctx, g, "output_norm.weight") ||
           (!cfg.tied_lm_head && upload(ctx, g, "output.weight"));
  static const char* const per_layer[] = {"attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight",
                                          "attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.weight",
                                          "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
  for (uint32_t l = 0; !rc && l < cfg.n_layers; ++l)
    for (size_t k = 0; !rc && k < sizeof per_layer / sizeof per_layer[0]; ++k) {
      snprintf(name, sizeof name, "blk.%u.%s", l, per_layer[k]);
      rc = upload(ctx, g, name);
    }
  if (rc) return rc;
  if (frn_finalize(ctx)) return fail("frn_finalize");
  uint32_t next = 0, done = 0;
  if (frn_prefill(ctx, prompt, (uint32_t)n_prompt, &next)) return fail("frn_prefill");
  got[0] = next;
  if (n_want > 1 && frn_decode_greedy(ctx, next, (uint32_t)(n_want - 1), NULL, 0, got + 1, &done))
    return fail("frn_decode_greedy");
  int bad = 0;
  for (int i = 0; i < n_want; ++i)
    if (got[i] != want[i]) {
      if (!bad) fprintf(stderr, "capi_static: id %d is %u, expected %u\n", i, got[i], want[i]);
      ++bad;
    }
  frn_destroy(ctx);
  frn_gguf_close(g);
  printf("capi_static: %d of %d ids match\n", n_want - bad, n_want);
  return bad ? 1 : 0;
}
