/* Test infrastructure only (the oracle).  Restates src/gguf.rs parse /
 * open / tensor: bounds-checked reads over an mmap, metadata values, tensor
 * table, data blob at the next multiple of general.alignment (default 32). */
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include "oracle_gguf.h"
#include "oracle_internal.h"

typedef struct {
  const uint8_t* d;
  size_t len, pos;
  int bad;
} cur_t;

static const uint8_t* take(cur_t* c, size_t n) { /* gguf.rs:33-44 */
  if (c->bad || n > c->len - c->pos) {
    if (!c->bad) orc_set_error("unexpected EOF: need %zu bytes at offset %zu", n, c->pos);
    c->bad = 1;
    return NULL;
  }
  const uint8_t* p = c->d + c->pos;
  c->pos += n;
  return p;
}
static uint64_t rd(cur_t* c, int n) {
  const uint8_t* p = take(c, (size_t)n);
  uint64_t v = 0;
  if (!p) return 0;
  for (int i = n - 1; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}

/* gguf.rs:101-126: value types 0..12 (9 = array). */
static int read_value(cur_t* c, uint32_t tag, gguf_kv* kv, int depth) {
  switch (tag) {
    case 0: kv->u = rd(c, 1); kv->i = (int64_t)kv->u; break;
    case 1: kv->i = (int8_t)rd(c, 1); kv->u = (uint64_t)kv->i; break;
    case 2: kv->u = rd(c, 2); kv->i = (int64_t)kv->u; break;
    case 3: kv->i = (int16_t)rd(c, 2); kv->u = (uint64_t)kv->i; break;
    case 4: kv->u = rd(c, 4); kv->i = (int64_t)kv->u; break;
    case 5: kv->i = (int32_t)rd(c, 4); kv->u = (uint64_t)kv->i; break;
    case 6: { uint32_t b = (uint32_t)rd(c, 4); float f; memcpy(&f, &b, 4); kv->f = f; break; }
    case 7: kv->u = rd(c, 1) != 0; break;
    case 8: {
      uint64_t n = rd(c, 8);
      kv->str = (const char*)take(c, (size_t)n);
      kv->str_len = (size_t)n;
      break;
    }
    case 9: {
      uint32_t et = (uint32_t)rd(c, 4);
      uint64_t n = rd(c, 8);
      kv->arr_type = et;
      kv->arr_len = n;
      if (depth > 4) { orc_set_error("metadata array nesting too deep"); return -1; }
      for (uint64_t i = 0; i < n && !c->bad; ++i) {
        gguf_kv tmp;
        memset(&tmp, 0, sizeof tmp);
        if (read_value(c, et, &tmp, depth + 1)) return -1;
      }
      break;
    }
    case 10: kv->u = rd(c, 8); kv->i = (int64_t)kv->u; break;
    case 11: kv->i = (int64_t)rd(c, 8); kv->u = (uint64_t)kv->i; break;
    case 12: { uint64_t b = rd(c, 8); double f; memcpy(&f, &b, 8); kv->f = f; break; }
    default: orc_set_error("unknown metadata value type tag %u", tag); return -1;
  }
  return c->bad ? -1 : 0;
}

static int known_type(uint32_t v) { /* gguf.rs:218-242 */
  static const uint32_t ok[] = {0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 24, 25, 26, 27, 28, 30};
  for (size_t i = 0; i < sizeof ok / sizeof ok[0]; ++i)
    if (ok[i] == v) return 1;
  return 0;
}

/* gguf.rs:315-363 parse */
int gguf_parse(const uint8_t* data, size_t len, gguf_file* g) {
  cur_t c = {data, len, 0, 0};
  const uint8_t* magic = take(&c, 4);
  if (!magic) return -1;
  if (memcmp(magic, "GGUF", 4) != 0) {
    orc_set_error("not a GGUF file (bad magic %02x %02x %02x %02x)", magic[0], magic[1], magic[2], magic[3]);
    return -1;
  }
  g->version = (uint32_t)rd(&c, 4);
  if (c.bad) return -1;
  if (g->version != 2 && g->version != 3) {
    orc_set_error("unsupported GGUF version %u (only 2 and 3)", g->version);
    return -1;
  }
  uint64_t n_t = rd(&c, 8), n_kv = rd(&c, 8);
  if (c.bad) return -1;
  if (n_kv > len || n_t > len) { orc_set_error("unexpected EOF: counts exceed file"); return -1; }
  g->kv = (gguf_kv*)calloc(n_kv ? n_kv : 1, sizeof(gguf_kv));
  g->n_kv = 0;
  for (uint64_t i = 0; i < n_kv; ++i) {
    gguf_kv* kv = &g->kv[i];
    uint64_t kl = rd(&c, 8);
    kv->key = (const char*)take(&c, (size_t)kl);
    kv->key_len = (size_t)kl;
    kv->type = (uint32_t)rd(&c, 4);
    if (c.bad || read_value(&c, kv->type, kv, 0)) return -1;
    g->n_kv = i + 1;
  }
  g->tensors = (gguf_tensor*)calloc(n_t ? n_t : 1, sizeof(gguf_tensor));
  g->n_tensors = 0;
  for (uint64_t i = 0; i < n_t; ++i) { /* gguf.rs:278-290 */
    gguf_tensor* t = &g->tensors[i];
    uint64_t nl = rd(&c, 8);
    t->name = (const char*)take(&c, (size_t)nl);
    t->name_len = (size_t)nl;
    t->n_dims = (uint32_t)rd(&c, 4);
    if (c.bad) return -1;
    if (t->n_dims > 4) { orc_set_error("tensor has %u dims, max is 4", t->n_dims); return -1; }
    for (uint32_t d = 0; d < t->n_dims; ++d) t->dims[d] = rd(&c, 8);
    t->type = (uint32_t)rd(&c, 4);
    if (c.bad) return -1;
    if (!known_type(t->type)) { orc_set_error("unsupported ggml tensor type %u", t->type); return -1; }
    t->offset = rd(&c, 8);
    if (c.bad) return -1;
    g->n_tensors = i + 1;
  }
  uint64_t align = 32;
  const gguf_kv* a = gguf_find(g, "general.alignment");
  if (a && (a->type == 4 || a->type == 10) && a->u <= 0xFFFFFFFFu) align = a->u;
  if (align == 0 || (align & (align - 1))) {
    orc_set_error("general.alignment %llu is not a power of two", (unsigned long long)align);
    return -1;
  }
  size_t ds = (c.pos + (size_t)align - 1) / (size_t)align * (size_t)align;
  if (ds > len) {
    orc_set_error("file truncated: tensor data would start at %zu but file is %zu bytes", ds, len);
    return -1;
  }
  g->data = data;
  g->len = len;
  g->data_start = ds;
  return 0;
}

const gguf_kv* gguf_find(const gguf_file* g, const char* key) {
  size_t kl = strlen(key);
  for (size_t i = 0; i < g->n_kv; ++i)
    if (g->kv[i].key_len == kl && memcmp(g->kv[i].key, key, kl) == 0) return &g->kv[i];
  return NULL;
}

const gguf_tensor* gguf_find_tensor(const gguf_file* g, const char* name) {
  size_t nl = strlen(name);
  for (size_t i = 0; i < g->n_tensors; ++i)
    if (g->tensors[i].name_len == nl && memcmp(g->tensors[i].name, name, nl) == 0) return &g->tensors[i];
  return NULL;
}

/* gguf.rs:262-276 byte_size + :412-434 tensor */
int gguf_tensor_data(const gguf_file* g, const gguf_tensor* t, const uint8_t** p, size_t* bytes) {
  size_t be, bb, n = 1;
  for (uint32_t d = 0; d < t->n_dims; ++d) n *= (size_t)t->dims[d];
  if (orc_block_layout(t->type, &be, &bb)) { orc_set_error("dtype %u not supported yet", t->type); return -1; }
  if (n % be) { orc_set_error("tensor has %zu elements, not a multiple of block size %zu", n, be); return -1; }
  size_t size = n / be * bb, start = g->data_start + (size_t)t->offset;
  if (start < g->data_start || size > g->len || start > g->len - size) {
    orc_set_error("tensor data runs past end of file (%zu bytes)", g->len);
    return -1;
  }
  *p = g->data + start;
  *bytes = size;
  return 0;
}

/* gguf.rs:366-380 open (read-only mmap) */
int gguf_open(const char* path, gguf_file* g) {
  memset(g, 0, sizeof *g);
  int fd = open(path, O_RDONLY);
  if (fd < 0) { orc_set_error("cannot open %s", path); return -1; }
  struct stat st;
  if (fstat(fd, &st)) { close(fd); orc_set_error("cannot stat %s", path); return -1; }
  size_t len = (size_t)st.st_size;
  void* m = len ? mmap(NULL, len, PROT_READ, MAP_PRIVATE, fd, 0) : NULL;
  close(fd);
  if (len && m == MAP_FAILED) { orc_set_error("mmap failed for %s", path); return -1; }
  g->map = m;
  g->map_len = len;
  if (gguf_parse((const uint8_t*)m, len, g)) { gguf_close(g); return -1; }
  return 0;
}

void gguf_close(gguf_file* g) {
  if (g->map) munmap(g->map, g->map_len);
  free(g->kv);
  free(g->tensors);
  memset(g, 0, sizeof *g);
}

/* gguf.rs:128-163 as_u32 / as_f32 */
int gguf_u32(const gguf_file* g, const char* key, uint32_t* out) {
  const gguf_kv* kv = gguf_find(g, key);
  if (kv && kv->type == 4) { *out = (uint32_t)kv->u; return 0; }
  if (kv && kv->type == 10 && kv->u <= 0xFFFFFFFFu) { *out = (uint32_t)kv->u; return 0; }
  orc_set_error("metadata key '%s' missing or not a u32", key);
  return -1;
}
int gguf_f32(const gguf_file* g, const char* key, float* out) {
  const gguf_kv* kv = gguf_find(g, key);
  if (kv && (kv->type == 6 || kv->type == 12)) { *out = (float)kv->f; return 0; }
  orc_set_error("metadata key '%s' missing or not a float", key);
  return -1;
}
