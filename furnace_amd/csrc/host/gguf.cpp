// GGUF parsing (furnace src/gguf.rs): see gguf.hpp.
#include "gguf.hpp"

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../common.hpp"

namespace frn_host {

namespace {

struct Cursor {  // gguf.rs:23-76
  const uint8_t* d;
  size_t len, pos = 0;
  bool bad = false;
  const uint8_t* take(size_t n) {
    if (bad || n > len - pos) {
      if (!bad) frn_fail(FRN_EINVAL, "unexpected EOF: need %zu bytes at offset %zu", n, pos);
      bad = true;
      return nullptr;
    }
    const uint8_t* p = d + pos;
    pos += n;
    return p;
  }
  uint64_t le(int n) {
    const uint8_t* p = take((size_t)n);
    uint64_t v = 0;
    if (p)
      for (int i = n - 1; i >= 0; --i) v = (v << 8) | p[i];
    return v;
  }
  bool str(std::string* s) {
    uint64_t n = le(8);
    const uint8_t* p = take((size_t)n);
    if (!p) return false;
    s->assign((const char*)p, (size_t)n);
    return true;
  }
};

bool read_value(Cursor& c, uint32_t tag, Value* v, int depth) {  // gguf.rs:101-126
  v->tag = tag;
  switch (tag) {
    case 0: v->u = c.le(1); v->i = (int64_t)v->u; break;
    case 1: v->i = (int8_t)c.le(1); v->u = (uint64_t)v->i; break;
    case 2: v->u = c.le(2); v->i = (int64_t)v->u; break;
    case 3: v->i = (int16_t)c.le(2); v->u = (uint64_t)v->i; break;
    case 4: v->u = c.le(4); v->i = (int64_t)v->u; break;
    case 5: v->i = (int32_t)c.le(4); v->u = (uint64_t)v->i; break;
    case 6: { uint32_t b = (uint32_t)c.le(4); float f; memcpy(&f, &b, 4); v->f = f; break; }
    case 7: v->u = c.le(1) != 0; break;
    case 8: if (!c.str(&v->s)) return false; break;
    case 9: {
      v->arr_tag = (uint32_t)c.le(4);
      v->arr_len = c.le(8);
      if (depth > 4) { frn_fail(FRN_EINVAL, "metadata array nesting too deep"); return false; }
      Value tmp;
      for (uint64_t k = 0; k < v->arr_len && !c.bad; ++k)
        if (!read_value(c, v->arr_tag, &tmp, depth + 1)) return false;
      break;
    }
    case 10: v->u = c.le(8); v->i = (int64_t)v->u; break;
    case 11: v->i = (int64_t)c.le(8); v->u = (uint64_t)v->i; break;
    case 12: { uint64_t b = c.le(8); double f; memcpy(&f, &b, 8); v->f = f; break; }
    default: frn_fail(FRN_EINVAL, "unknown metadata value type tag %u", tag); return false;
  }
  return !c.bad;
}

bool known_type(uint32_t v) {  // gguf.rs:218-242
  static const uint32_t ok[] = {0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 24, 25, 26, 27, 28, 30};
  for (uint32_t k : ok)
    if (k == v) return true;
  return false;
}

}  // namespace

uint64_t TensorInfo::n_elements() const {
  uint64_t n = 1;
  for (uint64_t d : dims) n *= d;
  return n;
}

File::~File() {
  if (map) munmap(map, map_len);
}

bool block_layout(uint32_t type, size_t* elems, size_t* bytes) {
  switch (type) {
    case 0: *elems = 1; *bytes = 4; return true;
    case 1: *elems = 1; *bytes = 2; return true;
    case 8: *elems = 32; *bytes = 34; return true;
    case 6: *elems = 32; *bytes = 22; return true;
    case 12: *elems = 256; *bytes = 144; return true;
    case 14: *elems = 256; *bytes = 210; return true;
    default: return false;
  }
}

frn_status parse(const uint8_t* data, size_t len, File* f) {
  Cursor c{data, len};
  const uint8_t* magic = c.take(4);
  if (!magic) return FRN_EINVAL;
  if (memcmp(magic, "GGUF", 4) != 0)
    return frn_fail(FRN_EINVAL, "not a GGUF file (bad magic %02x %02x %02x %02x)", magic[0], magic[1], magic[2], magic[3]);
  f->version = (uint32_t)c.le(4);
  if (c.bad) return FRN_EINVAL;
  if (f->version != 2 && f->version != 3)
    return frn_fail(FRN_EINVAL, "unsupported GGUF version %u (only 2 and 3)", f->version);
  uint64_t n_t = c.le(8), n_kv = c.le(8);
  if (c.bad) return FRN_EINVAL;
  for (uint64_t k = 0; k < n_kv; ++k) {
    std::string key;
    if (!c.str(&key)) return FRN_EINVAL;
    uint32_t tag = (uint32_t)c.le(4);
    Value v;
    if (c.bad || !read_value(c, tag, &v, 0)) return FRN_EINVAL;
    f->meta[key] = v;
  }
  for (uint64_t k = 0; k < n_t; ++k) {  // gguf.rs:278-290
    TensorInfo t;
    if (!c.str(&t.name)) return FRN_EINVAL;
    uint32_t nd = (uint32_t)c.le(4);
    if (c.bad) return FRN_EINVAL;
    if (nd > 4) return frn_fail(FRN_EINVAL, "tensor '%s' has %u dims, max is 4", t.name.c_str(), nd);
    for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.le(8));
    t.type = (uint32_t)c.le(4);
    if (c.bad) return FRN_EINVAL;
    if (!known_type(t.type)) return frn_fail(FRN_EINVAL, "tensor '%s': unsupported ggml tensor type %u", t.name.c_str(), t.type);
    t.offset = c.le(8);
    if (c.bad) return FRN_EINVAL;
    f->tensors.push_back(std::move(t));
  }
  uint64_t align = 32;  // gguf.rs:344-354
  auto it = f->meta.find("general.alignment");
  if (it != f->meta.end() && (it->second.tag == 4 || (it->second.tag == 10 && it->second.u <= 0xFFFFFFFFull)))
    align = it->second.u;
  if (align == 0 || (align & (align - 1)))
    return frn_fail(FRN_EINVAL, "general.alignment %llu is not a power of two", (unsigned long long)align);
  size_t ds = (c.pos + (size_t)align - 1) / (size_t)align * (size_t)align;
  if (ds > len)
    return frn_fail(FRN_EINVAL, "file truncated: tensor data would start at %zu but file is %zu bytes", ds, len);
  f->data_start = ds;
  return FRN_OK;
}

frn_status open(const char* path, File* f) {
  int fd = ::open(path, O_RDONLY);
  if (fd < 0) return frn_fail(FRN_EINVAL, "cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st)) {
    ::close(fd);
    return frn_fail(FRN_EINVAL, "cannot stat %s", path);
  }
  size_t len = (size_t)st.st_size;
  void* m = len ? mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
  ::close(fd);
  if (len && m == MAP_FAILED) return frn_fail(FRN_EINVAL, "mmap failed for %s", path);
  f->map = m;
  f->map_len = len;
  return parse((const uint8_t*)m, len, f);
}

frn_status tensor(const File& f, const std::string& name, const TensorInfo** info, const uint8_t** data, size_t* bytes) {
  for (const TensorInfo& t : f.tensors) {
    if (t.name != name) continue;
    size_t be, bb;
    if (!block_layout(t.type, &be, &bb)) return frn_fail(FRN_EDTYPE, "dtype %u not supported yet", t.type);
    uint64_t n = t.n_elements();
    if (n % be)
      return frn_fail(FRN_ESHAPE, "tensor '%s' has %llu elements, not a multiple of block size %zu", t.name.c_str(),
                      (unsigned long long)n, be);
    size_t size = (size_t)(n / be) * bb, start = f.data_start + (size_t)t.offset;
    if (start < f.data_start || size > f.map_len || start > f.map_len - size)
      return frn_fail(FRN_EINVAL, "tensor '%s' data [%zu, %zu+%zu) runs past end of file (%zu bytes)", t.name.c_str(),
                      start, start, size, f.map_len);
    *info = &t;
    *data = (const uint8_t*)f.map + start;
    *bytes = size;
    return FRN_OK;
  }
  return frn_fail(FRN_EINVAL, "no tensor named '%s'", name.c_str());
}

frn_status meta_u32(const File& f, const char* key, uint32_t* out) {  // gguf.rs:128-134, 389-394
  auto it = f.meta.find(key);
  if (it != f.meta.end()) {
    const Value& v = it->second;
    if (v.tag == 4 || (v.tag == 10 && v.u <= 0xFFFFFFFFull)) {
      *out = (uint32_t)v.u;
      return FRN_OK;
    }
  }
  return frn_fail(FRN_EINVAL, "metadata key '%s' missing or not a u32", key);
}

frn_status meta_f32(const File& f, const char* key, float* out) {  // gguf.rs:150-156, 396-401
  auto it = f.meta.find(key);
  if (it != f.meta.end() && (it->second.tag == 6 || it->second.tag == 12)) {
    *out = (float)it->second.f;
    return FRN_OK;
  }
  return frn_fail(FRN_EINVAL, "metadata key '%s' missing or not a float", key);
}

}  // namespace frn_host
