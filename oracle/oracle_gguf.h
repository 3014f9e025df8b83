/* Test infrastructure only: the oracle's GGUF reader (restates src/gguf.rs). */
#ifndef FURNACE_ORACLE_GGUF_H
#define FURNACE_ORACLE_GGUF_H
#include <stddef.h>
#include <stdint.h>
#include "oracle.h"
typedef struct {
  const char* key;
  size_t key_len;
  uint32_t type;
  uint64_t u;
  int64_t i;
  double f;
  const char* str;
  size_t str_len;
  uint32_t arr_type;
  uint64_t arr_len;
} gguf_kv;
typedef struct {
  const char* name;
  size_t name_len;
  uint32_t n_dims, type;
  uint64_t dims[4];
  uint64_t offset;
} gguf_tensor;
typedef struct {
  void* map;
  size_t map_len;
  const uint8_t* data;
  size_t len, data_start;
  uint32_t version;
  gguf_kv* kv;
  size_t n_kv;
  gguf_tensor* tensors;
  size_t n_tensors;
} gguf_file;
int gguf_parse(const uint8_t* data, size_t len, gguf_file* g);
int gguf_open(const char* path, gguf_file* g);
void gguf_close(gguf_file* g);
const gguf_kv* gguf_find(const gguf_file* g, const char* key);
const gguf_tensor* gguf_find_tensor(const gguf_file* g, const char* name);
int gguf_tensor_data(const gguf_file* g, const gguf_tensor* t, const uint8_t** p, size_t* bytes);
int gguf_u32(const gguf_file* g, const char* key, uint32_t* out);
int gguf_f32(const gguf_file* g, const char* key, float* out);
#endif
