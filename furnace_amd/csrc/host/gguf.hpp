// GGUF reader for the host side (restates furnace src/gguf.rs): a
// bounds-checked cursor over a read-only mmap, typed metadata, the tensor
// table in ggml dim order, and zero-copy tensor slices.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/furnace_hip.h"

namespace frn_host {

struct Value {  // gguf.rs:83-97 GgufValue (arrays keep only their length)
  uint32_t tag = 0;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0;
  std::string s;
  uint32_t arr_tag = 0;
  uint64_t arr_len = 0;
};

struct TensorInfo {  // gguf.rs:246-254
  std::string name;
  std::vector<uint64_t> dims;  // ggml order: dims[0] contiguous
  uint32_t type = 0;
  uint64_t offset = 0;
  uint64_t n_elements() const;
};

struct File {
  void* map = nullptr;
  size_t map_len = 0;
  uint32_t version = 0;
  std::unordered_map<std::string, Value> meta;
  std::vector<TensorInfo> tensors;
  size_t data_start = 0;
  ~File();
};

// gguf.rs:315-363; returns FRN_OK or FRN_EINVAL with the reference's message.
frn_status parse(const uint8_t* data, size_t len, File* f);
frn_status open(const char* path, File* f);
// gguf.rs:206-216 (elements, bytes) per block; false for unknown types
bool block_layout(uint32_t type, size_t* elems, size_t* bytes);
// gguf.rs:412-434
frn_status tensor(const File& f, const std::string& name, const TensorInfo** info, const uint8_t** data, size_t* bytes);
frn_status meta_u32(const File& f, const char* key, uint32_t* out);
frn_status meta_f32(const File& f, const char* key, float* out);

}  // namespace frn_host
