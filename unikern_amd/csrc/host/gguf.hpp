// GGUF reader: the header, metadata and tensor directory of a GGUF file (version 2 or 3), and
// the bytes of one tensor. Q8_0 tensors are stored exactly as the Q8_0 GEMM consumes them
// (N rows of K/32 blocks of {binary16 d, int8 q[32]}), so a weight tensor goes to HBM as one copy.
//
// Layout (the published GGUF format, as the reference's probe/phase63_gguf_header.py reads it):
//   u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count,
//   kv_count x { string key, u32 type, value },
//   tensor_count x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset },
//   padding to general.alignment (default 32), then the data section; offsets are relative to it.
// Strings are u64 length + bytes; arrays are u32 element type + u64 count + elements.
#pragma once

#include <cstdint>
#include <map>
#include <optional>
#include <string>
#include <vector>

namespace uk {

enum GgmlType : uint32_t { kGgmlF32 = 0, kGgmlF16 = 1, kGgmlQ8_0 = 8, kGgmlBF16 = 30 };

struct GgufTensor {
  std::string name;
  std::vector<int64_t> ne;  // ne[0] is the innermost (row) length
  uint32_t type = 0;
  uint64_t offset = 0;      // absolute file offset of the first byte
  uint64_t nbytes = 0;      // 0 for a type whose size this reader does not know
};

struct GgufFile {
  std::string path;
  uint32_t version = 0;
  uint64_t alignment = 32;
  uint64_t data_offset = 0;
  uint64_t file_size = 0;
  std::map<std::string, std::string> kv;  // scalars and strings as text; arrays as "[n x type]"
  std::vector<GgufTensor> tensors;
};

std::optional<GgufFile> gguf_open(const std::string& path, std::string* err);
int gguf_find(const GgufFile& f, const std::string& name);
bool gguf_read(const GgufFile& f, int index, void* dst, uint64_t cap, std::string* err);
const char* ggml_type_name(uint32_t t);

}  // namespace uk
