// GGUF reader (see gguf.hpp). Every read is bounds-checked against the file size, so a truncated
// or corrupt file is rejected with a message instead of read past its end.
#include "gguf.hpp"

#include <cstdio>
#include <cstring>
#include <sstream>

namespace uk {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint64_t kMaxString = uint64_t(1) << 24;
constexpr uint64_t kMaxArray = uint64_t(1) << 28;
constexpr uint64_t kMaxCount = uint64_t(1) << 24;

// GGUF metadata value types.
enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kStr = 8, kArr = 9,
  kU64 = 10, kI64 = 11, kF64 = 12
};

class Cursor {
 public:
  Cursor(std::FILE* f, uint64_t size) : f_(f), size_(size) {}
  bool bytes(void* dst, uint64_t n) {
    if (!ok_ || n > size_ - pos_) return fail("unexpected end of file");
    if (n && std::fread(dst, 1, n, f_) != n) return fail("read error");
    pos_ += n;
    return true;
  }
  bool skip(uint64_t n) {
    if (!ok_ || n > size_ - pos_) return fail("unexpected end of file");
    if (std::fseek(f_, (long)n, SEEK_CUR) != 0) return fail("seek error");
    pos_ += n;
    return true;
  }
  template <class T>
  bool get(T* v) { return bytes(v, sizeof(T)); }
  bool str(std::string* s) {
    uint64_t n = 0;
    if (!get(&n)) return false;
    if (n > kMaxString) return fail("string length " + std::to_string(n) + " out of range");
    s->resize(n);
    return bytes(s->data(), n);
  }
  bool fail(const std::string& m) {
    if (ok_) msg_ = m + " at byte " + std::to_string(pos_);
    ok_ = false;
    return false;
  }
  uint64_t pos() const { return pos_; }
  const std::string& msg() const { return msg_; }

 private:
  std::FILE* f_;
  uint64_t size_, pos_ = 0;
  bool ok_ = true;
  std::string msg_;
};

uint64_t scalar_size(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

bool scalar_text(Cursor& c, uint32_t t, std::string* out) {
  std::ostringstream os;
  switch (t) {
    case kU8: { uint8_t v; if (!c.get(&v)) return false; os << unsigned(v); break; }
    case kI8: { int8_t v; if (!c.get(&v)) return false; os << int(v); break; }
    case kU16: { uint16_t v; if (!c.get(&v)) return false; os << v; break; }
    case kI16: { int16_t v; if (!c.get(&v)) return false; os << v; break; }
    case kU32: { uint32_t v; if (!c.get(&v)) return false; os << v; break; }
    case kI32: { int32_t v; if (!c.get(&v)) return false; os << v; break; }
    case kF32: { float v; if (!c.get(&v)) return false; os << v; break; }
    case kBool: { uint8_t v; if (!c.get(&v)) return false; os << (v ? "true" : "false"); break; }
    case kU64: { uint64_t v; if (!c.get(&v)) return false; os << v; break; }
    case kI64: { int64_t v; if (!c.get(&v)) return false; os << v; break; }
    case kF64: { double v; if (!c.get(&v)) return false; os << v; break; }
    case kStr: return c.str(out);
    default: return c.fail("unknown metadata type " + std::to_string(t));
  }
  *out = os.str();
  return true;
}

bool value_text(Cursor& c, uint32_t t, std::string* out) {
  if (t != kArr) return scalar_text(c, t, out);
  uint32_t et = 0;
  uint64_t n = 0;
  if (!c.get(&et) || !c.get(&n)) return false;
  if (n > kMaxArray) return c.fail("array length out of range");
  if (et == kArr) return c.fail("nested arrays are not part of the format");
  if (et == kStr) {
    std::string s;
    for (uint64_t i = 0; i < n; ++i)
      if (!c.str(&s)) return false;
  } else {
    const uint64_t es = scalar_size(et);
    if (!es) return c.fail("unknown array element type " + std::to_string(et));
    if (!c.skip(es * n)) return false;
  }
  *out = "[" + std::to_string(n) + " x type " + std::to_string(et) + "]";
  return true;
}

// Bytes of a tensor of `elems` elements with row length ne0, for the types this reader sizes.
uint64_t tensor_bytes(uint32_t type, int64_t ne0, uint64_t elems) {
  switch (type) {
    case kGgmlF32: return elems * 4;
    case kGgmlF16: case kGgmlBF16: return elems * 2;
    case kGgmlQ8_0: return (ne0 % 32) ? 0 : elems / 32 * 34;
    default: return 0;
  }
}

}  // namespace

const char* ggml_type_name(uint32_t t) {
  switch (t) {
    case kGgmlF32: return "f32";
    case kGgmlF16: return "f16";
    case kGgmlQ8_0: return "q8_0";
    case kGgmlBF16: return "bf16";
    default: return "other";
  }
}

std::optional<GgufFile> gguf_open(const std::string& path, std::string* err) {
  std::FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) {
    if (err) *err = "cannot open " + path;
    return std::nullopt;
  }
  GgufFile g;
  g.path = path;
  std::fseek(f, 0, SEEK_END);
  g.file_size = (uint64_t)std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  Cursor c(f, g.file_size);
  auto bail = [&](const std::string& m) -> std::optional<GgufFile> {
    std::fclose(f);
    if (err) *err = path + ": " + m;
    return std::nullopt;
  };
  uint32_t magic = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  if (!c.get(&magic)) return bail(c.msg());
  if (magic != kMagic) return bail("not a GGUF file (bad magic)");
  if (!c.get(&g.version) || !c.get(&n_tensors) || !c.get(&n_kv)) return bail(c.msg());
  if (g.version < 2 || g.version > 3) return bail("GGUF version " + std::to_string(g.version) + " is not 2 or 3");
  if (n_tensors > kMaxCount || n_kv > kMaxCount) return bail("tensor or metadata count out of range");
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key, val;
    uint32_t t = 0;
    if (!c.str(&key) || !c.get(&t) || !value_text(c, t, &val)) return bail(c.msg());
    if (key == "general.alignment") {
      if (t != kU32) return bail("general.alignment must be u32");
      g.alignment = std::stoull(val);
      if (g.alignment == 0 || (g.alignment & (g.alignment - 1))) return bail("general.alignment must be a power of two");
    }
    g.kv[key] = val;
  }
  std::vector<uint64_t> rel;
  for (uint64_t i = 0; i < n_tensors; ++i) {
    GgufTensor t;
    uint32_t nd = 0;
    if (!c.str(&t.name) || !c.get(&nd)) return bail(c.msg());
    if (nd == 0 || nd > 4) return bail("tensor '" + t.name + "' has " + std::to_string(nd) + " dims (1..4 allowed)");
    uint64_t elems = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      uint64_t ne = 0;
      if (!c.get(&ne)) return bail(c.msg());
      if (ne == 0 || ne > (uint64_t(1) << 40) || elems > (uint64_t(1) << 62) / ne)
        return bail("tensor '" + t.name + "' has an out-of-range dimension");
      elems *= ne;
      t.ne.push_back((int64_t)ne);
    }
    uint64_t off = 0;
    if (!c.get(&t.type) || !c.get(&off)) return bail(c.msg());
    t.nbytes = tensor_bytes(t.type, t.ne[0], elems);
    rel.push_back(off);
    g.tensors.push_back(std::move(t));
  }
  g.data_offset = (c.pos() + g.alignment - 1) / g.alignment * g.alignment;
  for (size_t i = 0; i < g.tensors.size(); ++i) {
    GgufTensor& t = g.tensors[i];
    if (rel[i] % g.alignment) return bail("tensor '" + t.name + "' offset is not aligned");
    t.offset = g.data_offset + rel[i];
    if (t.offset > g.file_size || t.nbytes > g.file_size - t.offset)
      return bail("tensor '" + t.name + "' extends past the end of the file");
  }
  std::fclose(f);
  return g;
}

int gguf_find(const GgufFile& f, const std::string& name) {
  for (size_t i = 0; i < f.tensors.size(); ++i)
    if (f.tensors[i].name == name) return (int)i;
  return -1;
}

bool gguf_read(const GgufFile& f, int index, void* dst, uint64_t cap, std::string* err) {
  if (index < 0 || index >= (int)f.tensors.size()) {
    if (err) *err = "tensor index out of range";
    return false;
  }
  const GgufTensor& t = f.tensors[index];
  if (!t.nbytes) {
    if (err) *err = "tensor '" + t.name + "' has a type this reader does not size (" + ggml_type_name(t.type) + ")";
    return false;
  }
  if (cap < t.nbytes) {
    if (err) *err = "destination holds " + std::to_string(cap) + " bytes, tensor needs " + std::to_string(t.nbytes);
    return false;
  }
  std::FILE* fp = std::fopen(f.path.c_str(), "rb");
  if (!fp) {
    if (err) *err = "cannot open " + f.path;
    return false;
  }
  bool ok = std::fseek(fp, (long)t.offset, SEEK_SET) == 0 &&
            std::fread(dst, 1, t.nbytes, fp) == t.nbytes;
  std::fclose(fp);
  if (!ok && err) *err = "read of tensor '" + t.name + "' failed";
  return ok;
}

}  // namespace uk
