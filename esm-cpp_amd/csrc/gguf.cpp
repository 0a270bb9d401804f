// GGUF v3 reader (layout: reference src/io/gguf.cpp:1-19; value types
// :36-50; Q8_ESM sizes :178-199). Every read is bounds-checked against the
// mapped file; errors carry the reference reader's messages where it has one.
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace esm_gfx950 {
namespace gguf {
namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read little-endian
constexpr uint32_t kVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;

// gguf metadata value types.
enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32v = 6, kBool = 7, kString = 8, kArray = 9,
  kU64 = 10, kI64 = 11, kF64 = 12
};

// Bounds-checked little-endian cursor over the mapped bytes.
struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  std::string* err;

  bool take(void* dst, size_t n) {
    if (static_cast<size_t>(end - p) < n) {
      *err = "gguf: truncated read";
      return false;
    }
    std::memcpy(dst, p, n);
    p += n;
    return true;
  }
  template <class T>
  bool get(T* v) {
    return take(v, sizeof(T));
  }
  bool str(std::string* s) {
    uint64_t n;
    if (!get(&n)) return false;
    if (static_cast<uint64_t>(end - p) < n) {
      *err = "gguf: string overruns file";
      return false;
    }
    s->assign(reinterpret_cast<const char*>(p), n);
    p += n;
    return true;
  }
  // One scalar of type t, widened to int64 / double / bool / string.
  bool scalar(uint32_t t, Value* v) {
    switch (t) {
      case kU8: { uint8_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = x; return true; }
      case kI8: { int8_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = x; return true; }
      case kU16: { uint16_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = x; return true; }
      case kI16: { int16_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = x; return true; }
      case kU32: { uint32_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = x; return true; }
      case kI32: { int32_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = x; return true; }
      case kU64: { uint64_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = static_cast<int64_t>(x); return true; }
      case kI64: { int64_t x; if (!get(&x)) return false; v->kind = Value::kInt; v->i = x; return true; }
      case kF32v: { float x; if (!get(&x)) return false; v->kind = Value::kFloat; v->f = x; return true; }
      case kF64: { double x; if (!get(&x)) return false; v->kind = Value::kFloat; v->f = x; return true; }
      case kBool: { uint8_t x; if (!get(&x)) return false; v->kind = Value::kBool; v->b = x != 0; return true; }
      case kString: v->kind = Value::kString; return str(&v->s);
      default:
        *err = "gguf: unknown metadata type " + std::to_string(t);
        return false;
    }
  }
  bool value(Value* v) {
    uint32_t t;
    if (!get(&t)) return false;
    if (t != kArray) return scalar(t, v);
    uint32_t et;
    uint64_t n;
    if (!get(&et) || !get(&n)) return false;
    if (et == kArray || et > kF64) {
      *err = "gguf: unsupported array element type " + std::to_string(et);
      return false;
    }
    // Every element takes at least one byte: a count beyond the file is
    // malformed, and checking first keeps the reserve below bounded.
    if (n > static_cast<uint64_t>(end - p)) {
      *err = "gguf: truncated read";
      return false;
    }
    v->kind = et == kString ? Value::kStringArray
              : (et == kF32v || et == kF64) ? Value::kFloatArray
                                            : Value::kIntArray;
    for (uint64_t k = 0; k < n; ++k) {
      Value e;
      if (!scalar(et, &e)) return false;
      if (v->kind == Value::kStringArray) v->strings.push_back(std::move(e.s));
      else if (v->kind == Value::kFloatArray) v->floats.push_back(e.f);
      else v->ints.push_back(e.kind == Value::kBool ? (e.b ? 1 : 0) : e.i);
    }
    return true;
  }
};

// Bytes of a tensor's data, or SIZE_MAX for an unknown type / bad shape.
size_t tensor_bytes(uint32_t type, const std::vector<uint64_t>& shape) {
  uint64_t n = 1;
  for (uint64_t d : shape) {
    if (d != 0 && n > UINT64_MAX / d) return SIZE_MAX;
    n *= d;
  }
  switch (type) {
    case kF32: return n * 4;
    case kF16: return n * 2;
    case kQ8Esm:
      if (shape.size() != 2) return SIZE_MAX;
      return shape[0] * shape[1] + shape[1] * 4;  // [N, K] int8 + [N] fp32
    default: return SIZE_MAX;
  }
}

}  // namespace

File::~File() {
  if (map_) munmap(map_, size_);
}

bool File::open(const std::string& path, std::string* err) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) {
    *err = "gguf: open failed: " + path;
    return false;
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    *err = "gguf: read failed: " + path;
    return false;
  }
  size_ = static_cast<size_t>(st.st_size);
  if (size_ < 24) {
    ::close(fd);
    *err = "gguf: file too small to be GGUF: " + path;
    return false;
  }
  void* m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) {
    *err = "gguf: read failed: " + path;
    return false;
  }
  map_ = m;
  const uint8_t* base = static_cast<const uint8_t*>(map_);
  Cursor c{base, base + size_, err};
  uint32_t magic, version;
  uint64_t ntensors, nmeta;
  if (!c.get(&magic) || !c.get(&version) || !c.get(&ntensors) || !c.get(&nmeta)) return false;
  if (magic != kMagic) {
    *err = "gguf: bad magic in " + path;
    return false;
  }
  if (version != kVersion) {
    *err = "gguf: version " + std::to_string(version) + " not supported (need v3)";
    return false;
  }
  for (uint64_t k = 0; k < nmeta; ++k) {
    std::string key;
    Value v;
    if (!c.str(&key) || !c.value(&v)) return false;
    meta_[std::move(key)] = std::move(v);
  }
  struct Info {
    std::string name;
    Tensor t;
    uint64_t offset;
  };
  std::vector<Info> infos;
  for (uint64_t k = 0; k < ntensors; ++k) {
    Info in;
    uint32_t ndim;
    if (!c.str(&in.name) || !c.get(&ndim)) return false;
    if (ndim > 8) {
      *err = "gguf: tensor " + in.name + " has " + std::to_string(ndim) + " dimensions";
      return false;
    }
    in.t.shape.resize(ndim);
    for (uint32_t d = 0; d < ndim; ++d)
      if (!c.get(&in.t.shape[d])) return false;
    if (!c.get(&in.t.type) || !c.get(&in.offset)) return false;
    infos.push_back(std::move(in));
  }
  uint64_t align = kDefaultAlignment;
  if (const Value* a = meta("general.alignment"); a && a->kind == Value::kInt && a->i > 0) align = a->i;
  const uint64_t header_end = static_cast<uint64_t>(c.p - base);
  const uint64_t data0 = (header_end + align - 1) / align * align;
  if (data0 > size_) {
    *err = "gguf: data section start past EOF";
    return false;
  }
  for (auto& in : infos) {
    const size_t bytes = tensor_bytes(in.t.type, in.t.shape);
    if (bytes == SIZE_MAX) {
      *err = "gguf: unknown tensor type " + std::to_string(in.t.type) + " or bad shape for " + in.name;
      return false;
    }
    if (in.offset > size_ - data0 || bytes > size_ - data0 - in.offset) {
      *err = "gguf: tensor data overruns file: " + in.name;
      return false;
    }
    in.t.data = base + data0 + in.offset;
    in.t.bytes = bytes;
    tensors_[in.name] = std::move(in.t);
  }
  return true;
}

const Value* File::meta(const std::string& key) const {
  auto it = meta_.find(key);
  return it == meta_.end() ? nullptr : &it->second;
}

const Tensor* File::tensor(const std::string& name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

}  // namespace gguf
}  // namespace esm_gfx950
