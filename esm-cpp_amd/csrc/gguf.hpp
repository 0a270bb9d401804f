// GGUF v3 container reader for esm.cpp weight files (reference
// src/io/gguf.cpp:1-19 documents the layout): magic "GGUF", version 3, tensor
// and metadata counts, metadata key/value pairs, tensor infos (name, dims,
// type, offset), padding to general.alignment (default 32), tensor data.
// The file is memory-mapped read-only; tensor data pointers stay valid while
// the GgufFile lives.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace esm_gfx950 {
namespace gguf {

// Tensor element types used by esm.cpp (reference include/esm_cpp/io.h:53-57):
// F32 and F16 follow ggml's numbering; Q8_ESM is esm.cpp's per-channel int8
// blob [N, K] int8 followed by [N] fp32 scales, wire shape [K, N].
enum TensorType : uint32_t { kF32 = 0, kF16 = 1, kQ8Esm = 100 };

struct Value {
  enum Kind { kNone, kInt, kFloat, kBool, kString, kIntArray, kFloatArray, kStringArray } kind = kNone;
  int64_t i = 0;
  double f = 0.0;
  bool b = false;
  std::string s;
  std::vector<int64_t> ints;
  std::vector<double> floats;
  std::vector<std::string> strings;
};

struct Tensor {
  uint32_t type = 0;
  std::vector<uint64_t> shape;  // as on the wire (fastest dimension first)
  const uint8_t* data = nullptr;
  size_t bytes = 0;
};

class File {
 public:
  File() = default;
  File(const File&) = delete;
  File& operator=(const File&) = delete;
  ~File();
  // Parses `path`; false with a message in *err on any malformed input.
  bool open(const std::string& path, std::string* err);
  const Value* meta(const std::string& key) const;
  const Tensor* tensor(const std::string& name) const;
  size_t tensor_count() const { return tensors_.size(); }

 private:
  void* map_ = nullptr;
  size_t size_ = 0;
  std::unordered_map<std::string, Value> meta_;
  std::unordered_map<std::string, Tensor> tensors_;
};

}  // namespace gguf
}  // namespace esm_gfx950
