#pragma once

// A read-only GGUF v3 reader over a memory mapping: the subset of the format the forward pass
// needs (metadata scalars, strings, array lengths; tensor infos with bounds-checked data
// views). Follows the layout trickymind1324/axon-infer parses in src/core/gguf.cpp:484-662:
// magic "GGUF", version 3, tensor and metadata counts, metadata, tensor infos (at most four
// dimensions), a data section at the declared alignment (default 32).

#include "expected.h"
#include "kernels.h"

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <string_view>
#include <vector>

namespace axon {

struct GgufValue {
  enum class Kind { UInt, Int, Float, Bool, String, Array } kind = Kind::UInt;
  std::uint64_t u = 0;
  std::int64_t i = 0;
  double f = 0.0;
  std::string s;
  std::uint64_t array_size = 0;
  std::uint32_t array_type = 0;
};

struct GgufTensor {
  std::string name;
  DType type = DType::F32;
  std::uint32_t n_dims = 0;
  std::uint64_t ne[4] = {1, 1, 1, 1};  // ne[0] innermost, as stored
  const std::byte* data = nullptr;
  std::size_t nbytes = 0;
};

// Bytes of one row of n elements of type t, or 0 when n is not a whole number of blocks or the
// type is not one of the table's.
std::size_t row_bytes_of(DType t, std::uint64_t n);

class GgufFile {
public:
  static Expected<GgufFile> open(const std::string& path);
  GgufFile(GgufFile&& other) noexcept;
  GgufFile& operator=(GgufFile&& other) noexcept;
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;
  ~GgufFile();

  const GgufValue* meta(const std::string& key) const;
  std::uint64_t uint_or(const std::string& key, std::uint64_t fallback) const;
  double float_or(const std::string& key, double fallback) const;
  std::string string_or(const std::string& key, const std::string& fallback) const;
  const GgufTensor* tensor(const std::string& name) const;
  std::size_t file_size() const { return size_; }

private:
  GgufFile() = default;
  void release();
  void* map_ = nullptr;
  std::size_t size_ = 0;
  std::map<std::string, GgufValue> meta_;
  std::map<std::string, GgufTensor> tensors_;
};

}  // namespace axon
