#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <utility>

namespace axon {

std::size_t row_bytes_of(DType t, std::uint64_t n) {
  switch (t) {
  case DType::F32: return 4 * n;
  case DType::F16:
  case DType::BF16: return 2 * n;
  case DType::Q8_0: return n % 32 ? 0 : n / 32 * sizeof(BlockQ8_0);
  case DType::Q4_0: return n % 32 ? 0 : n / 32 * sizeof(BlockQ4_0);
  case DType::Q4_1: return n % 32 ? 0 : n / 32 * sizeof(BlockQ4_1);
  case DType::Q6_K: return n % 256 ? 0 : n / 256 * sizeof(BlockQ6_K);
  }
  return 0;
}

namespace {

// A cursor over the mapped bytes; every read is bounds-checked.
struct Reader {
  const std::byte* p;
  std::size_t size;
  std::size_t off = 0;
  bool ok = true;

  template <class T>
  T get() {
    T v{};
    if (!ok || off + sizeof(T) > size) {
      ok = false;
      return v;
    }
    std::memcpy(&v, p + off, sizeof(T));
    off += sizeof(T);
    return v;
  }
  std::string str() {
    const auto n = get<std::uint64_t>();
    if (!ok || n > size - off) {
      ok = false;
      return {};
    }
    std::string s(reinterpret_cast<const char*>(p + off), n);
    off += n;
    return s;
  }
  bool skip(std::uint64_t n) {
    if (!ok || n > size - off) return ok = false;
    off += n;
    return true;
  }
};

std::size_t scalar_size(std::uint32_t t) {
  switch (t) {
  case 0: case 1: case 7: return 1;
  case 2: case 3: return 2;
  case 4: case 5: case 6: return 4;
  case 10: case 11: case 12: return 8;
  default: return 0;
  }
}

bool read_scalar(Reader& r, std::uint32_t t, GgufValue& v) {
  switch (t) {
  case 0: v.kind = GgufValue::Kind::UInt; v.u = r.get<std::uint8_t>(); break;
  case 1: v.kind = GgufValue::Kind::Int; v.i = r.get<std::int8_t>(); break;
  case 2: v.kind = GgufValue::Kind::UInt; v.u = r.get<std::uint16_t>(); break;
  case 3: v.kind = GgufValue::Kind::Int; v.i = r.get<std::int16_t>(); break;
  case 4: v.kind = GgufValue::Kind::UInt; v.u = r.get<std::uint32_t>(); break;
  case 5: v.kind = GgufValue::Kind::Int; v.i = r.get<std::int32_t>(); break;
  case 6: v.kind = GgufValue::Kind::Float; v.f = r.get<float>(); break;
  case 7: v.kind = GgufValue::Kind::Bool; v.u = r.get<std::uint8_t>(); break;
  case 8: v.kind = GgufValue::Kind::String; v.s = r.str(); break;
  case 10: v.kind = GgufValue::Kind::UInt; v.u = r.get<std::uint64_t>(); break;
  case 11: v.kind = GgufValue::Kind::Int; v.i = r.get<std::int64_t>(); break;
  case 12: v.kind = GgufValue::Kind::Float; v.f = r.get<double>(); break;
  default: return false;
  }
  if (v.kind == GgufValue::Kind::Int && v.i >= 0) v.u = static_cast<std::uint64_t>(v.i);
  return r.ok;
}

// Skips an array's elements (nested arrays included), keeping only its length.
bool skip_array(Reader& r, std::uint32_t et, std::uint64_t n, int depth) {
  if (depth > 4) return false;
  if (et == 8) {
    for (std::uint64_t k = 0; k < n; ++k) {
      const auto len = r.get<std::uint64_t>();
      if (!r.skip(len)) return false;
    }
    return r.ok;
  }
  if (et == 9) {
    for (std::uint64_t k = 0; k < n; ++k) {
      const auto t = r.get<std::uint32_t>();
      const auto m = r.get<std::uint64_t>();
      if (!r.ok || !skip_array(r, t, m, depth + 1)) return false;
    }
    return true;
  }
  const std::size_t s = scalar_size(et);
  if (s == 0 || n > (r.size - r.off) / s) return false;
  return r.skip(n * s);
}

Error corrupt(const std::string& path, const std::string& what) {
  return make_error(ErrorCode::Corrupt, path + ": " + what);
}

}  // namespace

Expected<GgufFile> GgufFile::open(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return make_error(ErrorCode::Io, path + ": cannot open: " + std::strerror(errno));
  struct stat st {};
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return make_error(ErrorCode::Io, path + ": cannot stat");
  }
  const auto size = static_cast<std::size_t>(st.st_size);
  if (size < 24) {
    ::close(fd);
    return corrupt(path, "too short for a GGUF header");
  }
  void* map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) return make_error(ErrorCode::Io, path + ": mmap failed");
  madvise(map, size, MADV_SEQUENTIAL);

  GgufFile f;
  f.map_ = map;
  f.size_ = size;
  Reader r{static_cast<const std::byte*>(map), size};
  if (r.get<std::uint32_t>() != 0x46554747u) return corrupt(path, "not a GGUF file (bad magic)");
  const auto version = r.get<std::uint32_t>();
  if (version != 3) return corrupt(path, "GGUF version " + std::to_string(version) + ", expected 3");
  const auto n_tensors = r.get<std::uint64_t>();
  const auto n_kv = r.get<std::uint64_t>();
  if (n_tensors > size || n_kv > size) return corrupt(path, "implausible tensor or metadata count");
  for (std::uint64_t k = 0; k < n_kv; ++k) {
    std::string key = r.str();
    const auto t = r.get<std::uint32_t>();
    GgufValue v;
    if (t == 9) {
      v.kind = GgufValue::Kind::Array;
      v.array_type = r.get<std::uint32_t>();
      v.array_size = r.get<std::uint64_t>();
      if (!r.ok || !skip_array(r, v.array_type, v.array_size, 0)) return corrupt(path, "bad array " + key);
    } else if (!read_scalar(r, t, v)) {
      return corrupt(path, "bad metadata value for " + key);
    }
    f.meta_[std::move(key)] = std::move(v);
  }
  std::vector<std::pair<GgufTensor, std::uint64_t>> infos;
  for (std::uint64_t k = 0; k < n_tensors; ++k) {
    GgufTensor t;
    t.name = r.str();
    t.n_dims = r.get<std::uint32_t>();
    if (!r.ok || t.n_dims == 0 || t.n_dims > 4) return corrupt(path, "tensor " + t.name + ": bad dimension count");
    for (std::uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = r.get<std::uint64_t>();
    if (!r.ok) return corrupt(path, "truncated tensor info");
    // Every extent non-zero and the element count representable, so that the byte size
    // computed below cannot wrap around to something that passes the bounds check.
    std::uint64_t elements = 1;
    for (std::uint32_t d = 0; d < t.n_dims; ++d) {
      if (t.ne[d] == 0) return corrupt(path, "tensor " + t.name + ": an extent of zero");
      if (t.ne[d] > UINT64_MAX / elements) return corrupt(path, "tensor " + t.name + ": element count overflows 64 bits");
      elements *= t.ne[d];
    }
    t.type = static_cast<DType>(r.get<std::uint32_t>());
    const auto offset = r.get<std::uint64_t>();
    if (!r.ok) return corrupt(path, "truncated tensor info");
    infos.emplace_back(std::move(t), offset);
  }
  const std::uint64_t align = f.uint_or("general.alignment", 32);
  if (align == 0 || (align & (align - 1)) != 0) return corrupt(path, "general.alignment is not a power of two");
  const std::size_t data = (r.off + align - 1) / align * align;
  if (data > size) return corrupt(path, "data section past the end of the file");
  for (auto& [t, offset] : infos) {
    if (t.ne[0] > (SIZE_MAX >> 3)) return corrupt(path, "tensor " + t.name + ": row length overflows");
    const std::size_t row = row_bytes_of(t.type, t.ne[0]);
    if (row == 0) {
      // Types outside the table's set are kept as size 0; binding rejects them by name.
      t.nbytes = 0;
    } else {
      const std::uint64_t rows = (t.n_dims > 1 ? t.ne[1] : 1) * (t.n_dims > 2 ? t.ne[2] : 1) * (t.n_dims > 3 ? t.ne[3] : 1);
      if (rows > SIZE_MAX / row) return corrupt(path, "tensor " + t.name + ": byte size overflows");
      t.nbytes = row * rows;
    }
    if (offset > size - data || t.nbytes > size - data - offset) return corrupt(path, "tensor " + t.name + " out of bounds");
    t.data = static_cast<const std::byte*>(map) + data + offset;
    std::string name = t.name;
    f.tensors_[std::move(name)] = std::move(t);
  }
  return f;
}

GgufFile::GgufFile(GgufFile&& o) noexcept
    : map_(std::exchange(o.map_, nullptr)), size_(std::exchange(o.size_, 0)), meta_(std::move(o.meta_)),
      tensors_(std::move(o.tensors_)) {}

GgufFile& GgufFile::operator=(GgufFile&& o) noexcept {
  if (this != &o) {
    release();
    map_ = std::exchange(o.map_, nullptr);
    size_ = std::exchange(o.size_, 0);
    meta_ = std::move(o.meta_);
    tensors_ = std::move(o.tensors_);
  }
  return *this;
}

GgufFile::~GgufFile() { release(); }

void GgufFile::release() {
  if (map_ != nullptr) munmap(map_, size_);
  map_ = nullptr;
}

const GgufValue* GgufFile::meta(const std::string& key) const {
  const auto it = meta_.find(key);
  return it == meta_.end() ? nullptr : &it->second;
}

std::uint64_t GgufFile::uint_or(const std::string& key, std::uint64_t fallback) const {
  const GgufValue* v = meta(key);
  if (v == nullptr) return fallback;
  if (v->kind == GgufValue::Kind::UInt || (v->kind == GgufValue::Kind::Int && v->i >= 0)) return v->u;
  return fallback;
}

double GgufFile::float_or(const std::string& key, double fallback) const {
  const GgufValue* v = meta(key);
  return v != nullptr && v->kind == GgufValue::Kind::Float ? v->f : fallback;
}

std::string GgufFile::string_or(const std::string& key, const std::string& fallback) const {
  const GgufValue* v = meta(key);
  return v != nullptr && v->kind == GgufValue::Kind::String ? v->s : fallback;
}

const GgufTensor* GgufFile::tensor(const std::string& name) const {
  const auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

}  // namespace axon
