#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <limits>
#include <stdexcept>

namespace malkin_hip {

namespace {

// ggml's block geometry per type id (ggml.h type enum; the GGUF tensor type field).
constexpr GgmlBlock kBlocks[] = {
    {0, 1, 4, "F32"},       {1, 1, 2, "F16"},       {2, 32, 18, "Q4_0"},    {3, 32, 20, "Q4_1"},
    {6, 32, 22, "Q5_0"},    {7, 32, 24, "Q5_1"},    {8, 32, 34, "Q8_0"},    {9, 32, 36, "Q8_1"},
    {10, 256, 84, "Q2_K"},  {11, 256, 110, "Q3_K"}, {12, 256, 144, "Q4_K"}, {13, 256, 176, "Q5_K"},
    {14, 256, 210, "Q6_K"}, {15, 256, 292, "Q8_K"}, {24, 1, 1, "I8"},       {25, 1, 2, "I16"},
    {26, 1, 4, "I32"},      {27, 1, 8, "I64"},      {28, 1, 8, "F64"},      {30, 1, 2, "BF16"},
    {39, 32, 17, "MXFP4"},
};

constexpr uint32_t kMagic = 0x46554747;  // "GGUF" read as a little-endian u32
constexpr int kMaxDims = 4;              // GGML_MAX_DIMS
constexpr int kMaxArrayNesting = 8;

// GGUF metadata value types.
enum : uint32_t { kU8, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64, kNumTypes };

// Byte width of a fixed-size value type; 0 for strings, arrays and unknown types.
size_t fixed_width(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

// Bounds-checked forward reader over the mapped header. Every check compares a length with the bytes left, so no
// offset arithmetic can wrap.
class Reader {
 public:
  Reader(const uint8_t* base, size_t size, const std::string& path, size_t at = 0)
      : base_(base), size_(size), at_(at), path_(path) {}

  const uint8_t* take(size_t n, const char* what) {
    if (n > size_ - at_) fail(std::string(what) + " runs past the end of the file");
    const uint8_t* p = base_ + at_;
    at_ += n;
    return p;
  }
  template <typename T>
  T get(const char* what) {
    T v;
    std::memcpy(&v, take(sizeof v, what), sizeof v);
    return v;
  }
  std::string text(const char* what) {
    const uint64_t n = get<uint64_t>(what);
    const uint8_t* p = take(n, what);
    return std::string(reinterpret_cast<const char*>(p), n);
  }
  size_t offset() const { return at_; }
  [[noreturn]] void fail(const std::string& why) const {
    throw std::runtime_error("gguf " + path_ + ": " + why + " (at byte " + std::to_string(at_) + ")");
  }

 private:
  const uint8_t* base_;
  size_t size_;
  size_t at_;
  const std::string& path_;
};

int64_t read_integer(Reader& r, uint32_t t) {
  switch (t) {
    case kU8: return r.get<uint8_t>("metadata value");
    case kI8: return r.get<int8_t>("metadata value");
    case kU16: return r.get<uint16_t>("metadata value");
    case kI16: return r.get<int16_t>("metadata value");
    case kU32: return r.get<uint32_t>("metadata value");
    case kI32: return r.get<int32_t>("metadata value");
    case kU64: {
      const uint64_t v = r.get<uint64_t>("metadata value");
      if (v > static_cast<uint64_t>(std::numeric_limits<int64_t>::max())) r.fail("u64 metadata value out of range");
      return static_cast<int64_t>(v);
    }
    case kI64: return r.get<int64_t>("metadata value");
    default: r.fail("metadata value type " + std::to_string(t) + " is not an integer");
  }
}

// Steps over an array's elements (their contents are not kept).
void skip_array(Reader& r, uint32_t elem, uint64_t count, int depth) {
  if (depth > kMaxArrayNesting) r.fail("metadata arrays nested too deeply");
  if (const size_t w = fixed_width(elem)) {
    if (count > std::numeric_limits<size_t>::max() / w) r.fail("metadata array too large");
    r.take(static_cast<size_t>(count) * w, "metadata array");
    return;
  }
  for (uint64_t i = 0; i < count; ++i) {
    if (elem == kStr) {
      r.text("metadata array string");
    } else if (elem == kArr) {
      const uint32_t e = r.get<uint32_t>("metadata array type");
      skip_array(r, e, r.get<uint64_t>("metadata array count"), depth + 1);
    } else {
      r.fail("metadata array of unknown type " + std::to_string(elem));
    }
  }
}

}  // namespace

const GgmlBlock* ggml_block(uint32_t type) {
  for (const GgmlBlock& b : kBlocks)
    if (b.type == type) return &b;
  return nullptr;
}

size_t ggml_row_size(uint32_t type, int64_t n) {
  const GgmlBlock* b = ggml_block(type);
  if (!b) throw std::runtime_error("ggml type " + std::to_string(type) + " is not supported");
  if (n < 0 || n % b->block)
    throw std::runtime_error(std::string(b->name) + ": a row of " + std::to_string(n) +
                             " values is not a whole number of blocks of " + std::to_string(b->block));
  return static_cast<size_t>(n / b->block) * static_cast<size_t>(b->bytes);
}

const char* ggml_type_name(uint32_t type) {
  const GgmlBlock* b = ggml_block(type);
  return b ? b->name : "unknown";
}

int64_t GgufTensor::nelements() const {
  int64_t n = 1;
  for (int64_t d : ne) n *= d;
  return n;
}

GgufFile::GgufFile(const std::string& path) {
  try {
    parse(path);
  } catch (...) {
    if (map_) munmap(map_, size_);
    if (fd_ >= 0) ::close(fd_);
    map_ = nullptr;
    fd_ = -1;
    throw;
  }
}

GgufFile::~GgufFile() {
  if (map_) munmap(map_, size_);
  if (fd_ >= 0) ::close(fd_);
}

void GgufFile::parse(const std::string& path) {
  fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd_ < 0) throw std::runtime_error("gguf " + path + ": open failed: " + std::strerror(errno));
  struct stat st {};
  if (fstat(fd_, &st) != 0) throw std::runtime_error("gguf " + path + ": stat failed: " + std::strerror(errno));
  size_ = static_cast<size_t>(st.st_size);
  if (size_ < 24) throw std::runtime_error("gguf " + path + ": file too short for a GGUF header");
  void* m = mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd_, 0);
  if (m == MAP_FAILED) throw std::runtime_error("gguf " + path + ": mmap failed: " + std::strerror(errno));
  map_ = m;
  const auto* base = static_cast<const uint8_t*>(map_);

  Reader r(base, size_, path);
  if (r.get<uint32_t>("magic") != kMagic) r.fail("not a GGUF file (bad magic)");
  const uint32_t version = r.get<uint32_t>("version");
  if (version < 3) r.fail("GGUF version " + std::to_string(version) + " is not supported (version 3 is)");
  const uint64_t n_tensors = r.get<uint64_t>("tensor count");
  const uint64_t n_meta = r.get<uint64_t>("metadata count");

  for (uint64_t i = 0; i < n_meta; ++i) {
    std::string key = r.text("metadata key");
    const uint32_t t = r.get<uint32_t>("metadata type");
    Meta v;
    if (t == kStr) {
      v.kind = Meta::kString;
      v.s = r.text("metadata string");
    } else if (t == kArr) {
      const uint32_t elem = r.get<uint32_t>("metadata array type");
      const uint64_t count = r.get<uint64_t>("metadata array count");
      v.elem = elem;
      v.at = r.offset();
      skip_array(r, elem, count, 0);
      v.kind = Meta::kArray;
      v.i = static_cast<int64_t>(count > static_cast<uint64_t>(std::numeric_limits<int64_t>::max())
                                     ? std::numeric_limits<int64_t>::max()
                                     : count);
    } else if (t == kF32) {
      v.kind = Meta::kFloat;
      v.f = r.get<float>("metadata value");
    } else if (t == kF64) {
      v.kind = Meta::kFloat;
      v.f = r.get<double>("metadata value");
    } else if (t == kBool) {
      v.kind = Meta::kBool;
      v.i = r.get<uint8_t>("metadata value") != 0;
    } else if (t < kNumTypes) {
      v.kind = Meta::kInt;
      v.i = read_integer(r, t);
    } else {
      r.fail("metadata type " + std::to_string(t) + " is unknown");
    }
    meta_[std::move(key)] = std::move(v);
  }

  // Tensor directory: the entries are kept in file order until the data section's start is known.
  struct Entry {
    GgufTensor t;
    uint64_t offset;
  };
  std::vector<Entry> dir;
  for (uint64_t i = 0; i < n_tensors; ++i) {
    Entry e;
    e.t.name = r.text("tensor name");
    const uint32_t nd = r.get<uint32_t>("tensor rank");
    if (nd < 1 || nd > kMaxDims) r.fail("tensor " + e.t.name + " has rank " + std::to_string(nd));
    int64_t count = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      const uint64_t n = r.get<uint64_t>("tensor shape");
      if (n > static_cast<uint64_t>(std::numeric_limits<int64_t>::max() / (count ? count : 1)))
        r.fail("tensor " + e.t.name + " has too many elements");
      count *= static_cast<int64_t>(n);
      e.t.ne.push_back(static_cast<int64_t>(n));
    }
    e.t.type = r.get<uint32_t>("tensor type");
    e.offset = r.get<uint64_t>("tensor offset");
    if (!ggml_block(e.t.type))
      r.fail("tensor " + e.t.name + " has unknown ggml type " + std::to_string(e.t.type));
    dir.push_back(std::move(e));
  }

  uint64_t align = 32;
  if (const auto a = get_int("general.alignment")) {
    if (*a <= 0 || *a > (1 << 20)) r.fail("general.alignment " + std::to_string(*a) + " is not usable");
    align = static_cast<uint64_t>(*a);
  }
  const uint64_t data = (r.offset() + align - 1) / align * align;
  if (data > size_) r.fail("tensor data section starts past the end of the file");
  const uint64_t avail = size_ - data;
  for (Entry& e : dir) {
    GgufTensor& t = e.t;
    const size_t row = ggml_row_size(t.type, t.ne[0]);
    const int64_t rows = t.rows();
    if (rows > 0 && row > std::numeric_limits<size_t>::max() / static_cast<size_t>(rows))
      r.fail("tensor " + t.name + " is too large");
    t.nbytes = row * static_cast<size_t>(rows);
    if (e.offset > avail || t.nbytes > avail - e.offset)
      throw std::runtime_error("gguf " + path + ": tensor " + t.name + " lies outside the file");
    t.data = base + data + e.offset;
    if (!tensors_.emplace(t.name, t).second)
      throw std::runtime_error("gguf " + path + ": tensor " + t.name + " appears twice");
  }
}

std::optional<int64_t> GgufFile::get_int(const std::string& key) const {
  const auto it = meta_.find(key);
  if (it == meta_.end()) return std::nullopt;
  const Meta& v = it->second;
  if (v.kind == Meta::kInt || v.kind == Meta::kBool) return v.i;
  return std::nullopt;
}

std::optional<double> GgufFile::get_float(const std::string& key) const {
  const auto it = meta_.find(key);
  if (it == meta_.end()) return std::nullopt;
  const Meta& v = it->second;
  if (v.kind == Meta::kFloat) return v.f;
  if (v.kind == Meta::kInt) return static_cast<double>(v.i);
  return std::nullopt;
}

std::optional<std::string> GgufFile::get_str(const std::string& key) const {
  const auto it = meta_.find(key);
  if (it == meta_.end() || it->second.kind != Meta::kString) return std::nullopt;
  return it->second.s;
}

size_t GgufFile::str_array_size(const std::string& key) const {
  const auto it = meta_.find(key);
  if (it == meta_.end() || it->second.kind != Meta::kArray) return 0;
  return static_cast<size_t>(it->second.i);
}

// The array was walked (every element in bounds) when the file was opened, so these re-reads cannot fail.
std::vector<std::string> GgufFile::str_array(const std::string& key) const {
  std::vector<std::string> out;
  const auto it = meta_.find(key);
  if (it == meta_.end() || it->second.kind != Meta::kArray || it->second.elem != kStr) return out;
  const std::string path = "(array " + key + ")";
  Reader r(static_cast<const uint8_t*>(map_), size_, path, it->second.at);
  out.reserve(static_cast<size_t>(it->second.i));
  for (int64_t k = 0; k < it->second.i; ++k) out.push_back(r.text("metadata array string"));
  return out;
}

std::vector<int64_t> GgufFile::int_array(const std::string& key) const {
  std::vector<int64_t> out;
  const auto it = meta_.find(key);
  if (it == meta_.end() || it->second.kind != Meta::kArray) return out;
  const uint32_t e = it->second.elem;
  if (e == kF32 || e == kF64 || !fixed_width(e)) return out;
  const std::string path = "(array " + key + ")";
  Reader r(static_cast<const uint8_t*>(map_), size_, path, it->second.at);
  out.reserve(static_cast<size_t>(it->second.i));
  for (int64_t k = 0; k < it->second.i; ++k) out.push_back(e == kBool ? r.get<uint8_t>("metadata array") : read_integer(r, e));
  return out;
}

const GgufTensor* GgufFile::tensor(const std::string& name) const {
  const auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

}  // namespace malkin_hip
