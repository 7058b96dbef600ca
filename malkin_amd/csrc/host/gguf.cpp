#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <stdexcept>

namespace malkin_hip {

namespace {

struct Traits {
  int64_t block;
  size_t bytes;
};

Traits traits(uint32_t t) {
  switch (t) {
    case 0: return {1, 4};      // F32
    case 1: return {1, 2};      // F16
    case 30: return {1, 2};     // BF16
    case 2: return {32, 18};    // Q4_0
    case 3: return {32, 20};    // Q4_1
    case 6: return {32, 22};    // Q5_0
    case 7: return {32, 24};    // Q5_1
    case 8: return {32, 34};    // Q8_0
    case 9: return {32, 36};    // Q8_1
    case 10: return {256, 84};  // Q2_K
    case 11: return {256, 110}; // Q3_K
    case 12: return {256, 144}; // Q4_K
    case 13: return {256, 176}; // Q5_K
    case 14: return {256, 210}; // Q6_K
    case 15: return {256, 292}; // Q8_K
    case 39: return {32, 17};   // MXFP4
    default: throw std::runtime_error("unknown ggml type " + std::to_string(t));
  }
}

class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : p_(p), end_(p + n) {}
  template <typename T>
  T get() {
    need(sizeof(T));
    T v;
    std::memcpy(&v, p_, sizeof v);
    p_ += sizeof v;
    return v;
  }
  std::string str() {
    const auto n = get<uint64_t>();
    need(n);
    std::string s(reinterpret_cast<const char*>(p_), n);
    p_ += n;
    return s;
  }
  void skip(size_t n) {
    need(n);
    p_ += n;
  }
  const uint8_t* pos() const { return p_; }

 private:
  void need(size_t n) const {
    if (static_cast<size_t>(end_ - p_) < n) throw std::runtime_error("gguf: truncated header");
  }
  const uint8_t* p_;
  const uint8_t* end_;
};

// GGUF value types: u8 i8 u16 i16 u32 i32 f32 bool str arr u64 i64 f64.
size_t scalar_bytes(uint32_t t) {
  static const size_t b[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  if (t >= 13 || t == 8 || t == 9) return 0;
  return b[t];
}

int64_t read_int(Cursor& c, uint32_t t) {
  switch (t) {
    case 0: return c.get<uint8_t>();
    case 1: return c.get<int8_t>();
    case 2: return c.get<uint16_t>();
    case 3: return c.get<int16_t>();
    case 4: return c.get<uint32_t>();
    case 5: return c.get<int32_t>();
    case 10: return static_cast<int64_t>(c.get<uint64_t>());
    case 11: return c.get<int64_t>();
    default: throw std::runtime_error("gguf: not an int type");
  }
}

void skip_value(Cursor& c, uint32_t t) {
  if (t == 8) {
    c.skip(c.get<uint64_t>());
  } else if (t == 9) {
    const auto et = c.get<uint32_t>();
    const auto n = c.get<uint64_t>();
    for (uint64_t i = 0; i < n; ++i) skip_value(c, et);
  } else {
    const size_t b = scalar_bytes(t);
    if (!b) throw std::runtime_error("gguf: bad value type " + std::to_string(t));
    c.skip(b);
  }
}

}  // namespace

size_t ggml_row_size(uint32_t type, int64_t n) {
  const Traits t = traits(type);
  if (n % t.block) throw std::runtime_error("row not a multiple of the block size");
  return static_cast<size_t>(n / t.block) * t.bytes;
}

const char* ggml_type_name(uint32_t t) {
  switch (t) {
    case 0: return "F32";
    case 1: return "F16";
    case 8: return "Q8_0";
    case 12: return "Q4_K";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    case 30: return "BF16";
    default: return "other";
  }
}

int64_t GgufTensor::nelements() const {
  int64_t n = 1;
  for (auto d : ne) n *= d;
  return n;
}

GgufFile::GgufFile(const std::string& path) {
  fd_ = ::open(path.c_str(), O_RDONLY);
  if (fd_ < 0) throw std::runtime_error("cannot open " + path + ": " + std::strerror(errno));
  struct stat st{};
  if (fstat(fd_, &st) != 0) throw std::runtime_error("cannot stat " + path);
  size_ = static_cast<size_t>(st.st_size);
  void* m = mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd_, 0);
  if (m == MAP_FAILED) {
    ::close(fd_);
    throw std::runtime_error("mmap failed: " + std::string(std::strerror(errno)));
  }
  base_ = static_cast<uint8_t*>(m);
  try {
    Cursor c(base_, size_);
    if (c.get<uint32_t>() != 0x46554747) throw std::runtime_error(path + " is not a GGUF file");
    const auto version = c.get<uint32_t>();
    if (version < 3) throw std::runtime_error("GGUF v" + std::to_string(version) + " unsupported, need v3");
    const auto n_tensors = c.get<uint64_t>();
    const auto n_kv = c.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; ++i) {
      std::string key = c.str();
      const auto t = c.get<uint32_t>();
      if (t == 8) {
        kv_[key] = c.str();
      } else if (t == 6) {
        kv_[key] = static_cast<double>(c.get<float>());
      } else if (t == 12) {
        kv_[key] = c.get<double>();
      } else if (t == 7) {
        kv_[key] = c.get<uint8_t>() != 0;
      } else if (t == 9) {
        const auto et = c.get<uint32_t>();
        const auto n = c.get<uint64_t>();
        for (uint64_t j = 0; j < n; ++j) skip_value(c, et);
        kv_[key] = static_cast<size_t>(n);
      } else {
        kv_[key] = read_int(c, t);
      }
    }
    struct Info {
      GgufTensor t;
      uint64_t off;
    };
    std::vector<Info> infos;
    for (uint64_t i = 0; i < n_tensors; ++i) {
      Info in;
      in.t.name = c.str();
      const auto nd = c.get<uint32_t>();
      for (uint32_t d = 0; d < nd; ++d) in.t.ne.push_back(static_cast<int64_t>(c.get<uint64_t>()));
      in.t.type = c.get<uint32_t>();
      in.off = c.get<uint64_t>();
      infos.push_back(std::move(in));
    }
    const size_t align = static_cast<size_t>(get_int("general.alignment").value_or(32));
    const size_t start = (static_cast<size_t>(c.pos() - base_) + align - 1) / align * align;
    for (auto& in : infos) {
      auto& t = in.t;
      t.nbytes = ggml_row_size(t.type, t.ne[0]) * static_cast<size_t>(t.rows());
      if (start + in.off + t.nbytes > size_) throw std::runtime_error("gguf: tensor " + t.name + " out of bounds");
      t.data = base_ + start + in.off;
      tensors_[t.name] = std::move(t);
    }
  } catch (...) {
    munmap(base_, size_);
    ::close(fd_);
    throw;
  }
}

GgufFile::~GgufFile() {
  if (base_) munmap(base_, size_);
  if (fd_ >= 0) ::close(fd_);
}

std::optional<int64_t> GgufFile::get_int(const std::string& key) const {
  auto it = kv_.find(key);
  if (it == kv_.end()) return std::nullopt;
  if (auto* i = std::get_if<int64_t>(&it->second)) return *i;
  if (auto* b = std::get_if<bool>(&it->second)) return *b ? 1 : 0;
  return std::nullopt;
}

std::optional<double> GgufFile::get_float(const std::string& key) const {
  auto it = kv_.find(key);
  if (it == kv_.end()) return std::nullopt;
  if (auto* d = std::get_if<double>(&it->second)) return *d;
  if (auto* i = std::get_if<int64_t>(&it->second)) return static_cast<double>(*i);
  return std::nullopt;
}

std::optional<std::string> GgufFile::get_str(const std::string& key) const {
  auto it = kv_.find(key);
  if (it == kv_.end()) return std::nullopt;
  if (auto* s = std::get_if<std::string>(&it->second)) return *s;
  return std::nullopt;
}

size_t GgufFile::str_array_size(const std::string& key) const {
  auto it = kv_.find(key);
  if (it == kv_.end()) return 0;
  if (auto* n = std::get_if<size_t>(&it->second)) return *n;
  return 0;
}

const GgufTensor* GgufFile::tensor(const std::string& name) const {
  auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

}  // namespace malkin_hip
