// GGUF v3 reader (memory-mapped): metadata and tensor table. Plays the role of the reference's GgufFile
// (gguf.h:44-69): same file format, same lookups, our own implementation.
#pragma once

#include <cstdint>
#include <map>
#include <optional>
#include <string>
#include <variant>
#include <vector>

namespace malkin_hip {

struct GgufTensor {
  std::string name;
  uint32_t type = 0;        // ggml type id
  std::vector<int64_t> ne;  // ne[0] innermost
  const uint8_t* data = nullptr;
  size_t nbytes = 0;
  int64_t nelements() const;
  int64_t rows() const { return ne.empty() ? 0 : nelements() / ne[0]; }
};

// ggml block traits (gguf.cpp:60-95): bytes of n elements of type t; throws for unknown types or partial blocks.
size_t ggml_row_size(uint32_t type, int64_t n);
const char* ggml_type_name(uint32_t type);

class GgufFile {
 public:
  explicit GgufFile(const std::string& path);
  ~GgufFile();
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;

  std::optional<int64_t> get_int(const std::string& key) const;
  std::optional<double> get_float(const std::string& key) const;
  std::optional<std::string> get_str(const std::string& key) const;
  size_t str_array_size(const std::string& key) const;  // 0 when absent
  const GgufTensor* tensor(const std::string& name) const;
  const std::map<std::string, GgufTensor>& tensors() const { return tensors_; }
  size_t size() const { return size_; }

 private:
  using Value = std::variant<int64_t, double, bool, std::string, size_t /* array length */>;
  int fd_ = -1;
  uint8_t* base_ = nullptr;
  size_t size_ = 0;
  std::map<std::string, Value> kv_;
  std::map<std::string, GgufTensor> tensors_;
};

}  // namespace malkin_hip
