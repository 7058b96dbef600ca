// Memory-mapped GGUF v3 file: the metadata table and the tensor directory, with every offset checked against the
// mapping. Serves the role of the reference's GgufFile (gguf.h:44-69) for the device model: same file format, same
// key and tensor lookups; the parser is written from the GGUF v3 format description.
//
// Format (little endian): magic "GGUF" (u32 0x46554747), version u32 (3), tensor count u64, metadata count u64;
// metadata entries {string key, u32 value type, value}; tensor entries {string name, u32 n_dims, u64 ne[n_dims],
// u32 ggml type, u64 offset}; tensor data starts at the next multiple of general.alignment (default 32) after the
// directory, each tensor at data start + offset. Strings are {u64 length, bytes}; arrays {u32 element type, u64
// count, elements}.
#pragma once

#include <cstdint>
#include <map>
#include <optional>
#include <string>
#include <vector>

namespace malkin_hip {

// Block geometry of a ggml tensor type: `block` values in `bytes` bytes.
struct GgmlBlock {
  uint32_t type;
  int block;
  int bytes;
  const char* name;
};
// nullptr for types this file reader does not know.
const GgmlBlock* ggml_block(uint32_t type);
// Bytes of n values of `type`; throws for unknown types and for n not a whole number of blocks.
size_t ggml_row_size(uint32_t type, int64_t n);
const char* ggml_type_name(uint32_t type);

struct GgufTensor {
  std::string name;
  uint32_t type = 0;
  std::vector<int64_t> ne;  // ne[0] is the row length
  const uint8_t* data = nullptr;
  size_t nbytes = 0;
  int64_t nelements() const;
  int64_t rows() const { return ne.empty() || ne[0] == 0 ? 0 : nelements() / ne[0]; }
};

class GgufFile {
 public:
  explicit GgufFile(const std::string& path);
  ~GgufFile();
  GgufFile(const GgufFile&) = delete;
  GgufFile& operator=(const GgufFile&) = delete;

  // Typed metadata lookups; nullopt when the key is absent or holds another kind of value. Integers of every width
  // and bools read as int; f32 / f64 (and integers) as float.
  std::optional<int64_t> get_int(const std::string& key) const;
  std::optional<double> get_float(const std::string& key) const;
  std::optional<std::string> get_str(const std::string& key) const;
  // Element count of an array value (the tokenizer's vocabulary, tokenizer.ggml.tokens); 0 when absent.
  size_t str_array_size(const std::string& key) const;
  // The elements of an array of strings / of integers (tokenizer.ggml.tokens, tokenizer.ggml.token_type); empty
  // when the key is absent or its elements are of another kind.
  std::vector<std::string> str_array(const std::string& key) const;
  std::vector<int64_t> int_array(const std::string& key) const;

  const GgufTensor* tensor(const std::string& name) const;
  const std::map<std::string, GgufTensor>& tensors() const { return tensors_; }
  size_t size() const { return size_; }

 private:
  // One decoded metadata value. Arrays keep their element count, element type and the file offset of their first
  // element (decoded on request).
  struct Meta {
    enum Kind { kInt, kFloat, kBool, kString, kArray } kind = kInt;
    int64_t i = 0;
    double f = 0;
    std::string s;
    uint32_t elem = 0;
    size_t at = 0;
  };
  void parse(const std::string& path);

  int fd_ = -1;
  void* map_ = nullptr;
  size_t size_ = 0;
  std::map<std::string, Meta> meta_;
  std::map<std::string, GgufTensor> tensors_;
};

}  // namespace malkin_hip
