// The .efq model container (include/ef/qfile.h:1-21): host-side reader with the reference's full
// validation (src/qfile.cpp:125-223), the model-config checks (src/model_config.cpp:72-131) and the
// quantization-policy re-derivation (src/qfile.cpp:48-86).  Pure host C++; the device upload of a
// parsed file lives in model.hip.
//
// Layout: "EFQ1", u32 LE version 1, u64 LE header length N, N bytes of space-padded JSON, then every
// tensor at an absolute 64-byte-aligned offset, rows contiguous, in forward order.
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace efh::efq {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// A strict JSON value (RFC 8259: no comments, no trailing commas, no duplicate keys).  Numbers
// keep their text; a number written without fraction or exponent that fits int64 is an integer.
struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object };
  Kind kind = Null;
  bool boolean = false;
  bool is_int = false;
  int64_t integer = 0;
  double number = 0.0;
  std::string text;                // string value, or the number as written
  std::vector<Json> items;         // array elements, or object values (in key order)
  std::vector<std::string> keys;   // object keys
  const Json* find(const std::string& key) const;  // objects only
  const Json& at(const std::string& key) const;    // throws when missing
  const std::string& str() const;
  const std::vector<Json>& list() const;           // array elements
  int64_t i64() const;
  uint64_t u64() const;
  double dbl() const;
  bool flag() const;
};
Json parse_json(const char* text, size_t n);

struct Tensor {
  std::string name, rule;
  int qtype = 0;                  // EF_QTYPE_*
  std::vector<uint64_t> shape;    // [rows, cols] or [n]
  uint64_t offset = 0, bytes = 0;
  double rel_rmse = 0.0, max_abs_err = 0.0;
  uint64_t rows() const { return shape.size() == 2 ? shape[0] : 1; }
  uint64_t cols() const { return shape.empty() ? 0 : shape.back(); }
};

// ModelConfig (include/ef/model_config.h:14-38): the Llama fields the decode path needs.
struct Config {
  int64_t hidden_size = 0, intermediate_size = 0, num_hidden_layers = 0, num_attention_heads = 0;
  int64_t num_key_value_heads = 0, head_dim = 0, vocab_size = 0, max_position_embeddings = 0;
  int64_t bos_token_id = -1, eos_token_id = -1;
  double rms_norm_eps = 0.0, rope_theta = 10000.0;
  bool tie_word_embeddings = false;
  int64_t kv_dim() const { return num_key_value_heads * head_dim; }
};
Config parse_config(const Json& root);

struct Override {
  std::string pattern;
  int qtype = 0;
};
struct Policy {
  int layers = 4, lm_head = 3, embed = 2;  // Q4_0, Q8_0, BF16
  std::vector<Override> overrides;
  std::string name;
};

struct Layout {
  uint64_t header_len = 0;
  Config cfg;
  Policy policy;
  std::vector<Tensor> tensors;
};

// parse_efq (src/qfile.cpp:125-223): throws Error with the reference's messages.
Layout parse(const uint8_t* file, uint64_t size);

bool glob_match(const std::string& pattern, const std::string& text);
struct Choice {
  int qtype;
  const char* rule;
};
Choice policy_choice(const Policy& p, const std::string& name, uint64_t cols);
struct Expected {
  std::string name;
  std::vector<uint64_t> shape;
};
std::vector<Expected> expected_tensors(const Config& c);  // src/model_config.cpp:145-167
const char* qtype_name(int qtype);
uint64_t row_bytes(int qtype, uint64_t cols);  // throws for a block type with cols % 32 != 0

// A validated file: memory-mapped from a path (QuantFile::open, src/qfile.cpp:225-243) or over a
// caller's buffer (which must outlive it).
class File {
 public:
  static std::unique_ptr<File> open(const std::string& path);
  static std::unique_ptr<File> over(const uint8_t* bytes, uint64_t size);
  ~File();
  File(const File&) = delete;
  File& operator=(const File&) = delete;

  const Layout& layout() const { return L_; }
  const Tensor* find(const std::string& name) const;
  const Tensor& at(const std::string& name) const;
  const uint8_t* data(const Tensor& t) const { return base_ + t.offset; }
  const uint8_t* base() const { return base_; }
  uint64_t size() const { return size_; }
  uint64_t bytes_per_token() const { return bytes_per_token_; }
  const std::string& path() const { return path_; }

 private:
  File() = default;
  void index();
  Layout L_;
  std::unordered_map<std::string, size_t> index_;
  uint64_t bytes_per_token_ = 0;
  const uint8_t* base_ = nullptr;
  uint64_t size_ = 0;
  void* map_ = nullptr;
  int fd_ = -1;
  std::string path_;
};

}  // namespace efh::efq
