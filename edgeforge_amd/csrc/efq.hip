// .efq reader (host code): strict JSON, the model-config checks, the tensor-table checks and the
// quantization-policy re-derivation of the reference reader (src/qfile.cpp:125-223,
// src/model_config.cpp:72-131).  Error texts carry the reference's key phrases ("bad magic",
// "past the end", "64-byte aligned", "header says", "policy gives", ...) so callers and tests
// that match on them behave the same.
#include "efq.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <charconv>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>

#include "common.h"

namespace efh::efq {

// ---------------------------------------------------------------- JSON

namespace {
const char* kind_name(Json::Kind k) {
  switch (k) {
    case Json::Null: return "null";
    case Json::Bool: return "bool";
    case Json::Number: return "number";
    case Json::String: return "string";
    case Json::Array: return "array";
    default: return "object";
  }
}
void expect(const Json& v, Json::Kind k) {
  if (v.kind != k) throw Error(std::string("JSON: expected ") + kind_name(k) + ", got " + kind_name(v.kind));
}
}  // namespace

const Json* Json::find(const std::string& key) const {
  expect(*this, Object);
  for (size_t i = 0; i < keys.size(); ++i)
    if (keys[i] == key) return &items[i];
  return nullptr;
}

const Json& Json::at(const std::string& key) const {
  const Json* v = find(key);
  if (v == nullptr) throw Error("JSON: missing key \"" + key + "\"");
  return *v;
}

const std::string& Json::str() const {
  expect(*this, String);
  return text;
}

const std::vector<Json>& Json::list() const {
  expect(*this, Array);
  return items;
}

int64_t Json::i64() const {
  expect(*this, Number);
  if (!is_int) throw Error("JSON: expected an integer, got " + text);
  return integer;
}

uint64_t Json::u64() const {
  const int64_t v = i64();
  if (v < 0) throw Error("JSON: expected a non-negative integer, got " + text);
  return static_cast<uint64_t>(v);
}

double Json::dbl() const {
  expect(*this, Number);
  return number;
}

bool Json::flag() const {
  expect(*this, Bool);
  return boolean;
}

namespace {

class JsonReader {
 public:
  JsonReader(const char* s, size_t n) : s_(s), n_(n) {}

  Json document() {
    skip_ws();
    Json v = value(0);
    skip_ws();
    if (i_ != n_) fail("unexpected characters after the top-level value");
    return v;
  }

 private:
  const char* s_;
  size_t n_;
  size_t i_ = 0;

  [[noreturn]] void fail(const std::string& what) const {
    throw Error("JSON: " + what + " at byte " + std::to_string(i_));
  }
  bool eof() const { return i_ >= n_; }
  void skip_ws() {
    while (!eof() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  static bool digit(char c) { return c >= '0' && c <= '9'; }

  Json value(int depth) {
    if (depth > 256) fail("nesting deeper than 256");
    if (eof()) fail("unexpected end of input, expected a value");
    const char c = s_[i_];
    if (c == '{') return object(depth + 1);
    if (c == '[') return array(depth + 1);
    if (c == '"') {
      Json v;
      v.kind = Json::String;
      v.text = string();
      return v;
    }
    if (c == 't') return literal("true");
    if (c == 'f') return literal("false");
    if (c == 'n') return literal("null");
    if (c == '-' || digit(c)) return number();
    fail(std::string("unexpected character '") + c + "', expected a value");
  }

  Json literal(const char* word) {
    const size_t len = std::strlen(word);
    if (n_ - i_ < len || std::memcmp(s_ + i_, word, len) != 0) fail(std::string("invalid literal, expected ") + word);
    i_ += len;
    Json v;
    if (word[0] == 'n') {
      v.kind = Json::Null;
    } else {
      v.kind = Json::Bool;
      v.boolean = word[0] == 't';
    }
    return v;
  }

  Json number() {
    const size_t start = i_;
    if (s_[i_] == '-') ++i_;
    if (eof() || !digit(s_[i_])) fail("invalid number: expected a digit");
    if (s_[i_] == '0') {
      ++i_;
      if (!eof() && digit(s_[i_])) fail("invalid number: leading zero");
    } else {
      while (!eof() && digit(s_[i_])) ++i_;
    }
    bool integral = true;
    if (!eof() && s_[i_] == '.') {
      ++i_;
      integral = false;
      if (eof() || !digit(s_[i_])) fail("invalid number: expected a digit after '.'");
      while (!eof() && digit(s_[i_])) ++i_;
    }
    if (!eof() && (s_[i_] == 'e' || s_[i_] == 'E')) {
      ++i_;
      integral = false;
      if (!eof() && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
      if (eof() || !digit(s_[i_])) fail("invalid number: expected a digit in the exponent");
      while (!eof() && digit(s_[i_])) ++i_;
    }
    Json v;
    v.kind = Json::Number;
    v.text.assign(s_ + start, i_ - start);
    const char* b = v.text.data();
    const char* e = b + v.text.size();
    double d = 0.0;
    const auto rd = std::from_chars(b, e, d);
    if (rd.ec == std::errc::result_out_of_range) {
      if (!underflows(v.text)) fail("number out of range: " + v.text);
      d = v.text[0] == '-' ? -0.0 : 0.0;  // below the smallest subnormal: the value is zero
    }
    v.number = d;
    if (integral) {
      int64_t iv = 0;
      const auto ri = std::from_chars(b, e, iv);
      if (ri.ec == std::errc() && ri.ptr == e) {
        v.is_int = true;
        v.integer = iv;
      }
    }
    return v;
  }

  // Decimal exponent of the leading significant digit of a well-formed number that from_chars
  // found out of range: negative means the magnitude is below 1 (an underflow, not an overflow).
  static bool underflows(const std::string& t) {
    size_t i = t[0] == '-' ? 1 : 0;
    long lead = 0;  // position of the first non-zero digit relative to the decimal point
    bool seen = false, frac = false;
    long int_digits = 0, zeros_after_point = 0;
    for (; i < t.size() && t[i] != 'e' && t[i] != 'E'; ++i) {
      if (t[i] == '.') {
        frac = true;
        continue;
      }
      if (!seen && t[i] == '0') {
        if (frac) ++zeros_after_point;
        continue;
      }
      if (!seen) seen = true;
      if (!frac) ++int_digits;
    }
    if (!seen) return true;  // all-zero significand
    lead = int_digits > 0 ? int_digits - 1 : -(zeros_after_point + 1);
    long ex = 0;
    if (i < t.size()) {
      ++i;
      const bool neg = i < t.size() && t[i] == '-';
      if (i < t.size() && (t[i] == '+' || t[i] == '-')) ++i;
      for (; i < t.size(); ++i) ex = std::min(ex * 10 + (t[i] - '0'), 100000000L);
      if (neg) ex = -ex;
    }
    return lead + ex < 0;
  }

  // Length of the well-formed UTF-8 sequence starting at s_[i] (Unicode Table 3-7), 0 if none.
  size_t utf8_len(size_t i) const {
    auto at = [&](size_t k) { return k < n_ ? static_cast<unsigned char>(s_[k]) : 0x100u; };
    auto in = [&](size_t k, unsigned lo, unsigned hi) { return at(k) >= lo && at(k) <= hi; };
    const unsigned b = at(i);
    if (b >= 0xC2 && b <= 0xDF) return in(i + 1, 0x80, 0xBF) ? 2 : 0;
    if (b >= 0xE0 && b <= 0xEF) {
      const unsigned lo = b == 0xE0 ? 0xA0 : 0x80, hi = b == 0xED ? 0x9F : 0xBF;
      return in(i + 1, lo, hi) && in(i + 2, 0x80, 0xBF) ? 3 : 0;
    }
    if (b >= 0xF0 && b <= 0xF4) {
      const unsigned lo = b == 0xF0 ? 0x90 : 0x80, hi = b == 0xF4 ? 0x8F : 0xBF;
      return in(i + 1, lo, hi) && in(i + 2, 0x80, 0xBF) && in(i + 3, 0x80, 0xBF) ? 4 : 0;
    }
    return 0;
  }

  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xC0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xE0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      out += static_cast<char>(0xF0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }

  uint32_t hex4() {
    if (n_ - i_ < 4) fail("truncated \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
      else fail("invalid hex digit in \\u escape");
    }
    return v;
  }

  std::string string() {
    ++i_;  // opening quote
    std::string out;
    while (true) {
      if (eof()) fail("unterminated string");
      const unsigned char c = static_cast<unsigned char>(s_[i_]);
      if (c == '"') {
        ++i_;
        return out;
      }
      if (c < 0x20) fail("control character in string");
      if (c >= 0x80) {
        const size_t len = utf8_len(i_);
        if (len == 0) fail("invalid UTF-8 byte sequence in string");
        out.append(s_ + i_, len);
        i_ += len;
        continue;
      }
      if (c != '\\') {
        out += static_cast<char>(c);
        ++i_;
        continue;
      }
      ++i_;
      if (eof()) fail("unterminated escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
            if (n_ - i_ < 2 || s_[i_] != '\\' || s_[i_ + 1] != 'u') fail("unpaired surrogate in \\u escape");
            i_ += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("unpaired surrogate in \\u escape");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            fail("unpaired surrogate in \\u escape");
          }
          utf8(out, cp);
          break;
        }
        default: fail(std::string("invalid escape \\") + e);
      }
    }
  }

  Json array(int depth) {
    ++i_;
    Json v;
    v.kind = Json::Array;
    skip_ws();
    if (!eof() && s_[i_] == ']') {
      ++i_;
      return v;
    }
    while (true) {
      skip_ws();
      v.items.push_back(value(depth));
      skip_ws();
      if (eof()) fail("unexpected end of input inside an array");
      if (s_[i_] == ',') {
        ++i_;
        skip_ws();
        if (!eof() && s_[i_] == ']') fail("trailing comma in array");
        continue;
      }
      if (s_[i_] == ']') {
        ++i_;
        return v;
      }
      fail("expected ',' or ']' in array");
    }
  }

  Json object(int depth) {
    ++i_;
    Json v;
    v.kind = Json::Object;
    skip_ws();
    if (!eof() && s_[i_] == '}') {
      ++i_;
      return v;
    }
    std::unordered_map<std::string, size_t> seen;
    while (true) {
      skip_ws();
      if (eof() || s_[i_] != '"') fail("expected a string key in object");
      std::string key = string();
      skip_ws();
      if (eof() || s_[i_] != ':') fail("expected ':' after object key");
      ++i_;
      skip_ws();
      Json item = value(depth);
      if (!seen.emplace(key, v.keys.size()).second) fail("duplicate key \"" + key + "\"");
      v.keys.push_back(std::move(key));
      v.items.push_back(std::move(item));
      skip_ws();
      if (eof()) fail("unexpected end of input inside an object");
      if (s_[i_] == ',') {
        ++i_;
        skip_ws();
        if (!eof() && s_[i_] == '}') fail("trailing comma in object");
        continue;
      }
      if (s_[i_] == '}') {
        ++i_;
        return v;
      }
      fail("expected ',' or '}' in object");
    }
  }
};

uint64_t le(const uint8_t* p, int n) {
  uint64_t v = 0;
  for (int i = n - 1; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}

bool is_norm(const std::string& name) { return name.find("norm") != std::string::npos; }

int qtype_from(const std::string& s) {  // "Q4_0" or "q4_0" (src/quant.cpp:114-121)
  for (int t = EF_QTYPE_F32; t <= EF_QTYPE_Q4_0; ++t) {
    std::string lower = qtype_name(t);
    for (char& ch : lower) ch = static_cast<char>(std::tolower(static_cast<unsigned char>(ch)));
    if (s == qtype_name(t) || s == lower) return t;
  }
  return -1;
}

std::string shape_str(const std::vector<uint64_t>& s) {
  std::string out = "[";
  for (size_t i = 0; i < s.size(); ++i) out += (i ? ", " : "") + std::to_string(s[i]);
  return out + "]";
}

// ---- config.json fields (src/model_config.cpp:18-70 semantics)
const Json* field(const Json& root, const char* key) {
  const Json* v = root.find(key);
  return v == nullptr || v->kind == Json::Null ? nullptr : v;
}

int64_t int_field(const Json& root, const char* key, int64_t lo, int64_t hi, const int64_t* def) {
  const Json* v = field(root, key);
  if (v == nullptr) {
    if (def != nullptr) return *def;
    throw Error(std::string("config.json: missing required field '") + key + "'");
  }
  if (v->kind != Json::Number || !v->is_int)
    throw Error(std::string("config.json: '") + key + "' must be an integer, got " +
                (v->kind == Json::Number ? v->text : std::string(kind_name(v->kind))));
  if (v->integer < lo || v->integer > hi) {
    throw Error(std::string("config.json: '") + key + "' = " + std::to_string(v->integer) + " is outside [" +
                std::to_string(lo) + ", " + std::to_string(hi) + "]");
  }
  return v->integer;
}

double num_field(const Json& root, const char* key, const double* def) {
  const Json* v = field(root, key);
  if (v == nullptr) {
    if (def != nullptr) return *def;
    throw Error(std::string("config.json: missing required field '") + key + "'");
  }
  if (v->kind != Json::Number)
    throw Error(std::string("config.json: '") + key + "' must be a number, got " + kind_name(v->kind));
  return v->number;
}

bool bool_field(const Json& root, const char* key, bool def) {
  const Json* v = field(root, key);
  if (v == nullptr) return def;
  if (v->kind != Json::Bool) throw Error(std::string("config.json: '") + key + "' must be true or false");
  return v->boolean;
}

std::string str_field(const Json& root, const char* key, const std::string& def) {
  const Json* v = field(root, key);
  if (v == nullptr) return def;
  if (v->kind != Json::String) throw Error(std::string("config.json: '") + key + "' must be a string");
  return v->text;
}

}  // namespace

Json parse_json(const char* text, size_t n) { return JsonReader(text, n).document(); }

// ---------------------------------------------------------------- types, policy, config

const char* qtype_name(int t) {
  switch (t) {
    case EF_QTYPE_F32: return "F32";
    case EF_QTYPE_F16: return "F16";
    case EF_QTYPE_BF16: return "BF16";
    case EF_QTYPE_Q8_0: return "Q8_0";
    case EF_QTYPE_Q4_0: return "Q4_0";
    default: return "?";
  }
}

uint64_t row_bytes(int t, uint64_t cols) {  // src/quant.cpp:136-149
  switch (t) {
    case EF_QTYPE_F32: return cols * 4;
    case EF_QTYPE_F16:
    case EF_QTYPE_BF16: return cols * 2;
    case EF_QTYPE_Q8_0:
    case EF_QTYPE_Q4_0:
      if (cols % 32 != 0)
        throw Error(std::string(qtype_name(t)) + " needs a row length divisible by 32, got " + std::to_string(cols));
      return cols / 32 * (t == EF_QTYPE_Q8_0 ? 34 : 18);
    default: throw Error("unknown storage type");
  }
}

// '*' matches any run of characters (including none); every other character matches itself.
// Dynamic programming over pattern prefixes: reach[j] = the first j pattern characters can
// match the text consumed so far.
bool glob_match(const std::string& p, const std::string& s) {
  std::vector<char> reach(p.size() + 1, 0), next(p.size() + 1, 0);
  reach[0] = 1;
  for (size_t j = 0; j < p.size() && p[j] == '*'; ++j) reach[j + 1] = 1;
  for (char c : s) {
    std::fill(next.begin(), next.end(), 0);
    for (size_t j = 0; j < p.size(); ++j) {
      if (p[j] == '*') {
        if (reach[j] || reach[j + 1]) next[j + 1] = 1;  // the star absorbs c
      } else if (reach[j] && p[j] == c) {
        next[j + 1] = 1;
      }
    }
    for (size_t j = 0; j < p.size(); ++j)  // stars may also match nothing after a step
      if (p[j] == '*' && next[j]) next[j + 1] = 1;
    reach.swap(next);
  }
  return reach[p.size()] != 0;
}

Choice policy_choice(const Policy& p, const std::string& name, uint64_t cols) {  // src/qfile.cpp:66-78
  if (is_norm(name)) return {EF_QTYPE_F32, "norm"};
  Choice c{p.layers, "layers"};
  if (name == "model.embed_tokens.weight") c = {p.embed, "embed"};
  if (name == "lm_head.weight") c = {p.lm_head, "lm_head"};
  for (const Override& o : p.overrides)
    if (glob_match(o.pattern, name)) c = {o.qtype, "override"};
  if ((c.qtype == EF_QTYPE_Q4_0 || c.qtype == EF_QTYPE_Q8_0) && cols % 32 != 0) c = {EF_QTYPE_BF16, "fallback-bf16"};
  return c;
}

std::vector<Expected> expected_tensors(const Config& c) {
  const auto D = static_cast<uint64_t>(c.hidden_size), F = static_cast<uint64_t>(c.intermediate_size);
  const auto V = static_cast<uint64_t>(c.vocab_size), KV = static_cast<uint64_t>(c.kv_dim());
  std::vector<Expected> out;
  out.push_back({"model.embed_tokens.weight", {V, D}});
  for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    out.push_back({p + "self_attn.q_proj.weight", {D, D}});
    out.push_back({p + "self_attn.k_proj.weight", {KV, D}});
    out.push_back({p + "self_attn.v_proj.weight", {KV, D}});
    out.push_back({p + "self_attn.o_proj.weight", {D, D}});
    out.push_back({p + "mlp.gate_proj.weight", {F, D}});
    out.push_back({p + "mlp.up_proj.weight", {F, D}});
    out.push_back({p + "mlp.down_proj.weight", {D, F}});
    out.push_back({p + "input_layernorm.weight", {D}});
    out.push_back({p + "post_attention_layernorm.weight", {D}});
  }
  out.push_back({"model.norm.weight", {D}});
  if (!c.tie_word_embeddings) out.push_back({"lm_head.weight", {V, D}});
  return out;
}

Config parse_config(const Json& root) {
  if (root.kind != Json::Object) throw Error("config.json: top level must be a JSON object");
  Config c;
  const std::string model_type = str_field(root, "model_type", "");
  if (model_type != "llama")
    throw Error("config.json: model_type '" + model_type + "' is not supported (EdgeForge targets 'llama')");
  const std::string act = str_field(root, "hidden_act", "silu");
  if (act != "silu") throw Error("config.json: hidden_act '" + act + "' is not supported (expected 'silu')");
  constexpr int64_t kMaxDim = int64_t{1} << 20;
  c.hidden_size = int_field(root, "hidden_size", 1, kMaxDim, nullptr);
  c.intermediate_size = int_field(root, "intermediate_size", 1, kMaxDim, nullptr);
  c.num_hidden_layers = int_field(root, "num_hidden_layers", 1, 4096, nullptr);
  c.num_attention_heads = int_field(root, "num_attention_heads", 1, 4096, nullptr);
  c.num_key_value_heads = int_field(root, "num_key_value_heads", 1, 4096, &c.num_attention_heads);
  c.vocab_size = int_field(root, "vocab_size", 1, int64_t{1} << 24, nullptr);
  const int64_t def_pos = 2048, def_id = -1;
  c.max_position_embeddings = int_field(root, "max_position_embeddings", 1, int64_t{1} << 24, &def_pos);
  c.rms_norm_eps = num_field(root, "rms_norm_eps", nullptr);
  const double def_theta = 10000.0;
  c.rope_theta = num_field(root, "rope_theta", &def_theta);
  c.tie_word_embeddings = bool_field(root, "tie_word_embeddings", false);
  const bool attention_bias = bool_field(root, "attention_bias", false);
  const bool mlp_bias = bool_field(root, "mlp_bias", false);
  c.bos_token_id = int_field(root, "bos_token_id", -1, int64_t{1} << 24, &def_id);
  c.eos_token_id = int_field(root, "eos_token_id", -1, int64_t{1} << 24, &def_id);
  if (c.hidden_size % c.num_attention_heads != 0)
    throw Error("config.json: hidden_size " + std::to_string(c.hidden_size) + " is not divisible by num_attention_heads " +
                std::to_string(c.num_attention_heads));
  const int64_t def_hd = c.hidden_size / c.num_attention_heads;
  c.head_dim = int_field(root, "head_dim", 1, kMaxDim, &def_hd);
  if (c.head_dim * c.num_attention_heads != c.hidden_size)
    throw Error("config.json: head_dim * num_attention_heads must equal hidden_size");
  if (c.head_dim % 2 != 0) throw Error("config.json: head_dim must be even for RoPE");
  if (c.num_attention_heads % c.num_key_value_heads != 0)
    throw Error("config.json: num_attention_heads " + std::to_string(c.num_attention_heads) +
                " is not divisible by num_key_value_heads " + std::to_string(c.num_key_value_heads));
  if (!(c.rms_norm_eps > 0.0) || !std::isfinite(c.rms_norm_eps))
    throw Error("config.json: rms_norm_eps must be a positive finite number");
  if (!(c.rope_theta > 0.0) || !std::isfinite(c.rope_theta))
    throw Error("config.json: rope_theta must be a positive finite number");
  if (field(root, "rope_scaling") != nullptr)
    throw Error("config.json: rope_scaling is set; scaled RoPE is not supported yet");
  if (attention_bias) throw Error("config.json: attention_bias=true is not supported");
  if (mlp_bias) throw Error("config.json: mlp_bias=true is not supported");
  return c;
}

// ---------------------------------------------------------------- the file

Layout parse(const uint8_t* file, uint64_t size) {
  if (size < 16) throw Error("file too small to be an .efq model (" + std::to_string(size) + " bytes)");
  if (std::memcmp(file, "EFQ1", 4) != 0) throw Error("not an EdgeForge .efq file (bad magic)");
  const uint64_t version = le(file + 4, 4);
  if (version != 1)
    throw Error("unsupported .efq version " + std::to_string(version) + " (this build reads 1)");
  Layout L;
  L.header_len = le(file + 8, 8);
  if (L.header_len == 0 || L.header_len > 100000000ull || L.header_len > size - 16)
    throw Error("invalid .efq header length " + std::to_string(L.header_len));
  Json h;
  try {
    h = parse_json(reinterpret_cast<const char*>(file + 16), static_cast<size_t>(L.header_len));
  } catch (const Error& e) {
    throw Error(std::string("invalid .efq header: ") + e.what());
  }
  if (h.at("format").str() != "edgeforge-quant") throw Error(".efq header: wrong \"format\"");
  L.cfg = parse_config(h.at("config"));
  const uint64_t data_start = 16 + L.header_len;

  for (const Json& e : h.at("tensors").list()) {
    Tensor t;
    t.name = e.at("name").str();
    t.qtype = qtype_from(e.at("type").str());
    if (t.qtype < 0) throw Error("tensor '" + t.name + "': unknown type " + e.at("type").str());
    if (const Json* r = e.find("rule")) t.rule = r->str();
    for (const Json& d : e.at("shape").list()) t.shape.push_back(d.u64());
    if (t.shape.empty() || t.shape.size() > 2) throw Error("tensor '" + t.name + "': shape must be 1-D or 2-D");
    t.offset = e.at("offset").u64();
    t.bytes = e.at("bytes").u64();
    if (const Json* r = e.find("rel_rmse")) t.rel_rmse = r->dbl();
    if (const Json* r = e.find("max_abs_err")) t.max_abs_err = r->dbl();
    const uint64_t rb = row_bytes(t.qtype, t.cols());
    if (t.rows() != 0 && rb > std::numeric_limits<uint64_t>::max() / t.rows())
      throw Error("tensor '" + t.name + "': size overflows");
    if (rb * t.rows() != t.bytes)
      throw Error("tensor '" + t.name + "': " + qtype_name(t.qtype) + " " + shape_str(t.shape) + " needs " +
                  std::to_string(rb * t.rows()) + " bytes, header says " + std::to_string(t.bytes));
    if (t.offset % 64 != 0) throw Error("tensor '" + t.name + "': offset is not 64-byte aligned");
    if (t.offset < data_start) throw Error("tensor '" + t.name + "': data overlaps the header");
    if (t.offset > size || t.bytes > size - t.offset)
      throw Error("tensor '" + t.name + "': data runs past the end of the file (truncated?)");
    L.tensors.push_back(std::move(t));
  }
  std::vector<size_t> order(L.tensors.size());
  std::iota(order.begin(), order.end(), size_t{0});
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return L.tensors[a].offset < L.tensors[b].offset; });
  for (size_t i = 1; i < order.size(); ++i) {
    const Tensor& p = L.tensors[order[i - 1]];
    const Tensor& c = L.tensors[order[i]];
    if (c.offset < p.offset + p.bytes) throw Error("tensors '" + p.name + "' and '" + c.name + "' overlap");
  }

  std::unordered_map<std::string, const Tensor*> by_name;
  for (const Tensor& t : L.tensors)
    if (!by_name.emplace(t.name, &t).second) throw Error("duplicate tensor '" + t.name + "'");
  const std::vector<Expected> expected = expected_tensors(L.cfg);
  for (const Expected& e : expected) {
    const auto it = by_name.find(e.name);
    if (it == by_name.end()) throw Error("missing tensor '" + e.name + "'");
    if (it->second->shape != e.shape)
      throw Error("tensor '" + e.name + "' has shape " + shape_str(it->second->shape) + ", config needs " +
                  shape_str(e.shape));
  }
  if (by_name.size() != expected.size()) throw Error(".efq file has tensors the config does not use");

  const Json& qs = h.at("quant");
  const Json* ov = qs.find("overrides");
  if (ov == nullptr)
    throw Error(".efq header has no \"overrides\" table: written by an older pre-release build, re-run "
                "edgeforge quantize");
  auto type_field = [](const Json& v, const char* what) {
    const int t = qtype_from(v.str());
    if (t < 0) throw Error(std::string(".efq header: unknown ") + what + " type " + v.str());
    return t;
  };
  L.policy.layers = type_field(qs.at("layers"), "layers");
  L.policy.lm_head = type_field(qs.at("lm_head"), "lm_head");
  L.policy.embed = type_field(qs.at("embed"), "embed");
  if (qs.at("norms").str() != "F32") throw Error(".efq header: norms must be F32");
  if (const Json* n = qs.find("policy")) L.policy.name = n->str();
  for (const Json& o : ov->list())
    L.policy.overrides.push_back({o.at("pattern").str(), type_field(o.at("type"), "override")});
  for (const Override& o : L.policy.overrides) {  // check_overrides (src/qfile.cpp:80-93)
    if (o.pattern.empty()) throw Error("override with an empty tensor pattern");
    size_t hits = 0;
    for (const Expected& e : expected) {
      if (!glob_match(o.pattern, e.name)) continue;
      if (is_norm(e.name))
        throw Error("override '" + o.pattern + "' matches norm tensor '" + e.name + "' (norms are always F32)");
      ++hits;
    }
    if (hits == 0) throw Error("override '" + o.pattern + "' matches no tensor of this model");
  }
  for (const Tensor& t : L.tensors) {
    const Choice c = policy_choice(L.policy, t.name, t.cols());
    if (t.qtype != c.qtype || t.rule != c.rule)
      throw Error("tensor '" + t.name + "' is stored as " + qtype_name(t.qtype) + " (rule \"" + t.rule +
                  "\") but the file's quantization policy gives " + qtype_name(c.qtype) + " (rule \"" + c.rule +
                  "\")");
  }
  return L;
}

void File::index() {
  for (size_t i = 0; i < L_.tensors.size(); ++i) {
    index_.emplace(L_.tensors[i].name, i);
    if (L_.tensors[i].name != "model.embed_tokens.weight") bytes_per_token_ += L_.tensors[i].bytes;
  }
  if (L_.cfg.tie_word_embeddings) bytes_per_token_ += at("model.embed_tokens.weight").bytes;
}

std::unique_ptr<File> File::open(const std::string& path) {
  std::unique_ptr<File> f(new File());
  f->path_ = path;
  f->fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (f->fd_ < 0) throw Error("cannot open '" + path + "': " + std::strerror(errno));
  struct stat st {};
  if (::fstat(f->fd_, &st) != 0) throw Error("cannot stat '" + path + "': " + std::strerror(errno));
  if (!S_ISREG(st.st_mode)) throw Error("'" + path + "' is not a regular file");
  f->size_ = static_cast<uint64_t>(st.st_size);
  if (f->size_ > 0) {
    void* p = ::mmap(nullptr, static_cast<size_t>(f->size_), PROT_READ, MAP_PRIVATE, f->fd_, 0);
    if (p == MAP_FAILED) throw Error("cannot mmap '" + path + "': " + std::strerror(errno));
    f->map_ = p;
    f->base_ = static_cast<const uint8_t*>(p);
  }
  static const uint8_t kEmpty[1] = {0};
  try {
    f->L_ = parse(f->base_ ? f->base_ : kEmpty, f->size_);
  } catch (const Error& e) {
    throw Error("'" + path + "': " + e.what());
  }
  f->index();
  return f;
}

std::unique_ptr<File> File::over(const uint8_t* bytes, uint64_t size) {
  std::unique_ptr<File> f(new File());
  f->base_ = bytes;
  f->size_ = size;
  f->L_ = parse(bytes, size);
  f->index();
  return f;
}

File::~File() {
  if (map_ != nullptr) ::munmap(map_, static_cast<size_t>(size_));
  if (fd_ >= 0) ::close(fd_);
}

const Tensor* File::find(const std::string& name) const {
  const auto it = index_.find(name);
  return it == index_.end() ? nullptr : &L_.tensors[it->second];
}

const Tensor& File::at(const std::string& name) const {
  if (const Tensor* t = find(name)) return *t;
  throw Error("tensor '" + name + "' not found in '" + path_ + "'");
}

}  // namespace efh::efq
