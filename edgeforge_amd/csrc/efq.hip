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

}  // namespace

Json parse_json(const char* text, size_t n) { return JsonReader(text, n).document(); }

// ---------------------------------------------------------------- types

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

// ---------------------------------------------------------------- config.json as a rule table
//
// The model-config fields are validated by walking one ordered table (src/model_config.cpp:72-131
// gives the semantics: which fields, their ranges and defaults, the accepted values, and which
// failure a file with several problems reports first).  A field row reads and checks one key; a
// constraint row checks fields read by earlier rows.  Reading follows the table's order, so the
// first failing row decides the message.

namespace {

struct ConfigState {
  const Json* root = nullptr;
  std::unordered_map<std::string, int64_t> ints;
  std::unordered_map<std::string, double> reals;
  std::unordered_map<std::string, bool> flags;
  std::unordered_map<std::string, std::string> texts;
};

enum class Row : uint8_t { Text, Int, Real, Flag, Constraint };
// How an absent (or null) key is treated.
enum class Absent : uint8_t { Required, Constant, SameAs, Quotient };

struct ConfigRow {
  Row kind;
  const char* key;            // the config.json key (Constraint rows: a label only)
  Absent absent;
  int64_t lo, hi;             // Int rows: accepted range
  double constant;            // Absent::Constant numeric default
  const char* text;           // Text default (Constant), or the key whose value is the default (SameAs),
                              // or the dividend key of a quotient default (Quotient)
  const char* text2;          // Quotient: the divisor key
  bool (*ok)(const ConfigState&);                 // Constraint rows, and Text rows with one accepted value
  std::string (*why)(const ConfigState&);         // message when ok() fails
};

const Json* present(const Json& root, const char* key) {
  const Json* v = root.find(key);
  return v == nullptr || v->kind == Json::Null ? nullptr : v;
}

std::string quoted(const char* key) { return std::string("config.json: '") + key + "'"; }

void read_row(const ConfigRow& r, ConfigState& st) {
  // an optional key given as null takes its default; a required key must be there, null or not,
  // and a null one fails its type check
  const Json* v = r.absent == Absent::Required ? st.root->find(r.key) : present(*st.root, r.key);
  const bool have = v != nullptr;
  if (!have && r.absent == Absent::Required) throw Error(std::string("config.json: missing required field '") + r.key + "'");
  switch (r.kind) {
    case Row::Text: {
      std::string val;
      if (have) {
        if (v->kind != Json::String) throw Error(quoted(r.key) + " must be a string");
        val = v->text;
      } else {
        val = r.absent == Absent::SameAs ? st.texts[r.text] : std::string(r.text ? r.text : "");
      }
      st.texts[r.key] = val;
      break;
    }
    case Row::Int: {
      int64_t val = 0;
      if (have) {
        if (v->kind != Json::Number || !v->is_int)
          throw Error(quoted(r.key) + " must be an integer, got " +
                      (v->kind == Json::Number ? v->text : std::string(kind_name(v->kind))));
        val = v->integer;
        if (val < r.lo || val > r.hi)
          throw Error(quoted(r.key) + " = " + std::to_string(val) + " is outside [" + std::to_string(r.lo) + ", " +
                      std::to_string(r.hi) + "]");
      } else if (r.absent == Absent::SameAs) {
        val = st.ints[r.text];
      } else if (r.absent == Absent::Quotient) {
        val = st.ints[r.text] / st.ints[r.text2];
      } else {
        val = static_cast<int64_t>(r.constant);
      }
      st.ints[r.key] = val;
      break;
    }
    case Row::Real: {
      double val = r.constant;
      if (have) {
        if (v->kind != Json::Number) throw Error(quoted(r.key) + " must be a number, got " + kind_name(v->kind));
        val = v->number;
      }
      st.reals[r.key] = val;
      break;
    }
    case Row::Flag: {
      bool val = r.constant != 0.0;
      if (have) {
        if (v->kind != Json::Bool) throw Error(quoted(r.key) + " must be true or false");
        val = v->boolean;
      }
      st.flags[r.key] = val;
      break;
    }
    case Row::Constraint: break;
  }
  if (r.ok != nullptr && !r.ok(st)) throw Error("config.json: " + r.why(st));
}

int64_t I(const ConfigState& s, const char* k) { return s.ints.at(k); }
double R(const ConfigState& s, const char* k) { return s.reals.at(k); }
bool positive_finite(double v) { return v > 0.0 && std::isfinite(v); }

constexpr int64_t kMaxDim = int64_t{1} << 20;
constexpr int64_t kMaxId = int64_t{1} << 24;

const ConfigRow kConfigRows[] = {
    {Row::Text, "model_type", Absent::Constant, 0, 0, 0.0, "", nullptr,
     [](const ConfigState& s) { return s.texts.at("model_type") == "llama"; },
     [](const ConfigState& s) {
       return "model_type '" + s.texts.at("model_type") + "' is not supported (EdgeForge targets 'llama')";
     }},
    {Row::Text, "hidden_act", Absent::Constant, 0, 0, 0.0, "silu", nullptr,
     [](const ConfigState& s) { return s.texts.at("hidden_act") == "silu"; },
     [](const ConfigState& s) { return "hidden_act '" + s.texts.at("hidden_act") + "' is not supported (expected 'silu')"; }},
    // informational strings: only their JSON type is checked ("torch_dtype" defaults to "dtype")
    {Row::Text, "dtype", Absent::Constant, 0, 0, 0.0, "", nullptr, nullptr, nullptr},
    {Row::Text, "torch_dtype", Absent::SameAs, 0, 0, 0.0, "dtype", nullptr, nullptr, nullptr},
    {Row::Int, "hidden_size", Absent::Required, 1, kMaxDim, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Int, "intermediate_size", Absent::Required, 1, kMaxDim, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Int, "num_hidden_layers", Absent::Required, 1, 4096, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Int, "num_attention_heads", Absent::Required, 1, 4096, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Int, "num_key_value_heads", Absent::SameAs, 1, 4096, 0.0, "num_attention_heads", nullptr, nullptr, nullptr},
    {Row::Int, "vocab_size", Absent::Required, 1, kMaxId, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Int, "max_position_embeddings", Absent::Constant, 1, kMaxId, 2048.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Real, "rms_norm_eps", Absent::Required, 0, 0, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Real, "rope_theta", Absent::Constant, 0, 0, 10000.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Flag, "tie_word_embeddings", Absent::Constant, 0, 0, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Flag, "attention_bias", Absent::Constant, 0, 0, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Flag, "mlp_bias", Absent::Constant, 0, 0, 0.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Int, "bos_token_id", Absent::Constant, -1, kMaxId, -1.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Int, "eos_token_id", Absent::Constant, -1, kMaxId, -1.0, nullptr, nullptr, nullptr, nullptr},
    {Row::Constraint, "heads divide hidden", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return I(s, "hidden_size") % I(s, "num_attention_heads") == 0; },
     [](const ConfigState& s) {
       return "hidden_size " + std::to_string(I(s, "hidden_size")) + " is not divisible by num_attention_heads " +
              std::to_string(I(s, "num_attention_heads"));
     }},
    {Row::Int, "head_dim", Absent::Quotient, 1, kMaxDim, 0.0, "hidden_size", "num_attention_heads", nullptr, nullptr},
    {Row::Constraint, "head_dim x heads", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return I(s, "head_dim") * I(s, "num_attention_heads") == I(s, "hidden_size"); },
     [](const ConfigState&) { return std::string("head_dim * num_attention_heads must equal hidden_size"); }},
    {Row::Constraint, "even head_dim", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return I(s, "head_dim") % 2 == 0; },
     [](const ConfigState&) { return std::string("head_dim must be even for RoPE"); }},
    {Row::Constraint, "kv heads divide heads", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return I(s, "num_attention_heads") % I(s, "num_key_value_heads") == 0; },
     [](const ConfigState& s) {
       return "num_attention_heads " + std::to_string(I(s, "num_attention_heads")) +
              " is not divisible by num_key_value_heads " + std::to_string(I(s, "num_key_value_heads"));
     }},
    {Row::Constraint, "eps", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return positive_finite(R(s, "rms_norm_eps")); },
     [](const ConfigState&) { return std::string("rms_norm_eps must be a positive finite number"); }},
    {Row::Constraint, "theta", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return positive_finite(R(s, "rope_theta")); },
     [](const ConfigState&) { return std::string("rope_theta must be a positive finite number"); }},
    {Row::Constraint, "rope scaling", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return present(*s.root, "rope_scaling") == nullptr; },
     [](const ConfigState&) { return std::string("rope_scaling is set; scaled RoPE is not supported yet"); }},
    {Row::Constraint, "attention bias", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return !s.flags.at("attention_bias"); },
     [](const ConfigState&) { return std::string("attention_bias=true is not supported"); }},
    {Row::Constraint, "mlp bias", Absent::Constant, 0, 0, 0.0, nullptr, nullptr,
     [](const ConfigState& s) { return !s.flags.at("mlp_bias"); },
     [](const ConfigState&) { return std::string("mlp_bias=true is not supported"); }},
};

}  // namespace

Config parse_config(const Json& root) {
  if (root.kind != Json::Object) throw Error("config.json: top level must be a JSON object");
  ConfigState st;
  st.root = &root;
  for (const ConfigRow& r : kConfigRows) read_row(r, st);
  Config c;
  c.hidden_size = I(st, "hidden_size");
  c.intermediate_size = I(st, "intermediate_size");
  c.num_hidden_layers = I(st, "num_hidden_layers");
  c.num_attention_heads = I(st, "num_attention_heads");
  c.num_key_value_heads = I(st, "num_key_value_heads");
  c.head_dim = I(st, "head_dim");
  c.vocab_size = I(st, "vocab_size");
  c.max_position_embeddings = I(st, "max_position_embeddings");
  c.bos_token_id = I(st, "bos_token_id");
  c.eos_token_id = I(st, "eos_token_id");
  c.rms_norm_eps = R(st, "rms_norm_eps");
  c.rope_theta = R(st, "rope_theta");
  c.tie_word_embeddings = st.flags.at("tie_word_embeddings");
  return c;
}

// ---------------------------------------------------------------- tensors the config implies

namespace {
// A tensor slot: name (a per-layer suffix or a whole name) and its shape in model dimensions
// ('D' hidden, 'F' intermediate, 'K' KV width, 'V' vocabulary, 0 for the second dim of a 1-D norm).
struct Slot {
  const char* name;
  char rows, cols;
};
constexpr Slot kLayerSlots[] = {
    {"self_attn.q_proj.weight", 'D', 'D'}, {"self_attn.k_proj.weight", 'K', 'D'},
    {"self_attn.v_proj.weight", 'K', 'D'}, {"self_attn.o_proj.weight", 'D', 'D'},
    {"mlp.gate_proj.weight", 'F', 'D'},    {"mlp.up_proj.weight", 'F', 'D'},
    {"mlp.down_proj.weight", 'D', 'F'},    {"input_layernorm.weight", 'D', 0},
    {"post_attention_layernorm.weight", 'D', 0},
};
}  // namespace

// Forward order: the embedding, each layer's slots, the final norm, then the lm_head unless tied
// to the embedding (src/model_config.cpp:145-167 lists the same set).
std::vector<Expected> expected_tensors(const Config& c) {
  auto dim = [&](char d) -> uint64_t {
    switch (d) {
      case 'D': return static_cast<uint64_t>(c.hidden_size);
      case 'F': return static_cast<uint64_t>(c.intermediate_size);
      case 'K': return static_cast<uint64_t>(c.kv_dim());
      default: return static_cast<uint64_t>(c.vocab_size);
    }
  };
  auto shape = [&](const Slot& s) {
    return s.cols ? std::vector<uint64_t>{dim(s.rows), dim(s.cols)} : std::vector<uint64_t>{dim(s.rows)};
  };
  std::vector<Expected> out;
  out.reserve(static_cast<size_t>(c.num_hidden_layers) * std::size(kLayerSlots) + 3);
  out.push_back({"model.embed_tokens.weight", shape({nullptr, 'V', 'D'})});
  for (int64_t l = 0; l < c.num_hidden_layers; ++l)
    for (const Slot& s : kLayerSlots)
      out.push_back({"model.layers." + std::to_string(l) + "." + s.name, shape(s)});
  out.push_back({"model.norm.weight", shape({nullptr, 'D', 0})});
  if (!c.tie_word_embeddings) out.push_back({"lm_head.weight", shape({nullptr, 'V', 'D'})});
  return out;
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

// The storage type a file's policy assigns to a tensor (src/qfile.cpp:66-78 semantics): norms are
// always F32; otherwise the last override whose pattern matches wins over the tensor's role
// (embedding, lm_head, or a layer matrix); a block type on rows that are not whole blocks falls
// back to BF16.
Choice policy_choice(const Policy& p, const std::string& name, uint64_t cols) {
  if (is_norm(name)) return {EF_QTYPE_F32, "norm"};
  const auto hit = std::find_if(p.overrides.rbegin(), p.overrides.rend(),
                                [&](const Override& o) { return glob_match(o.pattern, name); });
  Choice c = hit != p.overrides.rend()              ? Choice{hit->qtype, "override"}
             : name == "lm_head.weight"             ? Choice{p.lm_head, "lm_head"}
             : name == "model.embed_tokens.weight"  ? Choice{p.embed, "embed"}
                                                    : Choice{p.layers, "layers"};
  const bool block = c.qtype == EF_QTYPE_Q4_0 || c.qtype == EF_QTYPE_Q8_0;
  if (block && cols % 32 != 0) c = {EF_QTYPE_BF16, "fallback-bf16"};
  return c;
}

// ---------------------------------------------------------------- the file

namespace {

// One header tensor entry, decoded in key order with each key's own check right after it (a
// malformed entry reports the first problem in that order).
Tensor decode_entry(const Json& e) {
  Tensor t;
  t.name = e.at("name").str();
  const std::string& type = e.at("type").str();
  t.qtype = qtype_from(type);
  if (t.qtype < 0) throw Error("tensor '" + t.name + "': unknown type " + type);
  if (const Json* r = e.find("rule")) t.rule = r->str();
  for (const Json& d : e.at("shape").list()) t.shape.push_back(d.u64());
  if (t.shape.empty() || t.shape.size() > 2) throw Error("tensor '" + t.name + "': shape must be 1-D or 2-D");
  t.offset = e.at("offset").u64();
  t.bytes = e.at("bytes").u64();
  if (const Json* r = e.find("rel_rmse")) t.rel_rmse = r->dbl();
  if (const Json* r = e.find("max_abs_err")) t.max_abs_err = r->dbl();
  return t;
}

// Checks of one decoded entry against the file, in the order a file with several problems reports
// them: size arithmetic, declared bytes, alignment, placement after the header, bounds.
struct Placement {
  uint64_t data_start, file_size;
};
struct EntryRule {
  bool (*bad)(const Tensor&, const Placement&, uint64_t need, bool overflow);
  std::string (*why)(const Tensor&, uint64_t need);
};
const EntryRule kEntryRules[] = {
    {[](const Tensor&, const Placement&, uint64_t, bool overflow) { return overflow; },
     [](const Tensor&, uint64_t) { return std::string("size overflows"); }},
    {[](const Tensor& t, const Placement&, uint64_t need, bool) { return need != t.bytes; },
     [](const Tensor& t, uint64_t need) {
       return std::string(qtype_name(t.qtype)) + " " + shape_str(t.shape) + " needs " + std::to_string(need) +
              " bytes, header says " + std::to_string(t.bytes);
     }},
    {[](const Tensor& t, const Placement&, uint64_t, bool) { return t.offset % 64 != 0; },
     [](const Tensor&, uint64_t) { return std::string("offset is not 64-byte aligned"); }},
    {[](const Tensor& t, const Placement& p, uint64_t, bool) { return t.offset < p.data_start; },
     [](const Tensor&, uint64_t) { return std::string("data overlaps the header"); }},
    {[](const Tensor& t, const Placement& p, uint64_t, bool) {
       return t.offset > p.file_size || t.bytes > p.file_size - t.offset;
     },
     [](const Tensor&, uint64_t) { return std::string("data runs past the end of the file (truncated?)"); }},
};

void check_entry(const Tensor& t, const Placement& where) {
  const uint64_t rb = row_bytes(t.qtype, t.cols());
  const bool overflow = t.rows() != 0 && rb > std::numeric_limits<uint64_t>::max() / t.rows();
  const uint64_t need = overflow ? 0 : rb * t.rows();
  for (const EntryRule& r : kEntryRules)
    if (r.bad(t, where, need, overflow)) throw Error("tensor '" + t.name + "': " + r.why(t, need));
}

// No two tensors' byte ranges intersect: walked in offset order (ties in header order), the first
// range that starts before its predecessor ends is reported with that predecessor.
void check_disjoint(const std::vector<Tensor>& ts) {
  std::vector<std::pair<uint64_t, size_t>> by_offset;
  by_offset.reserve(ts.size());
  for (size_t i = 0; i < ts.size(); ++i) by_offset.emplace_back(ts[i].offset, i);
  std::sort(by_offset.begin(), by_offset.end());
  uint64_t end = 0;
  const Tensor* prev = nullptr;
  for (const auto& [off, i] : by_offset) {
    if (prev != nullptr && off < end) throw Error("tensors '" + prev->name + "' and '" + ts[i].name + "' overlap");
    prev = &ts[i];
    end = off + ts[i].bytes;
  }
}

// Exactly the tensors the configuration implies, each once, with the implied shapes.
void check_names_and_shapes(const std::vector<Tensor>& ts, const std::vector<Expected>& want) {
  std::unordered_map<std::string, const Tensor*> seen;
  for (const Tensor& t : ts)
    if (!seen.emplace(t.name, &t).second) throw Error("duplicate tensor '" + t.name + "'");
  for (const Expected& e : want) {
    const auto it = seen.find(e.name);
    if (it == seen.end()) throw Error("missing tensor '" + e.name + "'");
    if (it->second->shape != e.shape)
      throw Error("tensor '" + e.name + "' has shape " + shape_str(it->second->shape) + ", config needs " +
                  shape_str(e.shape));
  }
  if (seen.size() != want.size()) throw Error(".efq file has tensors the config does not use");
}

// The header's quantization policy: the three role types, F32 norms, the override list (each must
// name at least one tensor of this model and no norm; src/qfile.cpp:80-93 semantics).
Policy read_policy(const Json& qs, const std::vector<Expected>& want) {
  const Json* table = qs.find("overrides");
  if (table == nullptr)
    throw Error(".efq header has no \"overrides\" table: written by an older pre-release build, re-run "
                "edgeforge quantize");
  auto type_of = [](const Json& v, const char* what) {
    const int t = qtype_from(v.str());
    if (t < 0) throw Error(std::string(".efq header: unknown ") + what + " type " + v.str());
    return t;
  };
  Policy p;
  p.layers = type_of(qs.at("layers"), "layers");
  p.lm_head = type_of(qs.at("lm_head"), "lm_head");
  p.embed = type_of(qs.at("embed"), "embed");
  if (qs.at("norms").str() != "F32") throw Error(".efq header: norms must be F32");
  if (const Json* n = qs.find("policy")) p.name = n->str();
  for (const Json& o : table->list()) p.overrides.push_back({o.at("pattern").str(), type_of(o.at("type"), "override")});
  for (const Override& o : p.overrides) {
    if (o.pattern.empty()) throw Error("override with an empty tensor pattern");
    auto matches = [&](const Expected& e) { return glob_match(o.pattern, e.name); };
    const auto norm = std::find_if(want.begin(), want.end(), [&](const Expected& e) { return matches(e) && is_norm(e.name); });
    if (norm != want.end())
      throw Error("override '" + o.pattern + "' matches norm tensor '" + norm->name + "' (norms are always F32)");
    if (std::none_of(want.begin(), want.end(), matches))
      throw Error("override '" + o.pattern + "' matches no tensor of this model");
  }
  return p;
}

}  // namespace

// parse_efq (src/qfile.cpp:125-223 semantics): the fixed preamble, the JSON header, the config,
// every tensor entry, then the cross-entry checks and the policy, each stage reporting its first
// problem with the reference's wording.
Layout parse(const uint8_t* file, uint64_t size) {
  if (size < 16) throw Error("file too small to be an .efq model (" + std::to_string(size) + " bytes)");
  if (std::memcmp(file, "EFQ1", 4) != 0) throw Error("not an EdgeForge .efq file (bad magic)");
  if (const uint64_t version = le(file + 4, 4); version != 1)
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
  const Placement where{16 + L.header_len, size};
  for (const Json& e : h.at("tensors").list()) {
    L.tensors.push_back(decode_entry(e));
    check_entry(L.tensors.back(), where);
  }
  check_disjoint(L.tensors);
  const std::vector<Expected> want = expected_tensors(L.cfg);
  check_names_and_shapes(L.tensors, want);
  L.policy = read_policy(h.at("quant"), want);
  for (const Tensor& t : L.tensors) {
    const Choice c = policy_choice(L.policy, t.name, t.cols());
    if (t.qtype != c.qtype || t.rule != c.rule)
      throw Error("tensor '" + t.name + "' is stored as " + qtype_name(t.qtype) + " (rule \"" + t.rule +
                  "\") but the file's quantization policy gives " + qtype_name(c.qtype) + " (rule \"" + c.rule +
                  "\")");
  }
  return L;
}

// Name -> index over the validated table, and the bytes one decoded token streams: every tensor but
// the embedding (one row of it is read per token), plus the embedding when it doubles as the lm_head.
void File::index() {
  index_.reserve(L_.tensors.size());
  for (size_t i = 0; i < L_.tensors.size(); ++i) index_.emplace(L_.tensors[i].name, i);
  const bool tied = L_.cfg.tie_word_embeddings;
  bytes_per_token_ = std::accumulate(L_.tensors.begin(), L_.tensors.end(), uint64_t{0},
                                     [&](uint64_t acc, const Tensor& t) {
                                       const bool embed = t.name == "model.embed_tokens.weight";
                                       return acc + (!embed || tied ? t.bytes : 0);
                                     });
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
  const Tensor* t = find(name);
  if (t == nullptr) throw Error("tensor '" + name + "' not found in '" + path_ + "'");
  return *t;
}

}  // namespace efh::efq
