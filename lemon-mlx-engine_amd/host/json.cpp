// json.cpp -- the recursive-descent reader declared in json.hpp.
#include "json.hpp"

#include <cmath>
#include <cstdlib>
#include <stdexcept>

namespace mlx_lm {
namespace mi355x {

namespace {
[[noreturn]] void type_error(const char* want) { throw std::invalid_argument(std::string("json: not a ") + want); }
}  // namespace

const std::string& Json::str() const {
  if (type_ != Type::string) type_error("string");
  return s_;
}
double Json::num() const {
  if (type_ != Type::number) type_error("number");
  return n_;
}
int64_t Json::integer() const {
  const double v = num();
  if (v != std::floor(v) || std::fabs(v) > 9.007199254740992e15) type_error("integer");
  return static_cast<int64_t>(v);
}
bool Json::boolean() const {
  if (type_ != Type::boolean) type_error("boolean");
  return b_;
}
const std::vector<Json>& Json::items() const {
  if (type_ != Type::array) type_error("array");
  return a_;
}
const std::map<std::string, Json>& Json::fields() const {
  if (type_ != Type::object) type_error("object");
  return o_;
}
bool Json::contains(const std::string& key) const { return type_ == Type::object && o_.count(key) != 0; }
const Json& Json::at(const std::string& key) const {
  const auto& f = fields();
  const auto it = f.find(key);
  if (it == f.end()) throw std::invalid_argument("json: missing key '" + key + "'");
  return it->second;
}
int64_t Json::value(const std::string& key, int64_t fallback) const {
  return contains(key) && !at(key).is_null() ? at(key).integer() : fallback;
}
double Json::value(const std::string& key, double fallback) const {
  return contains(key) && !at(key).is_null() ? at(key).num() : fallback;
}
bool Json::value(const std::string& key, bool fallback) const {
  return contains(key) && !at(key).is_null() ? at(key).boolean() : fallback;
}

class JsonParser {
 public:
  explicit JsonParser(const std::string& t) : t_(t) {}

  Json document() {
    Json v = value(0);
    ws();
    if (i_ != t_.size()) fail("trailing characters");
    return v;
  }

 private:
  const std::string& t_;
  size_t i_ = 0;

  [[noreturn]] void fail(const char* what) const {
    throw std::invalid_argument(std::string("json: ") + what + " at offset " + std::to_string(i_));
  }
  void ws() {
    while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\t' || t_[i_] == '\n' || t_[i_] == '\r')) ++i_;
  }
  char peek() {
    ws();
    if (i_ >= t_.size()) fail("unexpected end");
    return t_[i_];
  }
  void expect(char c) {
    if (peek() != c) fail("unexpected character");
    ++i_;
  }
  bool literal(const char* word) {
    const std::string w(word);
    if (t_.compare(i_, w.size(), w) != 0) return false;
    i_ += w.size();
    return true;
  }

  Json value(int depth) {
    if (depth > 64) fail("nesting too deep");
    Json v;
    const char c = peek();
    if (c == '{') {
      v.type_ = Json::Type::object;
      ++i_;
      if (peek() == '}') {
        ++i_;
        return v;
      }
      for (;;) {
        if (peek() != '"') fail("object key expected");
        std::string key = string_body();
        expect(':');
        v.o_[key] = value(depth + 1);
        const char d = peek();
        ++i_;
        if (d == '}') break;
        if (d != ',') fail("',' or '}' expected");
      }
    } else if (c == '[') {
      v.type_ = Json::Type::array;
      ++i_;
      if (peek() == ']') {
        ++i_;
        return v;
      }
      for (;;) {
        v.a_.push_back(value(depth + 1));
        const char d = peek();
        ++i_;
        if (d == ']') break;
        if (d != ',') fail("',' or ']' expected");
      }
    } else if (c == '"') {
      v.type_ = Json::Type::string;
      v.s_ = string_body();
    } else if (literal("true")) {
      v.type_ = Json::Type::boolean;
      v.b_ = true;
    } else if (literal("false")) {
      v.type_ = Json::Type::boolean;
    } else if (literal("null")) {
      v.type_ = Json::Type::null;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      const char* begin = t_.c_str() + i_;
      char* end = nullptr;
      v.type_ = Json::Type::number;
      v.n_ = std::strtod(begin, &end);
      if (end == begin) fail("bad number");
      i_ += static_cast<size_t>(end - begin);
    } else {
      fail("unexpected character");
    }
    return v;
  }

  static void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xc0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xe0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    } else {
      out += static_cast<char>(0xf0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3f));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    }
  }
  uint32_t hex4() {
    if (i_ + 4 > t_.size()) fail("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = t_[i_++];
      v <<= 4;
      if (h >= '0' && h <= '9') v |= static_cast<uint32_t>(h - '0');
      else if (h >= 'a' && h <= 'f') v |= static_cast<uint32_t>(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') v |= static_cast<uint32_t>(h - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string string_body() {
    expect('"');
    std::string out;
    for (;;) {
      if (i_ >= t_.size()) fail("unterminated string");
      const char c = t_[i_++];
      if (c == '"') return out;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= t_.size()) fail("unterminated escape");
      const char e = t_[i_++];
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
          if (cp >= 0xd800 && cp < 0xdc00 && i_ + 1 < t_.size() && t_[i_] == '\\' && t_[i_ + 1] == 'u') {
            i_ += 2;
            const uint32_t lo = hex4();
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          put_utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }
};

Json parse_json(const std::string& text) { return JsonParser(text).document(); }

}  // namespace mi355x
}  // namespace mlx_lm
