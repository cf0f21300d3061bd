// Recursive-descent JSON reader (RFC 8259 grammar: literals, numbers, strings with escapes
// and UTF-16 surrogate pairs, arrays, objects), used for checkpoint metadata.
#include "fr_json.h"

#include <cstdlib>

#include "fr_runtime.h"

namespace fr {

namespace {
[[noreturn]] void parse_fail(const std::string& message) { fail(ErrorKind::Parse, message); }
}  // namespace

class JsonParser {
 public:
  explicit JsonParser(const std::string& s) : s_(s) {}

  JsonValue document() {
    JsonValue v = value(0);
    skip_ws();
    if (pos_ != s_.size()) parse_fail("unexpected trailing characters after JSON value at byte " + std::to_string(pos_));
    return v;
  }

 private:
  static constexpr int kMaxDepth = 512;
  const std::string& s_;
  size_t pos_ = 0;

  bool eof() const { return pos_ >= s_.size(); }
  char peek() const { return s_[pos_]; }
  void skip_ws() {
    while (!eof() && (peek() == ' ' || peek() == '\t' || peek() == '\n' || peek() == '\r')) ++pos_;
  }
  void expect(char c) {
    if (eof() || peek() != c) parse_fail(std::string("expected '") + c + "' at byte " + std::to_string(pos_));
    ++pos_;
  }

  JsonValue value(int depth) {
    if (depth > kMaxDepth) parse_fail("JSON nesting too deep");
    skip_ws();
    if (eof()) parse_fail("unexpected end of JSON input");
    const char c = peek();
    JsonValue v;
    if (c == '{') {
      v.kind_ = JsonValue::Kind::Object;
      ++pos_;
      skip_ws();
      if (!eof() && peek() == '}') {
        ++pos_;
        return v;
      }
      for (;;) {
        skip_ws();
        if (eof() || peek() != '"') parse_fail("expected object key at byte " + std::to_string(pos_));
        std::string key = string_body();
        skip_ws();
        expect(':');
        v.object_[key] = value(depth + 1);  // a repeated key keeps its last value
        skip_ws();
        if (!eof() && peek() == ',') {
          ++pos_;
          continue;
        }
        expect('}');
        return v;
      }
    }
    if (c == '[') {
      v.kind_ = JsonValue::Kind::Array;
      ++pos_;
      skip_ws();
      if (!eof() && peek() == ']') {
        ++pos_;
        return v;
      }
      for (;;) {
        v.array_.push_back(value(depth + 1));
        skip_ws();
        if (!eof() && peek() == ',') {
          ++pos_;
          continue;
        }
        expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind_ = JsonValue::Kind::String;
      v.text_ = string_body();
      return v;
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      v.kind_ = JsonValue::Kind::Number;
      v.text_ = number_text();
      return v;
    }
    if (literal("true")) {
      v.kind_ = JsonValue::Kind::Bool;
      v.boolean_ = true;
      return v;
    }
    if (literal("false")) {
      v.kind_ = JsonValue::Kind::Bool;
      return v;
    }
    if (literal("null")) return v;
    parse_fail("unexpected character in JSON at byte " + std::to_string(pos_));
  }

  bool literal(const char* word) {
    const std::string w(word);
    if (s_.compare(pos_, w.size(), w) != 0) return false;
    pos_ += w.size();
    return true;
  }

  std::string number_text() {
    const size_t start = pos_;
    auto digits = [&]() {
      const size_t d0 = pos_;
      while (!eof() && peek() >= '0' && peek() <= '9') ++pos_;
      return pos_ - d0;
    };
    if (peek() == '-') ++pos_;
    if (eof()) parse_fail("truncated JSON number");
    if (peek() == '0') {
      ++pos_;
    } else if (digits() == 0) {
      parse_fail("invalid JSON number at byte " + std::to_string(start));
    }
    if (!eof() && peek() == '.') {
      ++pos_;
      if (digits() == 0) parse_fail("invalid JSON number fraction at byte " + std::to_string(start));
    }
    if (!eof() && (peek() == 'e' || peek() == 'E')) {
      ++pos_;
      if (!eof() && (peek() == '+' || peek() == '-')) ++pos_;
      if (digits() == 0) parse_fail("invalid JSON number exponent at byte " + std::to_string(start));
    }
    return s_.substr(start, pos_ - start);
  }

  uint32_t hex4() {
    if (pos_ + 4 > s_.size()) parse_fail("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char h = s_[pos_++];
      v <<= 4;
      if (h >= '0' && h <= '9') v |= static_cast<uint32_t>(h - '0');
      else if (h >= 'a' && h <= 'f') v |= static_cast<uint32_t>(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') v |= static_cast<uint32_t>(h - 'A' + 10);
      else parse_fail("invalid hex digit in \\u escape");
    }
    return v;
  }

  static void put_utf8(std::string* out, uint32_t cp) {
    if (cp < 0x80) {
      out->push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
      out->push_back(static_cast<char>(0xc0 | (cp >> 6)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3f)));
    } else if (cp < 0x10000) {
      out->push_back(static_cast<char>(0xe0 | (cp >> 12)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3f)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3f)));
    } else {
      out->push_back(static_cast<char>(0xf0 | (cp >> 18)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3f)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3f)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3f)));
    }
  }

  std::string string_body() {
    expect('"');
    std::string out;
    for (;;) {
      if (eof()) parse_fail("unterminated JSON string");
      const char c = s_[pos_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) parse_fail("control character in JSON string");
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (eof()) parse_fail("unterminated escape in JSON string");
      const char e = s_[pos_++];
      switch (e) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xd800 && cp <= 0xdbff) {
            if (pos_ + 2 > s_.size() || s_[pos_] != '\\' || s_[pos_ + 1] != 'u') parse_fail("unpaired UTF-16 surrogate");
            pos_ += 2;
            const uint32_t lo = hex4();
            if (lo < 0xdc00 || lo > 0xdfff) parse_fail("invalid UTF-16 surrogate pair");
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          } else if (cp >= 0xdc00 && cp <= 0xdfff) {
            parse_fail("unpaired UTF-16 surrogate");
          }
          put_utf8(&out, cp);
          break;
        }
        default:
          parse_fail(std::string("invalid escape '\\") + e + "' in JSON string");
      }
    }
  }
};

JsonValue JsonValue::parse(const std::string& text) { return JsonParser(text).document(); }

const std::map<std::string, JsonValue>& JsonValue::as_object() const {
  if (kind_ != Kind::Object) parse_fail("expected JSON object");
  return object_;
}

const std::vector<JsonValue>& JsonValue::as_array() const {
  if (kind_ != Kind::Array) parse_fail("expected JSON array");
  return array_;
}

const std::string& JsonValue::as_str() const {
  if (kind_ != Kind::String) parse_fail("expected JSON string");
  return text_;
}

bool JsonValue::as_bool() const {
  if (kind_ != Kind::Bool) parse_fail("expected JSON boolean");
  return boolean_;
}

uint64_t JsonValue::as_u64() const {
  if (kind_ != Kind::Number) parse_fail("expected JSON number");
  uint64_t v = 0;
  bool ok = !text_.empty();
  for (char c : text_) {
    if (c < '0' || c > '9') {
      ok = false;
      break;
    }
    const uint64_t d = static_cast<uint64_t>(c - '0');
    if (v > (UINT64_MAX - d) / 10) {
      ok = false;
      break;
    }
    v = v * 10 + d;
  }
  if (!ok) parse_fail("failed to parse JSON number '" + text_ + "' as u64");
  return v;
}

double JsonValue::as_f64() const {
  if (kind_ != Kind::Number) parse_fail("expected JSON number");
  char* end = nullptr;
  const double v = std::strtod(text_.c_str(), &end);
  if (end == nullptr || *end != '\0') parse_fail("failed to parse JSON number '" + text_ + "' as f64");
  return v;
}

const JsonValue& JsonValue::get(const std::string& key) const {
  const auto& obj = as_object();
  const auto it = obj.find(key);
  if (it == obj.end()) parse_fail("missing JSON key '" + key + "'");
  return it->second;
}

const JsonValue* JsonValue::find(const std::string& key) const {
  if (kind_ != Kind::Object) return nullptr;
  const auto it = object_.find(key);
  return it == object_.end() ? nullptr : &it->second;
}

}  // namespace fr
