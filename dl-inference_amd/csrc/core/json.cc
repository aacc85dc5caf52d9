#include "json.h"

#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <stdexcept>

namespace dli::json {
namespace {

class Reader {
 public:
  explicit Reader(std::string_view text) : text_(text) {}

  Value document() {
    Value v = value(0);
    skipSpace();
    if (pos_ != text_.size()) fail("unexpected trailing JSON content");
    return v;
  }

 private:
  [[noreturn]] void fail(const std::string& what) const {
    throw std::invalid_argument(what + " at offset " + std::to_string(pos_));
  }

  void skipSpace() {
    while (pos_ < text_.size() && std::isspace(static_cast<unsigned char>(text_[pos_]))) ++pos_;
  }

  char peek() const { return pos_ < text_.size() ? text_[pos_] : '\0'; }

  void expect(char c) {
    skipSpace();
    if (peek() != c) fail(std::string("expected JSON token: ") + c);
    ++pos_;
  }

  bool accept(char c) {
    skipSpace();
    if (peek() != c) return false;
    ++pos_;
    return true;
  }

  bool acceptWord(std::string_view word) {
    if (text_.substr(pos_, word.size()) != word) return false;
    pos_ += word.size();
    return true;
  }

  Value value(int depth) {
    if (depth > 256) fail("JSON nesting too deep");
    skipSpace();
    if (pos_ >= text_.size()) fail("unexpected end of JSON");
    Value v;
    const char c = peek();
    if (c == '{') {
      ++pos_;
      v.kind = Value::Kind::Object;
      if (accept('}')) return v;
      do {
        skipSpace();
        if (peek() != '"') fail("JSON object key must be a string");
        std::string key = string();
        expect(':');
        v.fields.insert_or_assign(std::move(key), value(depth + 1));
      } while (accept(','));
      expect('}');
    } else if (c == '[') {
      ++pos_;
      v.kind = Value::Kind::Array;
      if (accept(']')) return v;
      do {
        v.items.push_back(value(depth + 1));
      } while (accept(','));
      expect(']');
    } else if (c == '"') {
      v.kind = Value::Kind::String;
      v.s = string();
    } else if (acceptWord("true")) {
      v.kind = Value::Kind::Bool;
      v.b = true;
    } else if (acceptWord("false")) {
      v.kind = Value::Kind::Bool;
      v.b = false;
    } else if (acceptWord("null")) {
      v.kind = Value::Kind::Null;
    } else if (c == '-' || std::isdigit(static_cast<unsigned char>(c))) {
      number(v);
    } else {
      fail("unexpected JSON token");
    }
    return v;
  }

  void digits() {
    const std::size_t start = pos_;
    while (pos_ < text_.size() && std::isdigit(static_cast<unsigned char>(text_[pos_]))) ++pos_;
    if (pos_ == start) fail("expected JSON digit");
  }

  void number(Value& v) {
    const std::size_t start = pos_;
    bool integral = true;
    if (peek() == '-') ++pos_;
    digits();
    if (peek() == '.') {
      ++pos_;
      digits();
      integral = false;
    }
    if (peek() == 'e' || peek() == 'E') {
      ++pos_;
      if (peek() == '+' || peek() == '-') ++pos_;
      digits();
      integral = false;
    }
    const std::string token(text_.substr(start, pos_ - start));
    errno = 0;
    if (integral) {
      v.kind = Value::Kind::Int;
      v.i = std::strtoll(token.c_str(), nullptr, 10);
      if (errno == ERANGE) fail("JSON integer out of range");
    } else {
      v.kind = Value::Kind::Double;
      v.d = std::strtod(token.c_str(), nullptr);
    }
  }

  static void appendUtf8(std::string& out, unsigned code) {
    if (code < 0x80) {
      out.push_back(static_cast<char>(code));
    } else if (code < 0x800) {
      out.push_back(static_cast<char>(0xC0 | (code >> 6)));
      out.push_back(static_cast<char>(0x80 | (code & 0x3F)));
    } else if (code < 0x10000) {
      out.push_back(static_cast<char>(0xE0 | (code >> 12)));
      out.push_back(static_cast<char>(0x80 | ((code >> 6) & 0x3F)));
      out.push_back(static_cast<char>(0x80 | (code & 0x3F)));
    } else {
      out.push_back(static_cast<char>(0xF0 | (code >> 18)));
      out.push_back(static_cast<char>(0x80 | ((code >> 12) & 0x3F)));
      out.push_back(static_cast<char>(0x80 | ((code >> 6) & 0x3F)));
      out.push_back(static_cast<char>(0x80 | (code & 0x3F)));
    }
  }

  unsigned hex4() {
    if (pos_ + 4 > text_.size()) fail("truncated JSON \\u escape");
    unsigned code = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = text_[pos_++];
      code <<= 4;
      if (h >= '0' && h <= '9') code |= static_cast<unsigned>(h - '0');
      else if (h >= 'a' && h <= 'f') code |= static_cast<unsigned>(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') code |= static_cast<unsigned>(h - 'A' + 10);
      else fail("invalid JSON \\u escape");
    }
    return code;
  }

  std::string string() {
    ++pos_;  // opening quote
    std::string out;
    while (true) {
      if (pos_ >= text_.size()) fail("unterminated JSON string");
      const char c = text_[pos_++];
      if (c == '"') return out;
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (pos_ >= text_.size()) fail("unterminated JSON escape");
      const char e = text_[pos_++];
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
          unsigned code = hex4();
          if (code >= 0xD800 && code < 0xDC00 && text_.substr(pos_, 2) == "\\u") {
            pos_ += 2;
            const unsigned low = hex4();
            code = 0x10000 + ((code - 0xD800) << 10) + (low - 0xDC00);
          }
          appendUtf8(out, code);
          break;
        }
        default: fail("unsupported JSON string escape");
      }
    }
  }

  std::string_view text_;
  std::size_t pos_ = 0;
};

}  // namespace

const Value* Value::find(const std::string& key) const {
  if (kind != Kind::Object) throw std::invalid_argument("expected JSON object");
  auto it = fields.find(key);
  return it == fields.end() ? nullptr : &it->second;
}

const Value& Value::at(const std::string& key) const {
  const Value* v = find(key);
  if (v == nullptr) throw std::invalid_argument("missing JSON field: " + key);
  return *v;
}

Value parse(std::string_view text) { return Reader(text).document(); }

std::string quote(std::string_view text) {
  std::string out = "\"";
  for (const char c : text) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      default:
        if (static_cast<unsigned char>(c) < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", static_cast<unsigned>(c));
          out += buf;
        } else {
          out.push_back(c);
        }
    }
  }
  out.push_back('"');
  return out;
}

std::string formatDouble(double value) {
  if (!std::isfinite(value)) throw std::invalid_argument("non-finite double cannot be written as JSON");
  char buf[40];
  for (int precision = 15; precision <= 17; ++precision) {
    std::snprintf(buf, sizeof(buf), "%.*g", precision, value);
    if (std::strtod(buf, nullptr) == value) break;
  }
  std::string text(buf);
  if (text.find_first_of(".eEn") == std::string::npos) text += ".0";
  return text;
}

std::string readFile(const std::string& path, const char* what) {
  std::ifstream file(path, std::ios::binary);
  if (!file) throw std::runtime_error(std::string("failed to open ") + what + ": " + path);
  std::ostringstream buffer;
  buffer << file.rdbuf();
  return buffer.str();
}

}  // namespace dli::json
