// json.cpp -- strict RFC 8259 parser and canonical compact writer.
#include "json.hpp"

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstring>
#include <limits>

namespace pk::json {

std::optional<bool> Value::as_bool() const {
  if (kind_ != Kind::Bool) return std::nullopt;
  return b_;
}

std::optional<double> Value::as_number() const {
  if (kind_ != Kind::Number) return std::nullopt;
  return is_int_ ? static_cast<double>(i_) : d_;
}

std::optional<int64_t> Value::as_integer() const {
  if (kind_ != Kind::Number) return std::nullopt;
  if (is_int_) return i_;
  double ip = 0.0;
  if (!std::isfinite(d_) || std::modf(d_, &ip) != 0.0) return std::nullopt;
  // [-2^63, 2^63): both bounds are exact doubles
  if (ip < -9223372036854775808.0 || ip >= 9223372036854775808.0) return std::nullopt;
  return static_cast<int64_t>(ip);
}

const Value *Get(const Object &obj, std::string_view key) {
  for (const auto &kv : obj)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

namespace {

constexpr int kMaxDepth = 256;

class Parser {
 public:
  explicit Parser(std::string_view t) : t_(t) {}

  ParseResult Run() {
    ParseResult r;
    Value v;
    SkipWs();
    if (!ParseValue(v, 0)) {
      r.error = Where(err_);
      return r;
    }
    SkipWs();
    if (p_ != t_.size()) {
      r.error = Where("unexpected trailing characters after the document");
      return r;
    }
    r.value = std::move(v);
    return r;
  }

 private:
  std::string_view t_;
  size_t p_ = 0;
  std::string err_;

  bool Fail(const char *msg) {
    if (err_.empty()) err_ = msg;
    return false;
  }

  std::string Where(const std::string &msg) const {
    size_t line = 1, col = 1;
    for (size_t i = 0; i < p_ && i < t_.size(); ++i) {
      if (t_[i] == '\n') {
        ++line;
        col = 1;
      } else {
        ++col;
      }
    }
    return msg + " at line " + std::to_string(line) + " column " + std::to_string(col);
  }

  void SkipWs() {
    while (p_ < t_.size() && (t_[p_] == ' ' || t_[p_] == '\t' || t_[p_] == '\n' || t_[p_] == '\r')) ++p_;
  }

  bool Literal(const char *word) {
    const size_t n = std::strlen(word);
    if (t_.substr(p_, n) != word) return Fail("invalid literal");
    p_ += n;
    return true;
  }

  bool ParseValue(Value &out, int depth) {
    if (depth > kMaxDepth) return Fail("nesting too deep");
    if (p_ >= t_.size()) return Fail("unexpected end of input, expected a value");
    switch (t_[p_]) {
      case 'n':
        if (!Literal("null")) return false;
        out = Value();
        return true;
      case 't':
        if (!Literal("true")) return false;
        out = Value(true);
        return true;
      case 'f':
        if (!Literal("false")) return false;
        out = Value(false);
        return true;
      case '"': {
        std::string s;
        if (!ParseString(s)) return false;
        out = Value(std::move(s));
        return true;
      }
      case '[':
        return ParseArray(out, depth);
      case '{':
        return ParseObject(out, depth);
      default:
        if (t_[p_] == '-' || (t_[p_] >= '0' && t_[p_] <= '9')) return ParseNumber(out);
        return Fail("unexpected character, expected a value");
    }
  }

  bool Digits() {
    const size_t s = p_;
    while (p_ < t_.size() && t_[p_] >= '0' && t_[p_] <= '9') ++p_;
    return p_ > s;
  }

  bool ParseNumber(Value &out) {
    const size_t start = p_;
    bool is_int = true;
    if (t_[p_] == '-') ++p_;
    if (p_ >= t_.size()) return Fail("truncated number");
    if (t_[p_] == '0') {
      ++p_;
    } else if (!Digits()) {
      return Fail("invalid number");
    }
    if (p_ < t_.size() && t_[p_] == '.') {
      is_int = false;
      ++p_;
      if (!Digits()) return Fail("invalid number: digits expected after '.'");
    }
    if (p_ < t_.size() && (t_[p_] == 'e' || t_[p_] == 'E')) {
      is_int = false;
      ++p_;
      if (p_ < t_.size() && (t_[p_] == '+' || t_[p_] == '-')) ++p_;
      if (!Digits()) return Fail("invalid number: digits expected in the exponent");
    }
    const char *b = t_.data() + start, *e = t_.data() + p_;
    if (is_int) {
      long long v = 0;
      auto [ptr, ec] = std::from_chars(b, e, v);
      if (ec == std::errc() && ptr == e) {
        out = Value(v);
        return true;
      }
      // out of int64 range: keep it as a double
    }
    double d = 0.0;
    auto [ptr, ec] = std::from_chars(b, e, d);
    if (ptr != e || (ec != std::errc() && ec != std::errc::result_out_of_range))
      return Fail("invalid number");
    if (!std::isfinite(d)) return Fail("number out of range");
    out = Value(d);
    return true;
  }

  static void PutUtf8(std::string &s, uint32_t cp) {
    if (cp < 0x80) {
      s.push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
      s.push_back(static_cast<char>(0xC0 | (cp >> 6)));
      s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      s.push_back(static_cast<char>(0xE0 | (cp >> 12)));
      s.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
      s.push_back(static_cast<char>(0xF0 | (cp >> 18)));
      s.push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
      s.push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      s.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
  }

  bool Hex4(uint32_t &v) {
    if (p_ + 4 > t_.size()) return Fail("truncated \\u escape");
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = t_[p_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
      else return Fail("invalid hex digit in \\u escape");
    }
    return true;
  }

  // One UTF-8 encoded code point starting at p_ (first byte >= 0x80).
  bool Utf8(std::string &s) {
    const auto byte = [&](size_t i) { return static_cast<unsigned char>(t_[i]); };
    const unsigned char c0 = byte(p_);
    int n = 0;
    uint32_t cp = 0, lo = 0;
    if (c0 >= 0xC2 && c0 <= 0xDF) { n = 1; cp = c0 & 0x1F; lo = 0x80; }
    else if (c0 >= 0xE0 && c0 <= 0xEF) { n = 2; cp = c0 & 0x0F; lo = 0x800; }
    else if (c0 >= 0xF0 && c0 <= 0xF4) { n = 3; cp = c0 & 0x07; lo = 0x10000; }
    else return Fail("invalid UTF-8 in string");
    if (p_ + n >= t_.size()) return Fail("truncated UTF-8 sequence");
    for (int i = 1; i <= n; ++i) {
      const unsigned char c = byte(p_ + i);
      if ((c & 0xC0) != 0x80) return Fail("invalid UTF-8 in string");
      cp = (cp << 6) | (c & 0x3F);
    }
    if (cp < lo || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return Fail("invalid UTF-8 in string");
    s.append(t_.substr(p_, n + 1));
    p_ += n + 1;
    return true;
  }

  bool ParseString(std::string &s) {
    ++p_;  // opening quote
    for (;;) {
      if (p_ >= t_.size()) return Fail("unterminated string");
      const unsigned char c = static_cast<unsigned char>(t_[p_]);
      if (c == '"') {
        ++p_;
        return true;
      }
      if (c < 0x20) return Fail("control character in string");
      if (c >= 0x80) {
        if (!Utf8(s)) return false;
        continue;
      }
      if (c != '\\') {
        s.push_back(static_cast<char>(c));
        ++p_;
        continue;
      }
      ++p_;
      if (p_ >= t_.size()) return Fail("unterminated escape");
      const char e = t_[p_++];
      switch (e) {
        case '"': s.push_back('"'); break;
        case '\\': s.push_back('\\'); break;
        case '/': s.push_back('/'); break;
        case 'b': s.push_back('\b'); break;
        case 'f': s.push_back('\f'); break;
        case 'n': s.push_back('\n'); break;
        case 'r': s.push_back('\r'); break;
        case 't': s.push_back('\t'); break;
        case 'u': {
          uint32_t cp = 0;
          if (!Hex4(cp)) return false;
          if (cp >= 0xD800 && cp <= 0xDBFF) {
            uint32_t lo = 0;
            if (t_.substr(p_, 2) != "\\u") return Fail("unpaired surrogate in \\u escape");
            p_ += 2;
            if (!Hex4(lo)) return false;
            if (lo < 0xDC00 || lo > 0xDFFF) return Fail("unpaired surrogate in \\u escape");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
            return Fail("unpaired surrogate in \\u escape");
          }
          PutUtf8(s, cp);
          break;
        }
        default:
          return Fail("invalid escape in string");
      }
    }
  }

  bool ParseArray(Value &out, int depth) {
    ++p_;
    Array arr;
    SkipWs();
    if (p_ < t_.size() && t_[p_] == ']') {
      ++p_;
      out = Value(std::move(arr));
      return true;
    }
    for (;;) {
      SkipWs();
      Value v;
      if (!ParseValue(v, depth + 1)) return false;
      arr.push_back(std::move(v));
      SkipWs();
      if (p_ >= t_.size()) return Fail("unterminated array");
      if (t_[p_] == ',') {
        ++p_;
        continue;
      }
      if (t_[p_] == ']') {
        ++p_;
        out = Value(std::move(arr));
        return true;
      }
      return Fail("expected ',' or ']' after an array element");
    }
  }

  bool ParseObject(Value &out, int depth) {
    ++p_;
    Object obj;
    SkipWs();
    if (p_ < t_.size() && t_[p_] == '}') {
      ++p_;
      out = Value(std::move(obj));
      return true;
    }
    for (;;) {
      SkipWs();
      if (p_ >= t_.size() || t_[p_] != '"') return Fail("expected a string key");
      std::string key;
      if (!ParseString(key)) return false;
      if (Get(obj, key) != nullptr) return Fail("duplicate object key");
      SkipWs();
      if (p_ >= t_.size() || t_[p_] != ':') return Fail("expected ':' after an object key");
      ++p_;
      SkipWs();
      Value v;
      if (!ParseValue(v, depth + 1)) return false;
      obj.emplace_back(std::move(key), std::move(v));
      SkipWs();
      if (p_ >= t_.size()) return Fail("unterminated object");
      if (t_[p_] == ',') {
        ++p_;
        continue;
      }
      if (t_[p_] == '}') {
        ++p_;
        out = Value(std::move(obj));
        return true;
      }
      return Fail("expected ',' or '}' after an object member");
    }
  }
};

void WriteString(std::string &out, const std::string &s) {
  static const char kHex[] = "0123456789abcdef";
  out.push_back('"');
  for (const char ch : s) {
    const unsigned char c = static_cast<unsigned char>(ch);
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (c < 0x20) {
          out += "\\u00";
          out.push_back(kHex[c >> 4]);
          out.push_back(kHex[c & 15]);
        } else {
          out.push_back(ch);
        }
    }
  }
  out.push_back('"');
}

void Write(std::string &out, const Value &v) {
  switch (v.kind()) {
    case Value::Kind::Null:
      out += "null";
      return;
    case Value::Kind::Bool:
      out += *v.as_bool() ? "true" : "false";
      return;
    case Value::Kind::Number: {
      char buf[64];
      std::to_chars_result r;
      const auto i = v.as_integer();
      const double d = *v.as_number();
      if (i && static_cast<double>(*i) == d && std::fabs(d) < 9007199254740992.0) {
        r = std::to_chars(buf, buf + sizeof buf, static_cast<long long>(*i));
      } else if (!std::isfinite(d)) {
        out += "null";
        return;
      } else {
        r = std::to_chars(buf, buf + sizeof buf, d);  // shortest round-trip form
      }
      out.append(buf, r.ptr);
      return;
    }
    case Value::Kind::String:
      WriteString(out, *v.as_string());
      return;
    case Value::Kind::Array: {
      out.push_back('[');
      bool first = true;
      for (const Value &e : *v.as_array()) {
        if (!first) out.push_back(',');
        first = false;
        Write(out, e);
      }
      out.push_back(']');
      return;
    }
    case Value::Kind::Object: {
      std::vector<const std::pair<std::string, Value> *> members;
      for (const auto &kv : *v.as_object()) members.push_back(&kv);
      std::sort(members.begin(), members.end(), [](auto *a, auto *b) { return a->first < b->first; });
      out.push_back('{');
      bool first = true;
      for (const auto *kv : members) {
        if (!first) out.push_back(',');
        first = false;
        WriteString(out, kv->first);
        out.push_back(':');
        Write(out, kv->second);
      }
      out.push_back('}');
      return;
    }
  }
}

}  // namespace

ParseResult Parse(std::string_view text) { return Parser(text).Run(); }

std::string Serialize(const Value &v) {
  std::string out;
  Write(out, v);
  return out;
}

}  // namespace pk::json
