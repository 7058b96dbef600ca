#include "json.h"

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>

namespace malkin_hip::json {

namespace {

const Value kNull;

class Parser {
 public:
  explicit Parser(std::string_view t) : t_(t) {}

  Value document() {
    Value v = value(0);
    space();
    if (p_ != t_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* what) const {
    throw ParseError(std::string(what) + " at offset " + std::to_string(p_));
  }
  void space() {
    while (p_ < t_.size() && (t_[p_] == ' ' || t_[p_] == '\t' || t_[p_] == '\n' || t_[p_] == '\r')) ++p_;
  }
  char peek() {
    space();
    if (p_ >= t_.size()) fail("unexpected end");
    return t_[p_];
  }
  void expect(char c) {
    if (peek() != c) fail("unexpected character");
    ++p_;
  }
  bool literal(std::string_view w) {
    if (t_.substr(p_, w.size()) != w) return false;
    p_ += w.size();
    return true;
  }

  Value value(int depth) {
    if (depth > 256) fail("nesting too deep");
    const char c = peek();
    if (c == '{') return object(depth);
    if (c == '[') return array(depth);
    if (c == '"') return Value(string());
    if (literal("true")) return Value(true);
    if (literal("false")) return Value(false);
    if (literal("null")) return Value();
    if (c == '-' || (c >= '0' && c <= '9')) return number();
    fail("unexpected character");
  }

  Value object(int depth) {
    expect('{');
    Value o = Value::object();
    if (peek() == '}') {
      ++p_;
      return o;
    }
    for (;;) {
      if (peek() != '"') fail("expected a key");
      std::string k = string();
      expect(':');
      o.set(k, value(depth + 1));
      const char c = peek();
      ++p_;
      if (c == '}') return o;
      if (c != ',') fail("expected , or }");
    }
  }

  Value array(int depth) {
    expect('[');
    Value a = Value::array();
    if (peek() == ']') {
      ++p_;
      return a;
    }
    for (;;) {
      a.push(value(depth + 1));
      const char c = peek();
      ++p_;
      if (c == ']') return a;
      if (c != ',') fail("expected , or ]");
    }
  }

  unsigned hex4() {
    if (p_ + 4 > t_.size()) fail("short \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = t_[p_++];
      v <<= 4;
      if (c >= '0' && c <= '9')
        v |= static_cast<unsigned>(c - '0');
      else if (c >= 'a' && c <= 'f')
        v |= static_cast<unsigned>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F')
        v |= static_cast<unsigned>(c - 'A' + 10);
      else
        fail("bad \\u escape");
    }
    return v;
  }

  static void utf8(std::string& out, unsigned cp) {
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

  std::string string() {
    expect('"');
    std::string out;
    for (;;) {
      if (p_ >= t_.size()) fail("unterminated string");
      const char c = t_[p_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p_ >= t_.size()) fail("unterminated escape");
      const char e = t_[p_++];
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
          unsigned cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
            if (!literal("\\u")) fail("lone surrogate");
            const unsigned lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            fail("lone surrogate");
          }
          utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }

  Value number() {
    const size_t start = p_;
    bool integral = true;
    if (t_[p_] == '-') ++p_;
    auto digits = [&] {
      const size_t s = p_;
      while (p_ < t_.size() && t_[p_] >= '0' && t_[p_] <= '9') ++p_;
      if (p_ == s) fail("bad number");
    };
    if (p_ < t_.size() && t_[p_] == '0')
      ++p_;
    else
      digits();
    if (p_ < t_.size() && t_[p_] == '.') {
      integral = false;
      ++p_;
      digits();
    }
    if (p_ < t_.size() && (t_[p_] == 'e' || t_[p_] == 'E')) {
      integral = false;
      ++p_;
      if (p_ < t_.size() && (t_[p_] == '+' || t_[p_] == '-')) ++p_;
      digits();
    }
    const std::string lit(t_.substr(start, p_ - start));
    if (integral) {
      errno = 0;
      if (lit[0] == '-') {
        const long long v = std::strtoll(lit.c_str(), nullptr, 10);
        if (errno == 0) return Value(static_cast<int64_t>(v));
      } else {
        const unsigned long long v = std::strtoull(lit.c_str(), nullptr, 10);
        if (errno == 0) return v <= INT64_MAX ? Value(static_cast<int64_t>(v)) : Value(static_cast<uint64_t>(v));
      }
    }
    return Value(std::strtod(lit.c_str(), nullptr));
  }

  std::string_view t_;
  size_t p_ = 0;
};

void escape(std::string& out, const std::string& s) {
  out += '"';
  for (const char ch : s) {
    const auto c = static_cast<unsigned char>(ch);
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof buf, "\\u%04x", c);
          out += buf;
        } else {
          out += ch;
        }
    }
  }
  out += '"';
}

}  // namespace

Value Value::array(std::vector<Value> items) {
  Value v;
  v.kind_ = Kind::Array;
  v.a_ = std::move(items);
  return v;
}

Value Value::object(std::initializer_list<std::pair<const std::string, Value>> items) {
  Value v;
  v.kind_ = Kind::Object;
  for (const auto& [k, x] : items) v.set(k, x);
  return v;
}

Value Value::parse(std::string_view text) { return Parser(text).document(); }

bool Value::as_bool() const {
  if (kind_ != Kind::Bool) throw std::invalid_argument("expected a boolean");
  return b_;
}

double Value::as_double() const {
  switch (kind_) {
    case Kind::Int: return static_cast<double>(i_);
    case Kind::Uint: return static_cast<double>(u_);
    case Kind::Double: return d_;
    default: throw std::invalid_argument("expected a number");
  }
}

int64_t Value::as_int() const {
  if (kind_ == Kind::Int) return i_;
  if (kind_ == Kind::Double && std::floor(d_) == d_ && std::fabs(d_) < 9.0e15) return static_cast<int64_t>(d_);
  throw std::invalid_argument(kind_ == Kind::Uint ? "integer out of range" : "expected an integer");
}

uint64_t Value::as_uint() const {
  if (kind_ == Kind::Uint) return u_;
  if (kind_ == Kind::Int && i_ >= 0) return static_cast<uint64_t>(i_);
  throw std::invalid_argument("expected a non-negative integer");
}

const std::string& Value::as_string() const {
  if (kind_ != Kind::String) throw std::invalid_argument("expected a string");
  return s_;
}

const std::vector<Value>& Value::items() const {
  if (kind_ != Kind::Array) throw std::invalid_argument("expected an array");
  return a_;
}

bool Value::has(const std::string& key) const {
  if (kind_ != Kind::Object) return false;
  for (const auto& [k, v] : o_)
    if (k == key) return true;
  return false;
}

const Value& Value::operator[](const std::string& key) const {
  if (kind_ == Kind::Object)
    for (const auto& [k, v] : o_)
      if (k == key) return v;
  return kNull;
}

Value& Value::set(const std::string& key, Value v) {
  if (kind_ != Kind::Object) throw std::invalid_argument("set on a non-object");
  for (auto& [k, x] : o_)
    if (k == key) return x = std::move(v);
  o_.emplace_back(key, std::move(v));
  return o_.back().second;
}

Value& Value::push(Value v) {
  if (kind_ != Kind::Array) throw std::invalid_argument("push on a non-array");
  a_.push_back(std::move(v));
  return a_.back();
}

std::string Value::dump() const {
  std::string out;
  dump_to(out);
  return out;
}

void Value::dump_to(std::string& out) const {
  switch (kind_) {
    case Kind::Null: out += "null"; break;
    case Kind::Bool: out += b_ ? "true" : "false"; break;
    case Kind::Int: out += std::to_string(i_); break;
    case Kind::Uint: out += std::to_string(u_); break;
    case Kind::Double: {
      if (!std::isfinite(d_)) {
        out += "null";
        break;
      }
      char buf[32];
      std::snprintf(buf, sizeof buf, "%.17g", d_);
      out += buf;
      break;
    }
    case Kind::String: escape(out, s_); break;
    case Kind::Array: {
      out += '[';
      for (size_t i = 0; i < a_.size(); ++i) {
        if (i) out += ',';
        a_[i].dump_to(out);
      }
      out += ']';
      break;
    }
    case Kind::Object: {
      out += '{';
      for (size_t i = 0; i < o_.size(); ++i) {
        if (i) out += ',';
        escape(out, o_[i].first);
        out += ':';
        o_[i].second.dump_to(out);
      }
      out += '}';
      break;
    }
  }
}

}  // namespace malkin_hip::json
