// json_lite.hpp -- a small JSON reader for the checkpoint's text files: the
// safetensors header, model.safetensors.index.json and config.json.  It
// builds a tree of values; numbers keep their text, so 64-bit offsets are read
// exactly.  Not a general-purpose library: no writer, no streaming.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

namespace qah {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // String: the decoded string; Number: the literal
  std::vector<Value> items;                           // Array
  std::vector<std::pair<std::string, Value>> fields;  // Object, in file order

  const Value* get(const std::string& key) const {
    if (kind != Object) return nullptr;
    for (const auto& f : fields)
      if (f.first == key) return &f.second;
    return nullptr;
  }
  bool is_int() const {
    if (kind != Number) return false;
    for (char c : text)
      if (c == '.' || c == 'e' || c == 'E') return false;
    return true;
  }
  int64_t as_int() const { return std::strtoll(text.c_str(), nullptr, 10); }
  uint64_t as_uint() const { return std::strtoull(text.c_str(), nullptr, 10); }
  double as_double() const { return std::strtod(text.c_str(), nullptr); }
};

class Parser {
 public:
  Parser(const char* p, size_t n) : p_(p), end_(p + n) {}
  // Parses one value followed only by whitespace; returns false (with
  // error() set) on malformed input.
  bool parse(Value* out) {
    if (!value(out, 0)) return false;
    ws();
    if (p_ != end_) return fail("trailing characters");
    return true;
  }
  const std::string& error() const { return err_; }

 private:
  const char* p_;
  const char* end_;
  std::string err_;

  bool fail(const char* what) {
    if (err_.empty()) err_ = what;
    return false;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    for (; *s; ++s, ++p_)
      if (p_ >= end_ || *p_ != *s) return fail("bad literal");
    return true;
  }
  static void utf8(uint32_t cp, std::string* s) {
    if (cp < 0x80) {
      s->push_back((char)cp);
    } else if (cp < 0x800) {
      s->push_back((char)(0xC0 | (cp >> 6)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      s->push_back((char)(0xE0 | (cp >> 12)));
      s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    } else {
      s->push_back((char)(0xF0 | (cp >> 18)));
      s->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
      s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    }
  }
  bool hex4(uint32_t* v) {
    if (end_ - p_ < 4) return fail("short \\u escape");
    *v = 0;
    for (int i = 0; i < 4; ++i, ++p_) {
      const char c = *p_;
      *v <<= 4;
      if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool string(std::string* s) {
    ++p_;  // opening quote
    while (true) {
      if (p_ >= end_) return fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return fail("control character in string");
      if (c != '\\') {
        s->push_back(c);
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s->push_back('"'); break;
        case '\\': s->push_back('\\'); break;
        case '/': s->push_back('/'); break;
        case 'b': s->push_back('\b'); break;
        case 'f': s->push_back('\f'); break;
        case 'n': s->push_back('\n'); break;
        case 'r': s->push_back('\r'); break;
        case 't': s->push_back('\t'); break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // a surrogate pair
            uint32_t lo;
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
            p_ += 2;
            if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(cp, s);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }
  bool number(Value* v) {
    const char* b = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                         *p_ == '+' || *p_ == '-'))
      ++p_;
    if (p_ == b) return fail("bad number");
    v->kind = Value::Number;
    v->text.assign(b, p_);
    return true;
  }
  bool value(Value* v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p_ >= end_) return fail("unexpected end");
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v->kind = Value::Object;
      ws();
      if (p_ < end_ && *p_ == '}') return ++p_, true;
      while (true) {
        ws();
        if (p_ >= end_ || *p_ != '"') return fail("expected a key");
        std::string key;
        if (!string(&key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
        ++p_;
        v->fields.emplace_back(std::move(key), Value{});
        if (!value(&v->fields.back().second, depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') { ++p_; continue; }
        if (p_ < end_ && *p_ == '}') return ++p_, true;
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      v->kind = Value::Array;
      ws();
      if (p_ < end_ && *p_ == ']') return ++p_, true;
      while (true) {
        v->items.emplace_back();
        if (!value(&v->items.back(), depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') { ++p_; continue; }
        if (p_ < end_ && *p_ == ']') return ++p_, true;
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v->kind = Value::String;
      return string(&v->text);
    }
    if (c == 't') { v->kind = Value::Bool; v->b = true; return lit("true"); }
    if (c == 'f') { v->kind = Value::Bool; v->b = false; return lit("false"); }
    if (c == 'n') { v->kind = Value::Null; return lit("null"); }
    return number(v);
  }
};

}  // namespace json
}  // namespace qah
