// Minimal JSON reader for task-graph descriptions (objects, arrays, strings,
// numbers, true/false/null).  Throws std::runtime_error on malformed input.
#pragma once
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace yr {
namespace json {

struct Value {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  bool has(const std::string& k) const { return kind == Obj && obj.count(k) && obj.at(k).kind != Null; }
  const Value& operator[](const std::string& k) const {
    static const Value null;
    if (kind != Obj) throw std::runtime_error("json: not an object (key '" + k + "')");
    auto it = obj.find(k);
    return it == obj.end() ? null : it->second;
  }
  const Value& operator[](size_t i) const {
    if (kind != Arr || i >= arr.size()) throw std::runtime_error("json: bad array index");
    return arr[i];
  }
  size_t size() const { return kind == Arr ? arr.size() : kind == Obj ? obj.size() : 0; }
  int64_t i64(int64_t dflt = 0) const {
    if (kind == Num) return (int64_t)num;
    if (kind == Bool) return b ? 1 : 0;
    return dflt;
  }
  double f64(double dflt = 0) const { return kind == Num ? num : dflt; }
  const std::string& s() const {
    if (kind != Str) throw std::runtime_error("json: expected a string");
    return str;
  }
};

class Parser {
 public:
  explicit Parser(const char* p) : p_(p) {}
  Value parse() {
    Value v = value();
    ws();
    if (*p_) throw std::runtime_error("json: trailing characters");
    return v;
  }

 private:
  const char* p_;
  void ws() {
    while (*p_ == ' ' || *p_ == '\n' || *p_ == '\t' || *p_ == '\r') p_++;
  }
  Value value() {
    ws();
    Value v;
    switch (*p_) {
      case '{': {
        v.kind = Value::Obj;
        p_++;
        ws();
        if (*p_ == '}') { p_++; return v; }
        for (;;) {
          ws();
          std::string k = string();
          ws();
          if (*p_++ != ':') throw std::runtime_error("json: expected ':'");
          v.obj[k] = value();
          ws();
          if (*p_ == ',') { p_++; continue; }
          if (*p_ == '}') { p_++; return v; }
          throw std::runtime_error("json: expected ',' or '}'");
        }
      }
      case '[': {
        v.kind = Value::Arr;
        p_++;
        ws();
        if (*p_ == ']') { p_++; return v; }
        for (;;) {
          v.arr.push_back(value());
          ws();
          if (*p_ == ',') { p_++; continue; }
          if (*p_ == ']') { p_++; return v; }
          throw std::runtime_error("json: expected ',' or ']'");
        }
      }
      case '"':
        v.kind = Value::Str;
        v.str = string();
        return v;
      case 't':
        expect("true"); v.kind = Value::Bool; v.b = true; return v;
      case 'f':
        expect("false"); v.kind = Value::Bool; v.b = false; return v;
      case 'n':
        expect("null"); return v;
      default: {
        char* end = nullptr;
        v.num = strtod(p_, &end);
        if (end == p_) throw std::runtime_error(std::string("json: unexpected character '") + *p_ + "'");
        v.kind = Value::Num;
        p_ = end;
        return v;
      }
    }
  }
  void expect(const char* w) {
    for (; *w; w++, p_++)
      if (*p_ != *w) throw std::runtime_error("json: bad literal");
  }
  std::string string() {
    if (*p_ != '"') throw std::runtime_error("json: expected a string");
    p_++;
    std::string s;
    while (*p_ && *p_ != '"') {
      if (*p_ == '\\') {
        p_++;
        char c = *p_++;
        switch (c) {
          case 'n': s += '\n'; break;
          case 't': s += '\t'; break;
          case 'r': s += '\r'; break;
          case 'b': s += '\b'; break;
          case 'f': s += '\f'; break;
          case 'u': {  // basic multilingual plane, ASCII subset only
            unsigned cp = (unsigned)strtoul(std::string(p_, 4).c_str(), nullptr, 16);
            p_ += 4;
            s += cp < 128 ? (char)cp : '?';
            break;
          }
          default: s += c;
        }
      } else {
        s += *p_++;
      }
    }
    if (*p_ != '"') throw std::runtime_error("json: unterminated string");
    p_++;
    return s;
  }
};

inline Value parse(const char* text) { return Parser(text).parse(); }

}  // namespace json
}  // namespace yr
