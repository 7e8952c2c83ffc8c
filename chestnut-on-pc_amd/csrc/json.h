// Minimal JSON reader for model specs (objects, arrays, numbers, strings,
// true/false/null).  Specs are small flat objects; this is not a general
// purpose parser and rejects anything it does not understand.
#pragma once

#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace ck {

struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  double num = 0;
  bool b = false;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;

  const JVal* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  explicit JParser(const std::string& s) : s_(s) {}
  JVal parse() {
    JVal v = value();
    ws();
    CK_REQUIRE(i_ == s_.size(), "spec json: trailing characters");
    return v;
  }

 private:
  const std::string& s_;
  size_t i_ = 0;

  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\t' || s_[i_] == '\r')) ++i_;
  }
  char peek() {
    ws();
    CK_REQUIRE(i_ < s_.size(), "spec json: unexpected end");
    return s_[i_];
  }
  void expect(char c) {
    CK_REQUIRE(peek() == c, std::string("spec json: expected '") + c + "'");
    ++i_;
  }
  std::string string_lit() {
    expect('"');
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      if (s_[i_] == '\\') {
        ++i_;
        CK_REQUIRE(i_ < s_.size(), "spec json: bad escape");
      }
      out.push_back(s_[i_++]);
    }
    CK_REQUIRE(i_ < s_.size(), "spec json: unterminated string");
    ++i_;
    return out;
  }
  JVal value() {
    JVal v;
    const char c = peek();
    if (c == '{') {
      v.kind = JVal::OBJ;
      ++i_;
      if (peek() == '}') { ++i_; return v; }
      while (true) {
        std::string k = string_lit();
        expect(':');
        v.obj.emplace_back(k, value());
        if (peek() == ',') { ++i_; continue; }
        expect('}');
        return v;
      }
    }
    if (c == '[') {
      v.kind = JVal::ARR;
      ++i_;
      if (peek() == ']') { ++i_; return v; }
      while (true) {
        v.arr.push_back(value());
        if (peek() == ',') { ++i_; continue; }
        expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = JVal::STR;
      v.str = string_lit();
      return v;
    }
    if (s_.compare(i_, 4, "true") == 0) { i_ += 4; v.kind = JVal::BOOL; v.b = true; return v; }
    if (s_.compare(i_, 5, "false") == 0) { i_ += 5; v.kind = JVal::BOOL; return v; }
    if (s_.compare(i_, 4, "null") == 0) { i_ += 4; return v; }
    const char* st = s_.c_str() + i_;
    char* end = nullptr;
    v.num = std::strtod(st, &end);
    CK_REQUIRE(end != st, "spec json: bad value");
    v.kind = JVal::NUM;
    i_ += (size_t)(end - st);
    return v;
  }
};

}  // namespace ck
