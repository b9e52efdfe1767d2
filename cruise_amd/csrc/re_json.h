// Minimal JSON reader for the engine's graph_config (objects, arrays,
// numbers, strings, booleans, null).  Enough for configuration files; not a
// general-purpose parser.
#pragma once

#include <cctype>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace re {

struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::map<std::string, Json> obj;

  const Json* get(const std::string& key) const {
    if (kind != kObject) return nullptr;
    auto it = obj.find(key);
    return it == obj.end() ? nullptr : &it->second;
  }
  double number_or(const std::string& key, double fallback) const {
    const Json* v = get(key);
    return (v && v->kind == kNumber) ? v->num : fallback;
  }
  std::string string_or(const std::string& key, const std::string& fallback) const {
    const Json* v = get(key);
    return (v && v->kind == kString) ? v->str : fallback;
  }
  bool bool_or(const std::string& key, bool fallback) const {
    const Json* v = get(key);
    return (v && v->kind == kBool) ? v->b : fallback;
  }
};

class JsonParser {
 public:
  explicit JsonParser(const std::string& text) : s_(text) {}
  bool parse(Json& out) {
    pos_ = 0;
    if (!value(out)) return false;
    ws();
    return pos_ == s_.size();
  }

 private:
  const std::string& s_;
  size_t pos_ = 0;

  void ws() {
    while (pos_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[pos_]))) ++pos_;
  }
  bool lit(const char* word) {
    size_t n = std::char_traits<char>::length(word);
    if (s_.compare(pos_, n, word) != 0) return false;
    pos_ += n;
    return true;
  }
  bool string(std::string& out) {
    if (pos_ >= s_.size() || s_[pos_] != '"') return false;
    ++pos_;
    out.clear();
    while (pos_ < s_.size() && s_[pos_] != '"') {
      char c = s_[pos_++];
      if (c == '\\') {
        if (pos_ >= s_.size()) return false;
        char e = s_[pos_++];
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u':
            if (pos_ + 4 > s_.size()) return false;
            out += '?';
            pos_ += 4;
            break;
          default: out += e;
        }
      } else {
        out += c;
      }
    }
    if (pos_ >= s_.size()) return false;
    ++pos_;
    return true;
  }
  bool value(Json& v) {
    ws();
    if (pos_ >= s_.size()) return false;
    char c = s_[pos_];
    if (c == '{') {
      ++pos_;
      v.kind = Json::kObject;
      ws();
      if (pos_ < s_.size() && s_[pos_] == '}') { ++pos_; return true; }
      while (true) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (pos_ >= s_.size() || s_[pos_] != ':') return false;
        ++pos_;
        Json child;
        if (!value(child)) return false;
        v.obj[key] = std::move(child);
        ws();
        if (pos_ < s_.size() && s_[pos_] == ',') { ++pos_; continue; }
        if (pos_ < s_.size() && s_[pos_] == '}') { ++pos_; return true; }
        return false;
      }
    }
    if (c == '[') {
      ++pos_;
      v.kind = Json::kArray;
      ws();
      if (pos_ < s_.size() && s_[pos_] == ']') { ++pos_; return true; }
      while (true) {
        Json child;
        if (!value(child)) return false;
        v.arr.push_back(std::move(child));
        ws();
        if (pos_ < s_.size() && s_[pos_] == ',') { ++pos_; continue; }
        if (pos_ < s_.size() && s_[pos_] == ']') { ++pos_; return true; }
        return false;
      }
    }
    if (c == '"') {
      v.kind = Json::kString;
      return string(v.str);
    }
    if (lit("true")) { v.kind = Json::kBool; v.b = true; return true; }
    if (lit("false")) { v.kind = Json::kBool; v.b = false; return true; }
    if (lit("null")) { v.kind = Json::kNull; return true; }
    const char* begin = s_.c_str() + pos_;
    char* end = nullptr;
    double d = std::strtod(begin, &end);
    if (end == begin) return false;
    pos_ += static_cast<size_t>(end - begin);
    v.kind = Json::kNumber;
    v.num = d;
    return true;
  }
};

}  // namespace re
