// A small JSON reader for the test fixtures under tests/golden/ (numbers,
// strings without escapes beyond \" \\ \/ \n \t, arrays, objects, true,
// false, null).  Objects keep their keys in file order.
#pragma once

#include <cctype>
#include <cstdlib>
#include <fstream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace json_lite {

struct Value {
  enum class Kind { kNull, kBool, kNumber, kString, kArray, kObject };
  Kind kind = Kind::kNull;
  bool boolean = false;
  double number = 0.0;
  std::string text;
  std::vector<Value> items;                            // array
  std::vector<std::pair<std::string, Value>> members;  // object

  [[nodiscard]] bool has(const std::string& key) const {
    for (const auto& m : members)
      if (m.first == key) return true;
    return false;
  }
  [[nodiscard]] const Value& operator[](const std::string& key) const {
    for (const auto& m : members)
      if (m.first == key) return m.second;
    throw std::out_of_range("json: no member '" + key + "'");
  }
  [[nodiscard]] const Value& operator[](std::size_t i) const { return items.at(i); }
  [[nodiscard]] std::size_t size() const {
    return kind == Kind::kArray ? items.size() : members.size();
  }
  [[nodiscard]] double num() const {
    if (kind != Kind::kNumber) throw std::runtime_error("json: not a number");
    return number;
  }
  [[nodiscard]] std::size_t index() const { return static_cast<std::size_t>(num()); }
  [[nodiscard]] const std::string& str() const {
    if (kind != Kind::kString) throw std::runtime_error("json: not a string");
    return text;
  }
  [[nodiscard]] std::vector<float> floats() const {
    std::vector<float> out;
    out.reserve(items.size());
    for (const Value& v : items) out.push_back(static_cast<float>(v.num()));
    return out;
  }
  [[nodiscard]] std::vector<std::size_t> indices() const {
    std::vector<std::size_t> out;
    out.reserve(items.size());
    for (const Value& v : items) out.push_back(v.index());
    return out;
  }
};

class Parser {
 public:
  explicit Parser(const std::string& text) : s_(text) {}
  Value parse() {
    Value v = value();
    space();
    if (i_ != s_.size()) error("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void error(const char* what) const {
    throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(i_));
  }
  void space() {
    while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
  }
  bool take(char c) {
    space();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!take(c)) error("unexpected character");
  }
  bool word(const char* w) {
    const std::size_t n = std::char_traits<char>::length(w);
    if (s_.compare(i_, n, w) == 0) {
      i_ += n;
      return true;
    }
    return false;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      char c = s_[i_++];
      if (c == '\\') {
        if (i_ >= s_.size()) error("bad escape");
        const char e = s_[i_++];
        c = e == 'n' ? '\n' : e == 't' ? '\t' : e;
        if (e != 'n' && e != 't' && e != '"' && e != '\\' && e != '/') error("unsupported escape");
      }
      out.push_back(c);
    }
    if (i_ >= s_.size()) error("unterminated string");
    ++i_;
    return out;
  }
  Value value() {
    space();
    if (i_ >= s_.size()) error("unexpected end");
    Value v;
    const char c = s_[i_];
    if (c == '{') {
      ++i_;
      v.kind = Value::Kind::kObject;
      if (take('}')) return v;
      do {
        space();
        std::string key = string();
        expect(':');
        v.members.emplace_back(std::move(key), value());
      } while (take(','));
      expect('}');
    } else if (c == '[') {
      ++i_;
      v.kind = Value::Kind::kArray;
      if (take(']')) return v;
      do {
        v.items.push_back(value());
      } while (take(','));
      expect(']');
    } else if (c == '"') {
      v.kind = Value::Kind::kString;
      v.text = string();
    } else if (word("true")) {
      v.kind = Value::Kind::kBool;
      v.boolean = true;
    } else if (word("false")) {
      v.kind = Value::Kind::kBool;
    } else if (word("null")) {
      v.kind = Value::Kind::kNull;
    } else if (word("NaN")) {
      v.kind = Value::Kind::kNumber;
      v.number = std::numeric_limits<double>::quiet_NaN();
    } else {
      const char* begin = s_.c_str() + i_;
      char* end = nullptr;
      v.number = std::strtod(begin, &end);
      if (end == begin) error("bad value");
      v.kind = Value::Kind::kNumber;
      i_ += static_cast<std::size_t>(end - begin);
    }
    return v;
  }

  const std::string& s_;
  std::size_t i_ = 0;
};

inline Value load(const std::string& path) {
  std::ifstream f(path);
  if (!f) throw std::runtime_error("json: cannot open " + path);
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string text = ss.str();
  return Parser(text).parse();
}

}  // namespace json_lite
