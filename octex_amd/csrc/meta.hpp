// meta.json of an index directory (format 1): a small JSON reader (objects, arrays, strings, numbers,
// booleans, null) and the writer of the reference's layout (build.cu:67-98).  Unknown keys (e.g.
// "build_seconds") are ignored, "files" maps array names to absolute or relative paths (load.cu
// :229-234).
#pragma once

#include "common.hpp"

#include <charconv>
#include <cstdlib>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

namespace cuvs::neighbors::octex::detail {

struct json_value {
  enum kind_t { null_v, bool_v, number_v, string_v, array_v, object_v } kind = null_v;
  bool b   = false;
  double d = 0;
  std::string s;
  std::vector<json_value> a;
  std::map<std::string, json_value> o;

  [[nodiscard]] auto get(std::string const& key) const -> const json_value*
  {
    if (kind != object_v) return nullptr;
    auto it = o.find(key);
    return it == o.end() ? nullptr : &it->second;
  }
  [[nodiscard]] auto number(std::string const& key, double dflt) const -> double
  {
    auto v = get(key);
    return v != nullptr && v->kind == number_v ? v->d : dflt;
  }
};

class json_parser {
 public:
  explicit json_parser(std::string const& text) : t_(text) {}
  auto parse() -> json_value
  {
    auto v = value();
    ws();
    OCTEX_EXPECTS(i_ == t_.size(), "octex: meta.json: trailing characters at %zu", i_);
    return v;
  }

 private:
  std::string const& t_;
  size_t i_ = 0;

  void ws()
  {
    while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\n' || t_[i_] == '\r' || t_[i_] == '\t'))
      i_++;
  }
  auto peek() -> char
  {
    ws();
    OCTEX_EXPECTS(i_ < t_.size(), "octex: meta.json: unexpected end");
    return t_[i_];
  }
  void expect(char c)
  {
    OCTEX_EXPECTS(peek() == c, "octex: meta.json: expected '%c' at %zu", c, i_);
    i_++;
  }
  auto str() -> std::string
  {
    expect('"');
    std::string out;
    while (i_ < t_.size() && t_[i_] != '"') {
      char c = t_[i_++];
      if (c == '\\' && i_ < t_.size()) {
        char e = t_[i_++];
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {
            OCTEX_EXPECTS(i_ + 4 <= t_.size(), "octex: meta.json: bad escape");
            unsigned cp = static_cast<unsigned>(std::stoul(t_.substr(i_, 4), nullptr, 16));
            i_ += 4;
            if (cp < 0x80) {
              out += static_cast<char>(cp);
            } else if (cp < 0x800) {
              out += static_cast<char>(0xc0 | (cp >> 6));
              out += static_cast<char>(0x80 | (cp & 0x3f));
            } else {
              out += static_cast<char>(0xe0 | (cp >> 12));
              out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
              out += static_cast<char>(0x80 | (cp & 0x3f));
            }
            break;
          }
          default: out += e;
        }
      } else {
        out += c;
      }
    }
    OCTEX_EXPECTS(i_ < t_.size(), "octex: meta.json: unterminated string");
    i_++;
    return out;
  }
  auto value() -> json_value
  {
    json_value v;
    char c = peek();
    if (c == '{') {
      i_++;
      v.kind = json_value::object_v;
      if (peek() == '}') {
        i_++;
        return v;
      }
      while (true) {
        std::string k = str();
        expect(':');
        v.o[k] = value();
        char e = peek();
        i_++;
        if (e == '}') break;
        OCTEX_EXPECTS(e == ',', "octex: meta.json: expected ',' or '}' at %zu", i_);
      }
    } else if (c == '[') {
      i_++;
      v.kind = json_value::array_v;
      if (peek() == ']') {
        i_++;
        return v;
      }
      while (true) {
        v.a.push_back(value());
        char e = peek();
        i_++;
        if (e == ']') break;
        OCTEX_EXPECTS(e == ',', "octex: meta.json: expected ',' or ']' at %zu", i_);
      }
    } else if (c == '"') {
      v.kind = json_value::string_v;
      v.s    = str();
    } else if (t_.compare(i_, 4, "true") == 0) {
      v.kind = json_value::bool_v;
      v.b    = true;
      i_ += 4;
    } else if (t_.compare(i_, 5, "false") == 0) {
      v.kind = json_value::bool_v;
      i_ += 5;
    } else if (t_.compare(i_, 4, "null") == 0) {
      i_ += 4;
    } else {
      const char* b = t_.c_str() + i_;
      char* e       = nullptr;
      v.d           = std::strtod(b, &e);
      OCTEX_EXPECTS(e != b, "octex: meta.json: bad value at %zu", i_);
      v.kind = json_value::number_v;
      i_ += static_cast<size_t>(e - b);
    }
    return v;
  }
};

/** Shortest text that reads back as the same float (the reference writer's json_float). */
inline auto json_float(double v) -> std::string
{
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof(buf), static_cast<float>(v));
  std::string s(buf, r.ptr);
  if (s.find_first_of(".en") == std::string::npos) s += ".0";
  return s;
}

}  // namespace cuvs::neighbors::octex::detail
