// .npy arrays of an index directory (NumPy's NEP 1 file format, versions 1.0, 2.0 and 3.0): a reader that
// maps a file and parses its header dictionary as the Python literal it is, and a streaming writer whose
// header bytes are the ones numpy.save writes (docs/design.md:27-54 of the reference names the files).
//
// Layout of a file: the magic "\x93NUMPY", a major and a minor version byte, the header length (2 bytes
// little endian for version 1, 4 bytes for 2 and 3), the header, then the raw C-order data.  The header is
// a dict literal such as {'descr': '<f4', 'fortran_order': False, 'shape': (3, 4), } padded with spaces
// and a final newline so that the data starts at a multiple of 64 bytes.
#pragma once

#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

namespace cuvs::neighbors::octex::detail {

/** The dtype string numpy writes for T on a little-endian machine (fp16 for any 2-byte type). */
template <typename T>
constexpr auto npy_descr() -> const char*
{
  if constexpr (std::is_same_v<T, int8_t> || std::is_same_v<T, signed char>) return "|i1";
  else if constexpr (std::is_same_v<T, uint8_t>) return "|u1";
  else if constexpr (std::is_same_v<T, int32_t>) return "<i4";
  else if constexpr (std::is_same_v<T, int64_t>) return "<i8";
  else if constexpr (std::is_same_v<T, float>) return "<f4";
  else if constexpr (std::is_same_v<T, double>) return "<f8";
  else if constexpr (sizeof(T) == 2) return "<f2";
  else return "";
}

/** What an .npy header says about its array. */
struct npy_header {
  std::string descr;           // e.g. "<f4", "|i1"
  bool fortran_order = false;
  std::vector<int64_t> shape;  // () for a scalar
  size_t data_offset = 0;      // bytes before the data

  /** Elements of the shape, or -1 when their count does not fit in int64. */
  [[nodiscard]] auto count() const -> int64_t
  {
    int64_t n = 1;
    for (int64_t v : shape)
      if (__builtin_mul_overflow(n, v, &n)) return -1;
    return n;
  }
  /** Bytes per element from the descr's size digits ("<f4" -> 4). */
  [[nodiscard]] auto item_bytes() const -> int64_t
  {
    int64_t b = 0;
    for (size_t i = 2; i < descr.size() && descr[i] >= '0' && descr[i] <= '9'; i++) {  // after byte order, kind
      b = b * 10 + (descr[i] - '0');
      if (b > (int64_t{1} << 20)) return -1;  // no element type is this wide
    }
    return b;
  }
};

/**
 * The header dictionary of an .npy file read as the Python literal numpy writes: string keys mapped to a
 * quoted string ('descr'), True / False ('fortran_order') or a tuple of integers ('shape').  Keys are
 * accepted in any order with any spacing, a trailing comma is allowed, and integers may carry Python 2's
 * "L" suffix; anything else is an error naming the file.
 */
class npy_header_parser {
 public:
  npy_header_parser(std::string text, std::string const& file) : t_(std::move(text)), file_(file) {}

  auto parse() -> npy_header
  {
    npy_header h;
    bool has_descr = false, has_shape = false;
    expect('{');
    for (;;) {
      skip();
      if (peek() == '}') break;
      const std::string key = quoted();
      expect(':');
      skip();
      if (key == "descr") {
        h.descr   = quoted();
        has_descr = true;
      } else if (key == "fortran_order") {
        h.fortran_order = boolean();
      } else if (key == "shape") {
        h.shape   = tuple();
        has_shape = true;
      } else {
        bad("unknown header key '" + key + "'");
      }
      skip();
      if (peek() == ',') i_++;
    }
    i_++;
    if (!has_descr || !has_shape) bad("header without descr or shape");
    return h;
  }

 private:
  std::string t_;
  std::string const& file_;
  size_t i_ = 0;

  [[noreturn]] void bad(std::string const& why) const
  {
    fail("octex: %s: malformed .npy header (%s)", file_.c_str(), why.c_str());
  }
  void skip()
  {
    while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\t' || t_[i_] == '\n' || t_[i_] == '\r'))
      i_++;
  }
  auto peek() const -> char { return i_ < t_.size() ? t_[i_] : '\0'; }
  void expect(char c)
  {
    skip();
    if (peek() != c) bad(std::string("expected '") + c + "'");
    i_++;
  }
  auto quoted() -> std::string
  {
    skip();
    const char q = peek();
    if (q != '\'' && q != '"') bad("expected a quoted string");
    const size_t end = t_.find(q, i_ + 1);
    if (end == std::string::npos) bad("unterminated string");
    std::string s = t_.substr(i_ + 1, end - i_ - 1);
    i_            = end + 1;
    return s;
  }
  auto boolean() -> bool
  {
    if (t_.compare(i_, 4, "True") == 0) {
      i_ += 4;
      return true;
    }
    if (t_.compare(i_, 5, "False") == 0) {
      i_ += 5;
      return false;
    }
    bad("expected True or False");
  }
  auto tuple() -> std::vector<int64_t>
  {
    std::vector<int64_t> v;
    expect('(');
    for (;;) {
      skip();
      if (peek() == ')') break;
      if (peek() < '0' || peek() > '9') bad("expected a dimension");
      int64_t x = 0;
      while (peek() >= '0' && peek() <= '9') {  // every dimension below 2^62: no overflow here or in count()'s checks
        const int digit = t_[i_++] - '0';
        if (x > ((int64_t{1} << 62) - 1 - digit) / 10) bad("a dimension of 2^62 or more");  // checked before the step
        x = x * 10 + digit;
      }
      if (peek() == 'L') i_++;
      v.push_back(x);
      skip();
      if (peek() == ',') i_++;
      else if (peek() != ')') bad("expected ',' or ')' in the shape");
    }
    i_++;
    return v;
  }
};

/** The header at the start of `bytes` (the first `len` bytes of a file). */
inline auto read_npy_header(const unsigned char* bytes, size_t len, std::string const& file) -> npy_header
{
  static const unsigned char magic[6] = {0x93, 'N', 'U', 'M', 'P', 'Y'};
  OCTEX_EXPECTS(len >= 10 && std::memcmp(bytes, magic, 6) == 0, "octex: %s is not an .npy file", file.c_str());
  const int major      = bytes[6];
  OCTEX_EXPECTS(major >= 1 && major <= 3, "octex: %s: .npy format version %d is not supported", file.c_str(), major);
  const size_t len_bytes = major == 1 ? 2 : 4;
  OCTEX_EXPECTS(len >= 8 + len_bytes, "octex: %s: truncated .npy header", file.c_str());
  size_t hlen = 0;
  for (size_t b = 0; b < len_bytes; b++)
    hlen |= static_cast<size_t>(bytes[8 + b]) << (8 * b);
  const size_t start = 8 + len_bytes;
  OCTEX_EXPECTS(start + hlen <= len, "octex: %s: truncated .npy header", file.c_str());
  npy_header h = npy_header_parser(std::string(reinterpret_cast<const char*>(bytes) + start, hlen), file).parse();
  h.data_offset = start + hlen;
  OCTEX_EXPECTS(!h.fortran_order, "octex: %s: Fortran-order arrays are not supported", file.c_str());
  OCTEX_EXPECTS(h.descr.size() >= 3 && (h.descr[0] == '<' || h.descr[0] == '|'),
                "octex: %s: dtype %s is not little endian", file.c_str(), h.descr.c_str());
  return h;
}

/** A read-only mapping of a whole file, unmapped on destruction (also when a constructor throws later). */
class file_map {
 public:
  file_map() = default;
  explicit file_map(std::string const& path)
  {
    const int fd = ::open(path.c_str(), O_RDONLY);
    OCTEX_EXPECTS(fd >= 0, "octex: cannot open %s", path.c_str());
    struct stat st {};
    len_    = ::fstat(fd, &st) == 0 ? static_cast<size_t>(st.st_size) : 0;
    void* p = len_ > 0 ? ::mmap(nullptr, len_, PROT_READ, MAP_SHARED, fd, 0) : MAP_FAILED;
    ::close(fd);
    OCTEX_EXPECTS(p != MAP_FAILED, "octex: cannot map %s (%zu bytes)", path.c_str(), len_);
    p_ = p;
  }
  file_map(file_map const&)                    = delete;
  auto operator=(file_map const&) -> file_map& = delete;
  file_map(file_map&& o) noexcept { *this = std::move(o); }
  auto operator=(file_map&& o) noexcept -> file_map&
  {
    std::swap(p_, o.p_);
    std::swap(len_, o.len_);
    return *this;
  }
  ~file_map()
  {
    if (p_ != nullptr) ::munmap(p_, len_);
  }
  [[nodiscard]] auto bytes() const -> const unsigned char* { return static_cast<const unsigned char*>(p_); }
  [[nodiscard]] auto size() const -> size_t { return len_; }

 private:
  void* p_    = nullptr;
  size_t len_ = 0;
};

/** An .npy file mapped read-only; `data` stays valid while the object lives. */
class npy_file {
 public:
  npy_header hdr;
  const char* data = nullptr;

  npy_file() = default;
  explicit npy_file(std::string const& path) : path_(path), map_(path)
  {
    hdr  = read_npy_header(map_.bytes(), map_.size(), path);
    data = reinterpret_cast<const char*>(map_.bytes()) + hdr.data_offset;
    int64_t need       = 0;
    const int64_t cnt  = hdr.count();
    OCTEX_EXPECTS(cnt >= 0 && hdr.item_bytes() >= 0 && !__builtin_mul_overflow(cnt, hdr.item_bytes(), &need) &&
                    need <= std::numeric_limits<int64_t>::max() - static_cast<int64_t>(hdr.data_offset),
                  "octex: %s: the shape's byte count overflows", path.c_str());
    OCTEX_EXPECTS(hdr.data_offset + static_cast<size_t>(need) <= map_.size(),
                  "octex: %s holds %zu data bytes, its shape needs %lld", path.c_str(),
                  map_.size() - hdr.data_offset, static_cast<long long>(need));
  }

  [[nodiscard]] auto shape() const -> std::vector<int64_t> const& { return hdr.shape; }
  [[nodiscard]] auto rank() const -> size_t { return hdr.shape.size(); }
  /** Extent i, or 1 past the rank. */
  [[nodiscard]] auto dim(size_t i) const -> int64_t { return i < hdr.shape.size() ? hdr.shape[i] : 1; }
  [[nodiscard]] auto path() const -> std::string const& { return path_; }
  /** The data as T, after checking the file's dtype is T's. */
  template <typename T>
  [[nodiscard]] auto as() const -> const T*
  {
    OCTEX_EXPECTS(hdr.descr == npy_descr<T>(), "octex: %s has dtype %s, expected %s", path_.c_str(), hdr.descr.c_str(),
                  npy_descr<T>());
    return reinterpret_cast<const T*>(data);
  }

 private:
  std::string path_;
  file_map map_;
};

/**
 * The bytes numpy.save puts before the data of a C-order array (format 1.0): magic, version, length, the
 * dict with its keys in sorted order and Python's tuple spelling of the shape ("(7,)" for one dimension),
 * spaces and a newline up to a multiple of 64 bytes.
 */
inline auto npy_preamble(std::string const& descr, std::vector<int64_t> const& shape) -> std::string
{
  std::string tup;
  for (size_t i = 0; i < shape.size(); i++)
    tup += (i > 0 ? ", " : "") + std::to_string(shape[i]);
  if (shape.size() == 1) tup += ",";
  std::string dict = "{'descr': '" + descr + "', 'fortran_order': False, 'shape': (" + tup + "), }";
  const size_t unpadded = 10 + dict.size() + 1;  // magic, version, length, dict, newline
  dict.append((64 - unpadded % 64) % 64, ' ');
  dict.push_back('\n');
  std::string out("\x93NUMPY\x01\x00", 8);
  out.push_back(static_cast<char>(dict.size() & 0xff));
  out.push_back(static_cast<char>(dict.size() >> 8));
  return out + dict;
}

/** An .npy file written front to back: the preamble, then the data in any number of pieces. */
class npy_writer {
 public:
  npy_writer(std::string const& path, std::string const& descr, std::vector<int64_t> const& shape) : path_(path)
  {
    f_ = std::fopen(path.c_str(), "wb");
    OCTEX_EXPECTS(f_ != nullptr, "octex: cannot write %s", path.c_str());
    const std::string pre = npy_preamble(descr, shape);
    put(pre.data(), pre.size());
  }
  npy_writer(npy_writer const&)                    = delete;
  auto operator=(npy_writer const&) -> npy_writer& = delete;
  ~npy_writer()
  {
    if (f_ != nullptr) std::fclose(f_);
  }
  void put(const void* p, size_t bytes)
  {
    OCTEX_EXPECTS(bytes == 0 || std::fwrite(p, 1, bytes, f_) == bytes, "octex: short write %s", path_.c_str());
  }
  void zeros(size_t bytes)
  {
    static const std::vector<char> z(size_t{1} << 20, 0);
    for (size_t left = bytes; left > 0;) {
      const size_t m = std::min(left, z.size());
      put(z.data(), m);
      left -= m;
    }
  }
  void close()
  {
    FILE* f = f_;
    f_      = nullptr;
    OCTEX_EXPECTS(std::fclose(f) == 0, "octex: short write %s", path_.c_str());
  }

 private:
  std::string path_;
  FILE* f_ = nullptr;
};

/** A whole host array as one .npy file. */
template <typename T>
void write_npy(std::string const& path, const T* data, std::vector<int64_t> const& shape)
{
  int64_t n = 1;
  for (int64_t v : shape)
    n *= v;
  npy_writer w(path, npy_descr<T>(), shape);
  w.put(data, static_cast<size_t>(n) * sizeof(T));
  w.close();
}

}  // namespace cuvs::neighbors::octex::detail
