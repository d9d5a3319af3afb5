// .npy files of an index directory (format 1.0 / 2.0, little endian, C order): a memory-mapped reader
// and a writer whose header layout is numpy's own (the reference: detail/npy.hpp:222-413).
#pragma once

#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

namespace cuvs::neighbors::octex::detail {

template <typename T>
constexpr auto npy_descr() -> const char*
{
  if constexpr (std::is_same_v<T, float>) return "<f4";
  if constexpr (std::is_same_v<T, double>) return "<f8";
  if constexpr (std::is_same_v<T, int8_t>) return "|i1";
  if constexpr (std::is_same_v<T, uint8_t>) return "|u1";
  if constexpr (std::is_same_v<T, int32_t>) return "<i4";
  if constexpr (std::is_same_v<T, int64_t>) return "<i8";
  if constexpr (sizeof(T) == 2) return "<f2";
  return "";
}

/** Parsed header of an .npy file. */
struct npy_header {
  std::string descr;
  std::vector<int64_t> shape;
  size_t data_offset = 0;
  size_t data_bytes  = 0;
};

/** Parse the header text of an .npy file held in `p` (at least `len` bytes). */
inline auto parse_npy_header(const char* p, size_t len, std::string const& path) -> npy_header
{
  OCTEX_EXPECTS(len >= 10 && std::memcmp(p, "\x93NUMPY", 6) == 0, "octex: not an .npy file: %s",
                path.c_str());
  const int major = static_cast<unsigned char>(p[6]);
  size_t hlen = 0, hstart = 0;
  if (major == 1) {
    hlen   = static_cast<uint8_t>(p[8]) | (static_cast<size_t>(static_cast<uint8_t>(p[9])) << 8);
    hstart = 10;
  } else {
    OCTEX_EXPECTS(len >= 12, "octex: truncated header: %s", path.c_str());
    hlen = static_cast<uint8_t>(p[8]) | (static_cast<size_t>(static_cast<uint8_t>(p[9])) << 8) |
           (static_cast<size_t>(static_cast<uint8_t>(p[10])) << 16) |
           (static_cast<size_t>(static_cast<uint8_t>(p[11])) << 24);
    hstart = 12;
  }
  OCTEX_EXPECTS(hstart + hlen <= len, "octex: truncated header: %s", path.c_str());
  std::string hdr(p + hstart, hlen);
  OCTEX_EXPECTS(hdr.find("'fortran_order': True") == std::string::npos,
                "octex: Fortran order not supported: %s", path.c_str());
  npy_header out;
  auto d = hdr.find("'descr':");
  OCTEX_EXPECTS(d != std::string::npos, "octex: no descr in %s", path.c_str());
  auto q1   = hdr.find('\'', d + 8);
  auto q2   = hdr.find('\'', q1 + 1);
  out.descr = hdr.substr(q1 + 1, q2 - q1 - 1);
  auto sp   = hdr.find("'shape':");
  OCTEX_EXPECTS(sp != std::string::npos, "octex: no shape in %s", path.c_str());
  auto s = hdr.find('(', sp), e = hdr.find(')', s);
  std::string sh = hdr.substr(s + 1, e - s - 1);
  size_t pos     = 0;
  while (pos < sh.size()) {
    while (pos < sh.size() && (sh[pos] == ' ' || sh[pos] == ',' || sh[pos] == 'L'))
      pos++;
    if (pos >= sh.size()) break;
    size_t end = pos;
    while (end < sh.size() && sh[end] != ',')
      end++;
    out.shape.push_back(std::stoll(sh.substr(pos, end - pos)));
    pos = end;
  }
  out.data_offset = hstart + hlen;
  return out;
}

/** An .npy file mapped read-only. */
struct npy_file {
  npy_header hdr;
  const char* data = nullptr;
  size_t bytes     = 0;
  void* map_       = nullptr;
  size_t map_len_  = 0;

  npy_file() = default;
  explicit npy_file(std::string const& path)
  {
    int fd = ::open(path.c_str(), O_RDONLY);
    OCTEX_EXPECTS(fd >= 0, "octex: cannot open %s", path.c_str());
    struct stat st {};
    ::fstat(fd, &st);
    map_len_ = static_cast<size_t>(st.st_size);
    map_     = map_len_ > 0 ? ::mmap(nullptr, map_len_, PROT_READ, MAP_SHARED, fd, 0) : MAP_FAILED;
    ::close(fd);
    OCTEX_EXPECTS(map_ != MAP_FAILED, "octex: cannot map %s", path.c_str());
    hdr = parse_npy_header(static_cast<const char*>(map_), map_len_, path);
    OCTEX_EXPECTS(hdr.data_offset <= map_len_, "octex: truncated file %s", path.c_str());
    data  = static_cast<const char*>(map_) + hdr.data_offset;
    bytes = map_len_ - hdr.data_offset;
    int64_t want = numel() * item_size();
    OCTEX_EXPECTS(static_cast<int64_t>(bytes) >= want, "octex: %s holds %zu data bytes, its shape needs %lld",
                  path.c_str(), bytes, static_cast<long long>(want));
    path_ = path;
  }
  npy_file(npy_file const&)                    = delete;
  auto operator=(npy_file const&) -> npy_file& = delete;
  npy_file(npy_file&& o) noexcept { *this = std::move(o); }
  auto operator=(npy_file&& o) noexcept -> npy_file&
  {
    std::swap(hdr, o.hdr);
    std::swap(data, o.data);
    std::swap(bytes, o.bytes);
    std::swap(map_, o.map_);
    std::swap(map_len_, o.map_len_);
    std::swap(path_, o.path_);
    return *this;
  }
  ~npy_file()
  {
    if (map_ != nullptr && map_ != MAP_FAILED) ::munmap(map_, map_len_);
  }
  [[nodiscard]] auto shape() const -> std::vector<int64_t> const& { return hdr.shape; }
  [[nodiscard]] auto dim(size_t i) const -> int64_t { return i < hdr.shape.size() ? hdr.shape[i] : 1; }
  [[nodiscard]] auto numel() const -> int64_t
  {
    int64_t n = 1;
    for (auto v : hdr.shape)
      n *= v;
    return n;
  }
  [[nodiscard]] auto item_size() const -> int64_t
  {
    const auto& d = hdr.descr;
    if (d.size() >= 3) return std::stoll(d.substr(2));
    return 1;
  }
  template <typename T>
  [[nodiscard]] auto as() const -> const T*
  {
    OCTEX_EXPECTS(hdr.descr == npy_descr<T>(), "octex: %s has dtype %s, expected %s", path_.c_str(),
                  hdr.descr.c_str(), npy_descr<T>());
    return reinterpret_cast<const T*>(data);
  }

 private:
  std::string path_;
};

/** Write a C-order array (format 1.0, header padded to a multiple of 64 bytes). */
template <typename T>
void write_npy(std::string const& path, const T* data, std::vector<int64_t> const& shape)
{
  std::string sh = "(";
  int64_t n      = 1;
  for (size_t i = 0; i < shape.size(); i++) {
    sh += std::to_string(shape[i]);
    if (shape.size() == 1 || i + 1 < shape.size()) sh += ",";
    if (i + 1 < shape.size()) sh += " ";
    n *= shape[i];
  }
  sh += ")";
  std::string hdr = std::string("{'descr': '") + npy_descr<T>() +
                    "', 'fortran_order': False, 'shape': " + sh + ", }";
  const size_t total = 10 + hdr.size() + 1;
  hdr.append((64 - total % 64) % 64, ' ');
  hdr += '\n';
  FILE* f = std::fopen(path.c_str(), "wb");
  OCTEX_EXPECTS(f != nullptr, "octex: cannot write %s", path.c_str());
  const char magic[8] = {'\x93', 'N', 'U', 'M', 'P', 'Y', '\x01', '\x00'};
  bool ok             = std::fwrite(magic, 1, 8, f) == 8;
  const uint16_t hl   = static_cast<uint16_t>(hdr.size());
  ok                  = ok && std::fwrite(&hl, 2, 1, f) == 1;
  ok                  = ok && std::fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
  const size_t want   = static_cast<size_t>(n) * sizeof(T);
  ok                  = ok && (want == 0 || std::fwrite(data, 1, want, f) == want);
  ok                  = (std::fclose(f) == 0) && ok;
  OCTEX_EXPECTS(ok, "octex: short write %s", path.c_str());
}

}  // namespace cuvs::neighbors::octex::detail
