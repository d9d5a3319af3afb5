// A C++ caller of the cuvs::neighbors::octex API (include/cuvs/neighbors/octex.hpp), as the reference's C++ users
// (examples/cpp/search.cu, octex_bench) call it: build from a host dataset, load, search host queries.
// Usage: octex_search_cpp DIR N D M K DATA.f32 QUERIES.f32 OUT (as the C caller: writes OUT.i64 and OUT.f32).
#include <cuvs/neighbors/octex.hpp>
#include <raft/core/host_mdspan.hpp>
#include <raft/core/resources.hpp>

#include <cstdint>
#include <cstdio>
#include <exception>
#include <fstream>
#include <string>
#include <vector>

namespace octex = cuvs::neighbors::octex;

template <typename T>
static auto read_all(std::string const& path, size_t count) -> std::vector<T>
{
  std::vector<T> v(count);
  std::ifstream f(path, std::ios::binary);
  if (!f.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(count * sizeof(T))))
    throw std::runtime_error("cannot read " + path);
  return v;
}

template <typename T>
static void write_all(std::string const& path, std::vector<T> const& v)
{
  std::ofstream f(path, std::ios::binary);
  if (!f.write(reinterpret_cast<const char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T))))
    throw std::runtime_error("cannot write " + path);
}

int main(int argc, char** argv)
{
  if (argc != 9) {
    std::fprintf(stderr, "usage: %s DIR N D M K DATA.f32 QUERIES.f32 OUT\n", argv[0]);
    return 2;
  }
  try {
    const std::string dir = argv[1];
    const int64_t n = std::stoll(argv[2]), d = std::stoll(argv[3]), m = std::stoll(argv[4]), k = std::stoll(argv[5]);
    auto x = read_all<float>(argv[6], static_cast<size_t>(n * d));
    auto q = read_all<float>(argv[7], static_cast<size_t>(m * d));
    std::vector<int64_t> nb(static_cast<size_t>(m * k));
    std::vector<float> dist(static_cast<size_t>(m * k));

    raft::resources res;
    octex::index_params ip;
    ip.copies      = 16;
    ip.list_len    = 32;
    ip.table_len   = 32;
    ip.log_buckets = 12;
    ip.seed        = 1;
    octex::build(res, ip, raft::make_host_matrix_view<const float, int64_t>(x.data(), n, d), dir);
    auto index = octex::load(res, dir);
    if (index.size() != n || index.dim() != d) throw std::runtime_error("index shape differs from the dataset");

    octex::search_params sp;
    sp.read   = 16;
    sp.starts = 64;
    sp.waves  = 2;
    octex::search(res, sp, index, raft::make_host_matrix_view<const float, int64_t>(q.data(), m, d),
                  raft::make_host_matrix_view<int64_t, int64_t>(nb.data(), m, k),
                  raft::make_host_matrix_view<float, int64_t>(dist.data(), m, k));
    write_all(std::string(argv[8]) + ".i64", nb);
    write_all(std::string(argv[8]) + ".f32", dist);
    std::printf("c++ caller: %lld queries, first ids %lld %lld %lld\n", static_cast<long long>(m),
                static_cast<long long>(nb[0]), static_cast<long long>(nb[1]), static_cast<long long>(nb[2]));
  } catch (std::exception const& e) {
    std::fprintf(stderr, "octex: %s\n", e.what());
    return 1;
  }
  return 0;
}
