/*
 * octex C++ API for MI355X: namespace cuvs::neighbors::octex with the parameter structs, defaults,
 * index class and build/load/search functions of the reference (cpp/include/cuvs/neighbors/octex.hpp
 * :32-253), so that C++ callers recompile unchanged against this library.  The RAFT resource and view
 * types are this library's minimal ones (raft/core/ headers); the fp16 type is HIP's `half`.
 */
#pragma once

#include <hip/hip_fp16.h>

#include <cuvs/neighbors/common.hpp>
#include <raft/core/device_mdspan.hpp>
#include <raft/core/host_mdspan.hpp>
#include <raft/core/resources.hpp>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace cuvs::neighbors::octex {

/** Index build parameters; fields and defaults as octex.hpp:32-92. */
struct index_params : cuvs::neighbors::index_params {
  int copies                  = 200;
  int blocks                  = 4;
  int pca_dims                = 64;
  std::vector<float> spacings = {2.0f, 2.5f, 3.2f, 4.0f, 5.0f};
  int list_len                = 64;
  int min_cell                = 1;
  int log_buckets             = 20;
  int sketch_width            = 0;
  int table_len               = 64;
  bool reverse_edges          = true;
  bool exact_lists            = false;
  int list_probes             = 16;
  bool member_lists           = false;
  int64_t exact_table_max     = 20000000;
  int table_passes            = 3;
  bool table_sketch_order     = false;
  bool write_behind           = false;
  uint64_t seed               = 0;
  std::vector<int> devices{};
};

/** Search parameters; fields and defaults as octex.hpp:101-135. */
struct search_params : cuvs::neighbors::search_params {
  int read             = 32;
  int starts           = 128;
  int waves            = 2;
  int rerank           = 128;
  int wave_rerank      = 128;
  int batch            = 10000;
  bool sketch_rank     = false;
  int final_rerank     = 32;
  bool balanced_gather = true;
  bool fused_merge     = true;
  bool use_graph       = true;
};

/** octex.hpp:138-143. */
enum class placement : int { replicate = 0, shard = 1 };

/** octex.hpp:146-153. */
enum class sketch_placement : int { replicate = 0, shard = 1, host = 2 };

/** Load parameters; fields and defaults as octex.hpp:155-176. */
struct load_params {
  std::vector<int> devices{};
  placement mode            = placement::shard;
  bool vectors_on_host      = false;
  bool shard_vectors        = false;
  bool table_on_host        = false;
  sketch_placement sketch   = sketch_placement::replicate;
  int parts                 = 0;
  int copies_per_part       = 0;
  int copies_limit          = 0;
  int list_limit            = 0;
};

namespace detail {
struct index_impl;
}

/** An octex index placed on a GPU (octex.hpp:187-204). */
class index : public cuvs::neighbors::index {
 public:
  explicit index(std::shared_ptr<detail::index_impl> impl);
  index(index&&) noexcept;
  auto operator=(index&&) noexcept -> index&;
  ~index() override;

  [[nodiscard]] auto size() const noexcept -> int64_t;
  [[nodiscard]] auto dim() const noexcept -> int64_t;
  [[nodiscard]] auto copies() const noexcept -> int;
  [[nodiscard]] auto devices() const noexcept -> std::vector<int> const&;
  /** Device memory per GPU, in bytes. */
  [[nodiscard]] auto device_bytes() const -> std::vector<int64_t>;
  [[nodiscard]] auto impl() const noexcept -> detail::index_impl&;

 private:
  std::shared_ptr<detail::index_impl> impl_;
};

/** Build an index of a dataset [N, D] and write it to a directory (octex.hpp:214-222). */
void build(raft::resources const& res,
           index_params const& params,
           raft::host_matrix_view<const float, int64_t, raft::row_major> dataset,
           std::string const& path);

void build(raft::resources const& res,
           index_params const& params,
           raft::host_matrix_view<const half, int64_t, raft::row_major> dataset,
           std::string const& path);

/** Load an index directory onto the GPU (octex.hpp:225-226). */
auto load(raft::resources const& res, std::string const& path, load_params const& params = {})
  -> index;

/**
 * The k nearest neighbors of a batch of queries (octex.hpp:241-253); k = neighbors.extent(1).
 * Results are squared distances, nearest first.
 */
void search(raft::resources const& res,
            search_params const& params,
            index const& idx,
            raft::host_matrix_view<const float, int64_t, raft::row_major> queries,
            raft::host_matrix_view<int64_t, int64_t, raft::row_major> neighbors,
            raft::host_matrix_view<float, int64_t, raft::row_major> distances);

void search(raft::resources const& res,
            search_params const& params,
            index const& idx,
            raft::device_matrix_view<const float, int64_t, raft::row_major> queries,
            raft::device_matrix_view<int64_t, int64_t, raft::row_major> neighbors,
            raft::device_matrix_view<float, int64_t, raft::row_major> distances);

}  // namespace cuvs::neighbors::octex
