// The octex index builder (build.cpp): an index built in HBM, and the writer of its directory.
#pragma once

#include "index_impl.hpp"

#include <hip/hip_fp16.h>

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace cuvs::neighbors::octex::detail {

/** The host arrays of a build that its directory holds besides the device ones, and phase times. */
struct build_record {
  std::vector<float> mean, proj, shift, basis, scale;
  std::vector<int32_t> base;
  std::vector<int64_t> cells;
  std::vector<std::pair<std::string, double>> phases;
};

/** The dataset of a build: row-major [n, d], fp16 or fp32, in host or device memory. */
struct dataset_view {
  const void* data = nullptr;
  int64_t n = 0, d = 0;
  bool f32    = false;
  bool device = false;
};

/**
 * Build the index of x in the HBM of params.devices[0] (or the current GPU).  The rows are stored as
 * fp16 (round to nearest) whatever their type; a device dataset is read in place.
 */
auto build_in_memory(index_params const& params, dataset_view const& x, build_record& rec,
                     std::function<void(std::shared_ptr<index_impl> const&)> const& before_table = {})
  -> std::shared_ptr<index_impl>;
/** Write the format-1 directory of a built index (meta.json last). */
void write_index(index_impl const& ix, build_record const& rec, index_params const& params, std::string const& path);
/**
 * Build the index of x into the directory `path` and return it (build.cu:104-454).  With params.write_behind the
 * arrays that are final before the neighbor table are written by a background thread while the table is built,
 * and joined before table.npy and meta.json (meta.json last).  With OCTEX_TABLE_ONLY set in the environment the
 * directory already holds every array but table.npy and meta.json (a build that stopped in its table phase): only
 * the neighbor table is built, over those arrays, and table.npy and meta.json written.
 */
auto build_to_directory(index_params const& params, dataset_view const& x, std::string const& path,
                        build_record& rec) -> std::shared_ptr<index_impl>;
/** Replace / free the neighbor table of a loaded index (the reference's detail::set_table / drop_table). */
void set_table(index_impl& ix, std::vector<int32_t> const& rows, int k);
void drop_table(index_impl& ix);

}  // namespace cuvs::neighbors::octex::detail
