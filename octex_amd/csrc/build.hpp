// The octex index builder (build.cpp): an index built in HBM, and the writer of its directory.
#pragma once

#include "index_impl.hpp"

#include <hip/hip_fp16.h>

#include <cstdint>
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

/** Build the index of the fp16 rows x [n, d] (host) in the HBM of params.devices[0] (or the current GPU). */
auto build_in_memory(index_params const& params, const __half* x, int64_t n, int64_t d, build_record& rec)
  -> std::shared_ptr<index_impl>;
/** Write the format-1 directory of a built index (meta.json last). */
void write_index(index_impl const& ix, build_record const& rec, index_params const& params, std::string const& path);
/** Replace / free the neighbor table of a loaded index (the reference's detail::set_table / drop_table). */
void set_table(index_impl& ix, std::vector<int32_t> const& rows, int k);
void drop_table(index_impl& ix);

}  // namespace cuvs::neighbors::octex::detail
