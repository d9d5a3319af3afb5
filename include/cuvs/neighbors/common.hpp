/*
 * Base structs of cuVS neighbor indexes that the octex parameter structs and index derive from
 * (octex.hpp:32, 101, 187 in the reference).
 */
#pragma once

namespace cuvs::neighbors {

struct index_params {
  virtual ~index_params() = default;
};
struct search_params {
  virtual ~search_params() = default;
};
struct index {
  virtual ~index() = default;
};

}  // namespace cuvs::neighbors
