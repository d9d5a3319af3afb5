// octex::build (octex.hpp:214-222): index construction into a format-1 directory.
#include "common.hpp"

#include <cuvs/neighbors/octex.hpp>

namespace cuvs::neighbors::octex {

void build(raft::resources const&, index_params const&,
           raft::host_matrix_view<const float, int64_t, raft::row_major>, std::string const&)
{
  detail::fail("octex: build is not available in this build of the library");
}

void build(raft::resources const&, index_params const&,
           raft::host_matrix_view<const half, int64_t, raft::row_major>, std::string const&)
{
  detail::fail("octex: build is not available in this build of the library");
}

}  // namespace cuvs::neighbors::octex
