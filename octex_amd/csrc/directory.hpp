// An index directory (format 1) opened and checked on the host: meta.json parsed, every array mapped and its
// dtype and shape compared with what meta.json implies, before any device call (the reference reads the same
// files in load.cu:215-300).
#pragma once

#include "npy.hpp"

#include <cuvs/neighbors/octex.hpp>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace cuvs::neighbors::octex::detail {

struct directory {
  std::string path;
  int64_t n = 0, dim = 0;
  int all_copies = 0, blocks = 4, list_len = 0, log_buckets = 20, sketch_width = 0, table_len = 0;
  std::vector<double> spacings;               // the JSON values (inv_f is float(1 / value), load.cu:397-399)
  std::map<std::string, std::string> files;   // "files": array name -> absolute or directory-relative path
  std::vector<int> copy_list;                 // the copies a load with these parameters places
  // lists [C, rows * list_len] i4, keys [C, L, mmax] i8, offsets [C, L, 2^log_buckets + 1] i4, base [C, L] i4,
  // proj [C, dim, 8 blocks] f4, shift [C, 8 blocks] f4, mean [dim] f4, sketch_basis [dim, S] f4,
  // sketch_scale [S] f4, sketch [n, S] i1, vectors [n, dim] f2, table [n, table_len] i4 (table_len > 0)
  npy_file lists, keys, offsets, base, proj, shift, mean, basis, scale, sketch, vectors, table;
};

/**
 * Open the index directory at `path` for a load with `params`: parse meta.json (unknown keys ignored, "files"
 * remapping honoured), map every array, and check its dtype and full shape, the copy selection (parts,
 * copies_per_part, copies_limit) and that every level's cell table stays inside keys and lists.  Throws an
 * "octex: ..." error naming the file on any mismatch; makes no device call.
 */
auto open_directory(std::string const& path, load_params const& params) -> directory;
/** open_directory with the text of meta.json given (a build resumed before its meta.json is written). */
auto open_directory(std::string const& path, load_params const& params, std::string const& meta_text) -> directory;
/** The index of an opened directory on one GPU (the body of load()). */
auto load_directory(directory const& dir, std::string const& path, load_params const& params)
  -> std::shared_ptr<index_impl>;

}  // namespace cuvs::neighbors::octex::detail
